// Batched decode GEMV on MFMA (2 <= M <= 64 activation rows, f16 x).
//
//   int8:  y[m,n] = (sum_k W[n,k] x[m,k]) * s[n] (+ bias[n])
//          (crates/cellm-kernels/src/cpu_kernels.rs:66-133, one row per call)
//   q4:    y[m,n] = sum_k (q S + B)[n,k] x[m,k]   (crates/cellm-model/src/lfm.rs:985-1066)
//
// The reference decodes sessions one at a time (crates/cellm-sdk/src/lib.rs:622-680);
// batching M sessions reads every weight once for all of them.  At M <= 64
// the work is still HBM-bound (<= 128 flop per int8 weight byte), but a VALU
// dot product would need 2*M ops per weight, so the multiply runs on
// v_mfma_f32_16x16x32_f16 with A = X (M padded to 16-row tiles) and B = W.
//
// Each wave owns NT 16-row tiles of W.  W streams from HBM with 16-byte loads
// straight into B-operand registers -- no LDS for W, no sharing, each weight
// is read once.  A lane (row n = lane%16, slot group g = lane/16) holds one
// 16-byte chunk of its row per K block:
//   int8: 16 weights, k = kb + 16g .. +16, two MFMA k-steps (t = 0,1: 8 each);
//   q4:   32 weights (one group), k = kb + 32g .. +32, four k-steps.
// Both unpacks produce the weights of each 8-k word in natural order, so X is
// copied into LDS as it lies in memory.
//
// Dequant into the f16 B operand:
//   int8: u8 = w ^ 0x80 is exact in f16 as (1152 + w) - 1152 (v_perm_b32 +
//         v_pk_add_f16), so products are exact and the result differs from
//         the reference only by summation order; the row scale is applied
//         after the sum, as in the reference.
//   q4:   the converter's tile value RNE_f16(f32(q)*s + b)
//         (tools/convert/src/main.rs:4435-4436): q*s + b in f32 with the
//         group's scale and bias as stored (f32 scales: product and sum
//         rounded apart), then one rounding to f16.  The fp16-tile tolerance
//         of the MFMA paths applies; the tiles are exactly the ones the
//         prefill qGEMM and the oracle's f16 dequant produce.
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "launch_util.hpp"

namespace cellm {

namespace {

constexpr int kBlock = 256;
#ifndef CELLM_MFMA_XPAD
#define CELLM_MFMA_XPAD 8
#endif
constexpr int kXPad = CELLM_MFMA_XPAD;  // halves of padding after each staged X row
constexpr int kRowRor8 = 0x128;  // DPP control: rotate by 8 within each 16-lane row

// int8 word pair (8 weights) -> f16 x8 in natural order (exact): byte permutes place
// 0x64 above each biased byte, giving f16 1024 + (w + 128), and 1152 is subtracted.
__device__ __forceinline__ h8_t i8x8_to_f16(uint32_t w0, uint32_t w1)
{
    const uint32_t hi = 0x64646464u;
    const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t b0 = w0 ^ 0x80808080u, b1 = w1 ^ 0x80808080u;
    const h2_t a0 = as_h2(__builtin_amdgcn_perm(hi, b0, 0x04010400u)) - off;  // (w0, w1)
    const h2_t a1 = as_h2(__builtin_amdgcn_perm(hi, b0, 0x04030402u)) - off;  // (w2, w3)
    const h2_t a2 = as_h2(__builtin_amdgcn_perm(hi, b1, 0x04010400u)) - off;  // (w4, w5)
    const h2_t a3 = as_h2(__builtin_amdgcn_perm(hi, b1, 0x04030402u)) - off;  // (w6, w7)
    return h8_t{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
}

// Persistent streaming kernel.  WT: 0 = q4 affine, 1 = int8.  MS = 16-row
// tiles of X (ceil(M/16)); NT = 16-row tiles of W per wave; DEPTH = pairs of
// K blocks a wave loads per group; SBT = scale (and q4 bias) dtype; CHUNKED: X
// does not fit LDS whole and is staged per K chunk of KC columns (KC a
// multiple of a group's columns); BT = threads per block.  BT = 1024 is the
// one-block-per-CU form of the int8 kernel for an X of 80-152 KB (M = 49..64):
// the whole X stays in LDS (up to 160 KB per CU on gfx950) and 16 waves stream
// W, instead of restaging X chunks for every tile.  (The q4 form needs more
// than the 128 registers per lane a 1024-thread block leaves.)
//
// A block owns tiles of ROWS = 4*NT*16 weight rows: tile, tile+grid, ...  Each
// wave walks its rows in groups of DEPTH block pairs (128 B of every row per
// pair): it issues the whole group's loads (8 KB per wave), waits once, then
// runs the group's MFMAs.  Memory stays busy through the other waves of the
// CU (8-16 per CU), so no cross-iteration register ring is needed -- the
// compiler counts outstanding loads exactly only through straight-line code,
// and a ring that crosses tile boundaries would wait on every load anyway.
template <int WT, int MS, int NT, int DEPTH, int SBT, bool CHUNKED, bool SPLIT, int BT = kBlock, int WK = 1>
__global__ __launch_bounds__(BT) void qgemv_mfma_kernel(
    const void* __restrict__ W, const void* __restrict__ S, const void* __restrict__ Bz, int per_channel, int gshift,
    const _Float16* __restrict__ X, const float* __restrict__ bias, float* __restrict__ Y, int M, int N, int K, int KC,
    int ntiles, int pps, int nsplit, float* __restrict__ part)
{
    // X rows in LDS: with one X tile (M <= 16) just the M rows, the A operand of the others
    // selected to zero (a long K at small M then still fits whole); else MS*16 rows, the
    // padding zeroed
    extern __shared__ __align__(16) _Float16 xs[];  // [xrows][KC + kXPad]
    const int xrows = MS == 1 ? M : MS * 16;
    constexpr int KB = WT == 1 ? 64 : 128;  // K per block: 64 bytes of every row
    constexpr int TSTEPS = KB / 32;         // MFMA k-steps per block
    static_assert(!(CHUNKED && WK > 1), "waves splitting an item's K need the item's X whole");
    constexpr int WR = BT / 64 / WK;  // row groups; WK waves share each one's rows, splitting K
    constexpr int ROWS = WR * NT * 16;
    const int stride = KC + kXPad;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane & 15, g = lane >> 4;
    const int nkb = K / KB;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const size_t row_bytes = WT == 1 ? (size_t)K : (size_t)K / 2;
    const char* wb = reinterpret_cast<const char*>(W);
    const int wr = wave % WR, wk = wave / WR;
    const int row_in_tile = wr * NT * 16 + rl;

    // ---- X staging: columns [kb, kb + kcl) of the M rows, copied global -> LDS by
    // global_load_lds_dwordx4 (no registers; 16 bytes per lane, lane i at the wave's LDS base +
    // 16 i).  Chunk j of the padded layout is row j / (stride/8), word j % (stride/8); padding
    // words and rows M..MS*16-1 (zeroed once, below) are not written.  The caller waits vmcnt(0)
    // before the barrier that publishes the tile.
    auto stage = [&](int kb, int kcl) {
        const int words = kcl >> 3, rowc = stride >> 3, total = M * rowc;
        // this lane's first (row, chunk) by one division, then stepped BT chunks at a time (BT =
        // step_q rows + step_r chunks, step_r < rowc): no division per DMA
        const int step_q = BT / rowc, step_r = BT - step_q * rowc;
        int j = wave * 64 + lane, m = j / rowc, c = j - m * rowc;
        for (int j0 = wave * 64; j0 < total; j0 += BT) {
            if (j < total && c < words)
                __builtin_amdgcn_global_load_lds(X + (size_t)m * K + kb + c * 8, xs + (size_t)j0 * 8, 16, 0, 0);
            j += BT;
            m += step_q;
            c += step_r;
            if (c >= rowc) {
                c -= rowc;
                ++m;
            }
        }
    };
    // One block's B operands + MFMAs: w[t] is this lane's 16 bytes of row
    // (lane%16) of W tile t at the block's k slot 16*(lane/16) bytes; kx is the
    // block's first column in the staged X.
    f4_t acc[MS][NT];
    auto mma_block = [&](const u4_t(&w)[NT], const uint32_t(&s)[NT], const uint32_t(&b)[NT], int kx) {
        h8_t bf[NT][TSTEPS];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if constexpr (WT == 1) {
                bf[t][0] = i8x8_to_f16(w[t][0], w[t][1]);
                bf[t][1] = i8x8_to_f16(w[t][2], w[t][3]);
            } else {
                const float sc = raw_to_f32<SBT>(s[t]), bi = raw_to_f32<SBT>(b[t]);
#pragma unroll
                for (int q = 0; q < 4; ++q) bf[t][q] = dequant_word_bytes<SBT>(w[t][q], sc, bi);
            }
        }
#pragma unroll
        for (int st = 0; st < TSTEPS; ++st) {
            const int kof = kx + g * (KB / 4) + st * 8;
#pragma unroll
            for (int i = 0; i < MS; ++i) {
                h8_t a;
                if constexpr (MS == 1) {
                    const h8_t v = *reinterpret_cast<const h8_t*>(xs + (size_t)min(rl, M - 1) * stride + kof);
                    a = rl < M ? v : h8_t{};
                } else {
                    a = *reinterpret_cast<const h8_t*>(xs + (size_t)(i * 16 + rl) * stride + kof);
                }
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bf[t][st], acc[i][t], 0, 0, 0);
            }
        }
    };
    // stage the X chunk that starts at column kcol, if one does (chunks start at
    // the work item's first column k0 and end at its last, k1); returns the
    // column's offset in the staged X
    int k0 = 0, k1 = K;
    auto chunk_at = [&](int kcol) {
        if constexpr (CHUNKED) {
            const int rel = kcol - k0, c = rel / KC, off = rel - c * KC;
            if (off == 0) {
                __syncthreads();  // every wave is done with the previous chunk
                stage(k0 + c * KC, min(KC, k1 - (k0 + c * KC)));
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            }
            return off;
        } else {
            return kcol;
        }
    };

    // Weights load as full 128-byte row segments (two K blocks): load h of a
    // pair covers rows 8h..8h+7 of a 16-row tile, lane (rl, g) taking row
    // (rl & 7) + 8h at byte 16g + 64*((rl >> 3) ^ h).  Then, per lane,
    //   block 0 = rl < 8 ? load0 : load1                (row rl, byte 16g)
    //   block 1 = row_ror:8 of (rl < 8 ? load1 : load0) (row rl, byte 64 + 16g)
    // which is the MFMA B layout.  A 16-row x 64-byte load per block (the
    // layout itself) splits every cache line over two instructions and streams
    // about a quarter slower.
    const bool low8 = (rl & 8) == 0;
    const int npairs = nkb >> 1;
    const int nitems = ntiles * nsplit;
    // Work item = (tile, split): split s covers block pairs [s*pps, min(npairs, (s+1)*pps)), the
    // last split also the odd last K block.  Consecutive items share a split (and its X columns).
    int split = 0, tile = 0, pb = 0, pe = 0, wpb = 0, wpe = 0;  // item pairs; this wave's share
    bool last_split = true;
    const char* wpair[NT][2];
    const char* wtail[NT];
    size_t sbrow[NT];  // the tile row this lane loads (rows past N: N - 1)
    auto setup = [&](int item) {
        split = item / ntiles;
        tile = item - split * ntiles;
        pb = split * pps;
        pe = min(npairs, pb + pps);
        last_split = split == nsplit - 1;
        const int q = (pe - pb + WK - 1) / WK;
        wpb = min(pe, pb + wk * q);
        wpe = min(pe, wpb + q);
        k0 = pb * 2 * KB;
        k1 = last_split ? K : pe * 2 * KB;
        // rows past N read row N-1 and are never stored
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int base = tile * ROWS + wr * NT * 16 + t * 16;
            const int r = min(base + rl, N - 1);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                wpair[t][h] = wb + (size_t)min(base + (rl & 7) + 8 * h, N - 1) * row_bytes + 16 * g +
                              64 * ((rl >> 3) ^ h);
            wtail[t] = wb + (size_t)r * row_bytes + 16 * g;
            sbrow[t] = (size_t)r;
        }
    };
    // int8 row scale and bias of the current item, loaded unconditionally (without a bias the
    // load reads X and the value is replaced by 0) so that no branch changes the count of
    // memory operations in flight
    uint32_t sc_raw[NT];
    float bv[NT];
    auto load_scale = [&]() {
        if constexpr (WT == 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const size_t r = sbrow[t];
                sc_raw[t] = load_raw<SBT>(S, per_channel ? r : 0);
                const float b = *(bias ? bias + r : reinterpret_cast<const float*>(X));
                bv[t] = bias ? b : 0.0f;
            }
        }
    };
    // one group's weights (and q4 group scale/bias) in one burst; pairs past the item's end load
    // its last pair again (never used), so every group issues the same loads and the compiler's
    // wait counts stay exact
    u4_t ld[DEPTH][NT][2];
    uint32_t sr[DEPTH][2][NT], br[DEPTH][2][NT];
    auto issue = [&](int p0) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int p = max(pb, min(p0 + d, wpe - 1));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    ld[d][t][h] =
                        __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(wpair[t][h] + (size_t)p * 128));
                if constexpr (WT == 0) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const size_t gi = sbrow[t] * gpr + (((p * 2 + h) * KB + 32 * g) >> gshift);
                        sr[d][h][t] = load_raw<SBT>(S, gi);
                        br[d][h][t] = load_raw<SBT>(Bz, gi);
                    }
                }
            }
        }
    };
    // the group's MFMAs
    auto consume = [&](int p0) {
        const int kx0 = chunk_at(p0 * 2 * KB);
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (p0 + d < wpe) {
                u4_t w0[NT], w1[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const u4_t a = ld[d][t][0], b = ld[d][t][1];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        w0[t][j] = low8 ? a[j] : b[j];
                        w1[t][j] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(low8 ? b[j] : a[j]), kRowRor8, 0xF,
                                                                         0xF, false);
                    }
                }
                mma_block(w0, sr[d][0], br[d][0], kx0 + d * 2 * KB);
                mma_block(w1, sr[d][1], br[d][1], kx0 + d * 2 * KB + KB);
            }
        }
    };

    // The next item's first group is issued before this item's C tile is stored: gfx9 counts
    // loads and stores on one in-order counter, so stores issued first would hold that group's
    // wait until they had reached memory (the 1152 -> 262144 int8 lm_head at M = 64 ran 93 us
    // with its stores, ~71 us without them).  Every path issues the same memory operations
    // (items have at least one block pair; stores are buffer stores that drop out-of-range
    // lanes; loads are unconditional), so the compiler's waits count exactly.
    const uint32_t ybytes = (uint32_t)M * (uint32_t)N * 4u;
    const auto yr = buffer_rsrc(Y, ybytes);
    // C tile of the finished item: lane holds activation rows 4*(lane/16)+e, weight row lane%16.
    // Columns past N get an offset past 2^31, rows past M one past M*N*4: both are dropped.
    auto store_tile = [&](int n0, int cur_split, const float(&scl)[NT], const float(&bvc)[NT]) {
        uint32_t col[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) col[t] = wk == 0 && n0 + t * 16 < N ? (uint32_t)(n0 + t * 16) : 0x20000000u;
        auto put = [&](auto nt, __amdgpu_buffer_rsrc_t r, bool raw) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < MS; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t m = i * 16 + g * 4 + e;
                        const float v = raw ? acc[i][t][e] : acc[i][t][e] * scl[t] + bvc[t];
                        buffer_store_f32<decltype(nt)::value>(v, r, (m * (uint32_t)N + col[t]) * 4u);
                    }
        };
        if constexpr (SPLIT)
            // split-K: raw sums to part[split][m][n]; the reduction kernel applies the scale and bias
            put(std::false_type{}, buffer_rsrc(part + (size_t)cur_split * M * N, ybytes), true);
        else
            // plain (cached) stores: with the stores behind the next tile's loads, non-temporal
            // stores of the M = 64 logits measured 2 % slower (78.7-79.0 against 77.0-77.2 us)
            put(std::false_type{}, yr, false);
    };

    // the odd last K block (16 rows x 64 bytes, already in the B layout), loaded with the item's
    // first group
    u4_t tw[NT];
    uint32_t ts[NT], tb[NT];
    auto issue_tail = [&]() {
        if ((nkb & 1) && last_split && wk == WK - 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                tw[t] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(wtail[t] + (size_t)(nkb - 1) * 64));
                if constexpr (WT == 0) {
                    const size_t gi = sbrow[t] * gpr + (((nkb - 1) * KB + 32 * g) >> gshift);
                    ts[t] = load_raw<SBT>(S, gi);
                    tb[t] = load_raw<SBT>(Bz, gi);
                }
            }
        }
    };

    // K split over the WK waves of a row group: waves 1..WK-1 hand their sums to wave 0 through
    // LDS after the X tile; wave 0 adds them in wave order.
    f4_t* red = reinterpret_cast<f4_t*>(xs + (size_t)xrows * stride);
    auto reduce_waves = [&]() {
        if constexpr (WK > 1) {
            if (wk > 0) {
#pragma unroll
                for (int i = 0; i < MS; ++i)
#pragma unroll
                    for (int t = 0; t < NT; ++t) red[(((wk - 1) * WR + wr) * MS * NT + i * NT + t) * 64 + lane] = acc[i][t];
            }
            __syncthreads();
            if (wk == 0) {
                for (int j = 1; j < WK; ++j)
#pragma unroll
                    for (int i = 0; i < MS; ++i)
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc[i][t] += red[(((j - 1) * WR + wr) * MS * NT + i * NT + t) * 64 + lane];
            }
            __syncthreads();  // the slots are free for the next item
        }
    };

    int item = blockIdx.x;
    if (item >= nitems) return;
    setup(item);
    issue(wpb);
    issue_tail();
    // as many dropped stores as a C tile, so the first item's group has the same operations
    // behind it as every later one
    auto dummy_stores = [&]() {
#pragma unroll
        for (int u = 0; u < MS * NT * 4; ++u)
            buffer_store_f32<false>(0.0f, yr, kBufferDrop + 256u * u);  // distinct offsets: not merged
    };
    dummy_stores();
    // the padding rows of the last X tile (MS > 1): zero for every chunk
    for (int i = threadIdx.x; i < (xrows - M) * (stride >> 3); i += BT)
        reinterpret_cast<u4_t*>(xs + (size_t)M * stride)[i] = u4_t{0u, 0u, 0u, 0u};
    if constexpr (!CHUNKED) {
        // X staged while the first weights are in flight
        stage(0, K);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    int n0 = 0, cur_split = 0;
    float scl[NT], bvc[NT];
    for (;;) {
        load_scale();
#pragma unroll
        for (int i = 0; i < MS; ++i)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[i][t] = f4_t{0.f, 0.f, 0.f, 0.f};
        consume(wpb);
        for (int p0 = wpb + DEPTH; p0 < wpe; p0 += DEPTH) {
            issue(p0);
            consume(p0);
        }
        if ((nkb & 1) && last_split && wk == WK - 1) mma_block(tw, ts, tb, chunk_at((nkb - 1) * KB));
        reduce_waves();

        n0 = tile * ROWS + row_in_tile;
        cur_split = split;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            scl[t] = WT == 1 ? raw_to_f32<SBT>(sc_raw[t]) : 1.0f;
            bvc[t] = WT == 1 ? bv[t] : 0.0f;
        }
        item += gridDim.x;
        if (item >= nitems) break;
        setup(item);
        issue(wpb);
        issue_tail();
        store_tile(n0, cur_split, scl, bvc);
    }
    store_tile(n0, cur_split, scl, bvc);
}

// Blocks of one instantiation that fit a CU at this LDS size, times the CU
// count (cached per device and LDS size): the persistent grid.
template <typename Kern>
int resident_blocks(Kern kern, size_t lds)
{
    struct Entry {
        const void* kern;
        int dev;
        size_t lds;
        int blocks;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    const void* key = reinterpret_cast<const void*>(kern);
    std::lock_guard<std::mutex> lk(mu);
    for (const Entry& e : cache)
        if (e.kern == key && e.dev == dev && e.lds == lds) return e.blocks;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kBlock, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
    cache.push_back({key, dev, lds, per_cu * cus});
    return per_cu * cus;
}

constexpr size_t kWholeXLds = 152 * 1024;  // the BT = 1024 form holds X up to this size

// Split-K reduction: y[m,n] = (sum over splits, in split order, of part[s][m][n]) * scale + bias
// (int8; the scale after the sum, as cpu_kernels.rs:130 applies it), or the plain sum (q4).
template <int WT, int SBT>
__global__ __launch_bounds__(64) void mfma_splitk_reduce_kernel(const float* __restrict__ part, int nsplit,
                                                                 const void* __restrict__ S, int per_channel,
                                                                 const float* __restrict__ bias,
                                                                 float* __restrict__ Y, int M, int N)
{
    const size_t total = (size_t)M * N, plane = total;
    if ((N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
        const size_t n4 = total >> 2;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
            f4_t a = sum_splits_f4(reinterpret_cast<const f4_t*>(part) + i, plane >> 2, nsplit);
            if constexpr (WT == 1) {
                const int n = (int)((4 * i) % (size_t)N);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float s = raw_to_f32<SBT>(load_raw<SBT>(S, per_channel ? (size_t)(n + e) : 0));
                    a[e] = a[e] * s + (bias ? bias[n + e] : 0.0f);
                }
            }
            reinterpret_cast<f4_t*>(Y)[i] = a;
        }
        return;
    }
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        float a = part[i];
        for (int sp = 1; sp < nsplit; ++sp) a += part[sp * plane + i];
        if constexpr (WT == 1) {
            const int n = (int)(i % (size_t)N);
            const float s = raw_to_f32<SBT>(load_raw<SBT>(S, per_channel ? (size_t)n : 0));
            a = a * s + (bias ? bias[n] : 0.0f);
        }
        Y[i] = a;
    }
}

int device_cus()
{
    static std::mutex mu;
    static std::vector<std::pair<int, int>> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& e : cache)
        if (e.first == dev) return e.second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    cache.push_back({dev, cus});
    return cus;
}

// Split-K plan of the batched kernel.  Few 64-row W tiles (small N) over a long K leave most CUs
// idle while each wave walks the whole K; then K is cut into splits of pps block pairs, each
// (tile, split) is a work item, and a second kernel adds the splits' partial sums.
struct SplitPlan {
    int nsplit = 1, pps = 0;
};

SplitPlan split_plan(int wt, int M, int N, int K)
{
    SplitPlan p;
    const int KB = wt == 1 ? 64 : 128, npairs = (K / KB) >> 1;
    p.pps = npairs;
    constexpr int ROWS = (kBlock / 64) * 16;  // one 16-row tile per wave
    const int ntiles = (N + ROWS - 1) / ROWS, cus = device_cus();
    // the unsplit kernel's per-wave walk: pairs x 16-row X tiles, a q4 pair (256 k with its dequant)
    // counted twice; below ~20 the walk is short next to a second launch (measured on MI355X: int8
    // 1024->1152 at M=16 7.6 us unsplit, 9.2 us split; int8 2560->960 at M=8 14.6 / 9.8 us)
    const int walk = npairs * ((M + 15) / 16) * (wt == 1 ? 1 : 2);
    if (M < 2 || npairs < 2 || ntiles * 2 > cus || walk < 20) return p;
    // about one item per CU, each at least two block pairs: one-pair items measured 1-2 us slower
    // (q4 4864->896 and 6912->1152, int8 1152->1536, M = 8..64), four-pair items 2 us slower at
    // 6912->1152, M=64
    const int want = (cus + ntiles - 1) / ntiles;
    p.pps = std::max(2, (npairs + want - 1) / want);
    p.nsplit = (npairs + p.pps - 1) / p.pps;
    if (p.nsplit < 2) p = SplitPlan{1, npairs};
    return p;
}


template <int WT, int MS, int NT, int SBT>
hipError_t launch_mfma_nt(const void* W, const void* S, const void* B, int per_channel, int gshift, const _Float16* X,
                          const float* bias, float* Y, int M, int N, int K, const SplitPlan& sp, float* ws,
                          hipStream_t st)
{
    constexpr int KB = WT == 1 ? 64 : 128;
    if constexpr (MS == 4 && NT == 1) {
        // X too big for two blocks per CU but within one CU's LDS: one block per CU keeps it whole.
        // int8: 1024 threads, 16 waves of one W tile each (two tiles per wave need more than the 128
        // registers per lane a 1024-thread block leaves, and 8 waves of two tiles stream 12 % slower:
        // measured).  q4 (its dequant needs more registers): 512 threads.
        const size_t whole = (size_t)MS * 16 * (K + kXPad) * 2;  // MS == 4: padded rows
        if (sp.nsplit == 1 && whole > 80 * 1024 && whole <= kWholeXLds) {
#ifndef CELLM_WX_NT
#define CELLM_WX_NT 1
#define CELLM_WX_DEPTH 2
#define CELLM_WX_BT 1024
#endif
            constexpr int XNT = WT == 1 ? CELLM_WX_NT : 1;
            constexpr int BT = WT == 1 ? CELLM_WX_BT : 512, DEPTH = WT == 1 ? CELLM_WX_DEPTH : 2, ROWS = (BT / 64) * XNT * 16;
            auto kern = qgemv_mfma_kernel<WT, MS, XNT, DEPTH, SBT, false, false, BT>;
            if (hipError_t e = allow_big_lds(kern, (int)kWholeXLds); e != hipSuccess) return e;
            const int ntiles = (N + ROWS - 1) / ROWS;
            int per_cu = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, BT, whole) != hipSuccess || per_cu < 1)
                per_cu = 1;
            const int grid = std::min(ntiles, per_cu * device_cus());
            hipLaunchKernelGGL(kern, dim3(grid), dim3(BT), whole, st, W, S, B, per_channel, gshift, X, bias, Y, M, N, K,
                               K, ntiles, (K / KB) >> 1, 1, (float*)nullptr);
            return hipGetLastError();
        }
    }
    constexpr int DEPTH = 4 / NT;  // block pairs per group: 8 KB of weights per wave
    constexpr int ROWS = (kBlock / 64) * NT * 16;
    // X in LDS: at most 80 KB per block so two blocks share a CU; the whole K
    // when it fits, else chunks of KC columns (a multiple of the K block)
    const int xrows = MS == 1 ? M : MS * 16;  // the kernel's X rows in LDS
    int KC = std::max(1, (80 * 1024 / (xrows * 2) - kXPad) / (2 * DEPTH * KB)) * (2 * DEPTH * KB);
    if (KC >= K) KC = K;
    const int ntiles = (N + ROWS - 1) / ROWS;
    float* part = nullptr;
    if (sp.nsplit > 1) {
        // one split's columns (plus an odd last block) in one chunk when they fit
        const int span = sp.pps * 2 * KB + ((K / KB) & 1 ? KB : 0);
        if ((size_t)xrows * (span + kXPad) * 2 <= 80 * 1024 || span < KC) KC = span;
        part = ws;
    }
    const size_t lds = (size_t)xrows * (KC + kXPad) * 2;
    auto launch = [&](auto kern, int rows, size_t lds_bytes) {
        const int nt = (N + rows - 1) / rows, items = nt * sp.nsplit;
        const int grid = std::min(items, resident_blocks(kern, lds_bytes));
        hipLaunchKernelGGL(kern, dim3(grid), dim3(kBlock), lds_bytes, st, W, S, B, per_channel, gshift, X, bias, Y, M,
                           N, K, KC, nt, sp.pps, sp.nsplit, part);
    };
    if (part) {
        // split plans run one tile per wave (launch_mfma_ms)
        if constexpr (NT == 1) {
            if (KC < K) launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, true, true>, ROWS, lds);
            else launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, false, true>, ROWS, lds);
        }
    } else if (KC < K) {
        launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, true, false>, ROWS, lds);
    } else {
        // Few tiles over a K that takes a wave several load groups, or fewer 64-row tiles than CUs:
        // the block's waves share one tile row group and split its K (WK = 4 or 2), adding their sums
        // through LDS.  A wave's load group is no deeper than its share of the block pairs: a group
        // deeper than the share re-reads its last pair for every missing one (measured on MI355X at
        // M = 8..32: q4 1024->4096 7.8 -> 4.9 us, 896->4864 6.7 -> 5.5 us, int8 1024->1152 5.0 -> 4.6
        // us; the same split with 4-pair groups was slower than no split).
        const int npairs = (K / KB) >> 1, groups = (npairs + DEPTH - 1) / DEPTH;
        int wk = 1;
        if constexpr (NT == 1) {
            const int cus = device_cus();
            for (int cand : {4, 2})
                if ((groups > 1 || ntiles < cus) && npairs >= cand &&
                    (N + (4 / cand) * 16 - 1) / ((4 / cand) * 16) <= 2 * cus) {
                    wk = cand;
                    break;
                }
        }
        const size_t red = (size_t)(wk - 1) * (4 / wk) * MS * NT * 64 * 16;
        if constexpr (NT == 1) {
            const int share = (npairs + wk - 1) / wk;  // block pairs per wave
            if (wk == 4) {
                if (share <= 1) launch(qgemv_mfma_kernel<WT, MS, NT, 1, SBT, false, false, kBlock, 4>, 16, lds + red);
                else if (share <= 2) launch(qgemv_mfma_kernel<WT, MS, NT, 2, SBT, false, false, kBlock, 4>, 16, lds + red);
                else launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, false, false, kBlock, 4>, 16, lds + red);
            } else if (wk == 2) {
                if (share <= 2) launch(qgemv_mfma_kernel<WT, MS, NT, 2, SBT, false, false, kBlock, 2>, 32, lds + red);
                else launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, false, false, kBlock, 2>, 32, lds + red);
            }
        }
        if (wk == 1) launch(qgemv_mfma_kernel<WT, MS, NT, DEPTH, SBT, false, false>, ROWS, lds);
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess || sp.nsplit == 1) return e;
    // A second launch adds the splits.  Adding them inside the GEMV instead (device-coherent
    // partial stores, an arrival counter per tile and the last block summing in split order)
    // measured slower on MI355X: int8 1152->1536 at M = 64 15.8 vs 9.6 us per call, q4
    // 6912->1152 at M = 16 14.6 vs 11.1 us and at M = 64 35.5 vs 13.4 us.
    // One-wave blocks: a few thousand threads at most, spread over as many CUs as there are waves.
    const size_t work = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0 ? (size_t)M * N / 4 : (size_t)M * N;
    const unsigned blocks = (unsigned)std::min<size_t>((work + 63) / 64, 8192);
    hipLaunchKernelGGL((mfma_splitk_reduce_kernel<WT, SBT>), dim3(blocks), dim3(64), 0, st, ws, sp.nsplit, S,
                       per_channel, bias, Y, M, N);
    return hipGetLastError();
}

template <int WT, int MS, int SBT>
hipError_t launch_mfma_ms(const void* W, const void* S, const void* B, int per_channel, int gshift, const _Float16* X,
                          const float* bias, float* Y, int M, int N, int K, const SplitPlan& sp, float* ws,
                          hipStream_t st)
{
    // two 16-row W tiles per wave when there are rows enough to fill the chip, unless X needs the
    // one-block-per-CU form (one tile per wave there)
    const size_t whole = (size_t)MS * 16 * (K + kXPad) * 2;
    const bool whole_x = MS == 4 && whole > 80 * 1024 && whole <= kWholeXLds;
    if (sp.nsplit == 1 && N >= 128 * 512 && !whole_x)
        return launch_mfma_nt<WT, MS, 2, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
    return launch_mfma_nt<WT, MS, 1, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
}

template <int WT, int SBT>
hipError_t launch_mfma(const void* W, const void* S, const void* B, int per_channel, int gshift, const _Float16* X,
                       const float* bias, float* Y, int M, int N, int K, float* ws, size_t ws_bytes, hipStream_t st)
{
    SplitPlan sp = split_plan(WT, M, N, K);
    if (sp.nsplit > 1 && (!ws || ws_bytes < (size_t)sp.nsplit * M * N * sizeof(float)))
        sp = SplitPlan{1, (K / (WT == 1 ? 64 : 128)) >> 1};
    switch ((M + 15) / 16) {
    case 1: return launch_mfma_ms<WT, 1, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
    case 2: return launch_mfma_ms<WT, 2, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
    case 3: return launch_mfma_ms<WT, 3, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
    default: return launch_mfma_ms<WT, 4, SBT>(W, S, B, per_channel, gshift, X, bias, Y, M, N, K, sp, ws, st);
    }
}

}  // namespace

bool qgemv_mfma_supported(int wt, int M, int N, int K, int group_size)
{
    if (M < 2 || M > 64 || N <= 0) return false;
    // every 16-row X tile's output offsets fit the 2^31-byte buffer range of the stores
    if ((size_t)((M + 15) & ~15) * (size_t)N * 4 > 0x7FFFFFFFu) return false;
    // at least one 128-byte block pair per row (the kernel issues a work item's first pair
    // unconditionally)
    if (wt == 1) return K % 64 == 0 && K >= 128;
    return K % 128 == 0 && K >= 256 && group_size >= 32;
}

size_t qgemv_mfma_workspace_bytes(int wt, int M, int N, int K)
{
    if (M < 2 || M > 64 || K <= 0 || N <= 0) return 0;
    const SplitPlan sp = split_plan(wt, M, N, K);
    return sp.nsplit > 1 ? (size_t)sp.nsplit * M * N * sizeof(float) : 0;
}

hipError_t launch_qgemv_mfma_i8(const int8_t* w, const void* S, int sdt, int per_channel, const _Float16* x,
                                const float* bias, float* y, int M, int N, int K, float* ws, size_t ws_bytes,
                                hipStream_t st)
{
    if (sdt == DT_F16) return launch_mfma<1, DT_F16>(w, S, nullptr, per_channel, 0, x, bias, y, M, N, K, ws, ws_bytes, st);
    if (sdt == DT_F32) return launch_mfma<1, DT_F32>(w, S, nullptr, per_channel, 0, x, bias, y, M, N, K, ws, ws_bytes, st);
    return launch_mfma<1, DT_BF16>(w, S, nullptr, per_channel, 0, x, bias, y, M, N, K, ws, ws_bytes, st);
}

hipError_t launch_qgemv_mfma_q4(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                const _Float16* x, float* y, int M, int N, int K, float* ws, size_t ws_bytes,
                                hipStream_t st)
{
    const int gshift = __builtin_ctz((unsigned)group_size);
    if (sbt == DT_F16) return launch_mfma<0, DT_F16>(wq, S, B, 1, gshift, x, nullptr, y, M, N, K, ws, ws_bytes, st);
    if (sbt == DT_F32) return launch_mfma<0, DT_F32>(wq, S, B, 1, gshift, x, nullptr, y, M, N, K, ws, ws_bytes, st);
    return launch_mfma<0, DT_BF16>(wq, S, B, 1, gshift, x, nullptr, y, M, N, K, ws, ws_bytes, st);
}

}  // namespace cellm
