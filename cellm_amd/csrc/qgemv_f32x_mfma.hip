// q4 affine GEMV with f32 activations on MFMA, exact in the nibbles (M <= 4 rows, long N).
//
// The reference dequantizes each weight to f32 and multiplies the f32 x
// (crates/cellm-model/src/lfm.rs:985-1066; the affine lm_head lfm.rs:700-741):
//   y[m,n] = sum_k (q[n,k] s[n,g(k)] + b[n,g(k)]) x[m,k].
// Per group of 64 k the scale and bias factor out of the dot product:
//   y[m,n] = sum_g ( s[n,g] * sum_{k in g} q[n,k] x[m,k]  +  b[n,g] * sum_{k in g} x[m,k] ).
// Here the inner sums run on v_mfma_f32_16x16x32_f16 with the nibbles as exact f16
// integers (B) and x as two f16 parts, hi = RNE_f16(x') and lo = RNE_f16(x' - hi), in
// A rows m and M + m, where x' = x * 2^sh with one power of two per (row, group) chosen
// from the group's largest |x| (so every finite x stays inside f16's normal range).
// q * part is exact in f32, so the group sum carries x to about 22 bits, as the f32-x
// VALU kernels do; the fold  y += s * (2^-sh * acc) + b * sum(x)  runs once per group.
//
// MFMA k-slots and groups: a lane (row n = lane%16, slot group g = lane/16) loads 16
// bytes of its row per 128-k block, k = 32g .. 32g+31, i.e. words w0..w3 of 8 nibbles.
// One 16x16x32 k-step contracts the four lanes' words, which would mix the block's two
// groups; v_permlane32_swap of (w0, w1) and of (w2, w3) moves the words between lane
// halves so that each k-step holds one group:
//   R0 = swap(w0,w1).first : g = 0,1,2,3 -> k 0, 32, 8, 40 (+0..7)     group 0 of the block
//   R1 = swap(w0,w1).second: g = 0,1,2,3 -> k 64, 96, 72, 104           group 1
//   R2 = swap(w2,w3).first : k 16, 48, 24, 56                           group 0
//   R3 = swap(w2,w3).second: k 80, 112, 88, 120                         group 1
// The A fragment of lane (row, g) for a k-step reads those 8 k of its X row from LDS.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "launch_util.hpp"

namespace cellm {

namespace {

constexpr int kFxThreads = 256;  // four waves
constexpr int kFxMaxK = 1024;
constexpr int kFxMaxGroups = kFxMaxK / 64;
constexpr int kFxAPad = 8;        // halves after each staged X row
constexpr int kFxWaveLds = 2048;  // per wave: the tile's (scale, bias) table, then its output tile

// 8 nibbles of a word as exact f16 integers, in the order q0 q2 q4 q6 q1 q3 q5 q7
// (0x64 placed above each nibble byte gives f16 1024 + q; 1024 is then subtracted).
__device__ __forceinline__ h8_t q4_word_exact(uint32_t w)
{
    const uint32_t hi64 = 0x64646464u;
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const h2_t off = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2_t a0 = as_h2(__builtin_amdgcn_perm(hi64, lo, 0x04010400u)) - off;  // q0 q2
    const h2_t a1 = as_h2(__builtin_amdgcn_perm(hi64, lo, 0x04030402u)) - off;  // q4 q6
    const h2_t a2 = as_h2(__builtin_amdgcn_perm(hi64, hi, 0x04010400u)) - off;  // q1 q3
    const h2_t a3 = as_h2(__builtin_amdgcn_perm(hi64, hi, 0x04030402u)) - off;  // q5 q7
    return h8_t{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
}

// A tile's loads: its 16 W rows over the whole K as full 128-byte row segments (two
// 128-k blocks; load h covers rows 8h..8h+7, lane (rl, g) taking row (rl & 7) + 8h at byte
// 16g + 64((rl >> 3) ^ h), as the batched MFMA kernel loads them), the odd last block, and
// the (scale, bias) of groups 4g..4g+3 of row rl.
template <int NB>
struct FxTile {
    u4_t w[NB / 2 > 0 ? NB / 2 : 1][2];
    u4_t tail;
    uint32_t s[4], b[4];
};

// Four waves per block; wave w of block b takes tiles b*4 + w, += gridDim.x*4, a tile being
// 16 rows of W over the whole K (NB blocks of 128).  Each wave keeps its next tile's loads in
// flight while it computes the current one: two register sets, the loop unrolled by two so
// neither is copied, and a tile past the end loaded through a buffer offset out of range
// (zeros, no memory traffic), so every iteration issues the same loads.
template <int SBT, int NB>
__global__ __launch_bounds__(kFxThreads) void qgemv_q4_f32x_mfma_kernel(const uint32_t* __restrict__ W,
                                                                        const void* __restrict__ S,
                                                                        const void* __restrict__ Bz,
                                                                        const float* __restrict__ X,
                                                                        float* __restrict__ Y, int M, int N)
{
    constexpr int K = NB * 128, G = K / 64, NP = NB / 2, astride = K + kFxAPad;
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* A = reinterpret_cast<_Float16*>(smem);                              // [16][astride]
    float* P2 = reinterpret_cast<float*>(smem + (size_t)16 * astride * 2);        // [kFxMaxGroups][16]: 2^-sh
    float* SX = P2 + kFxMaxGroups * 16;                                           // [kFxMaxGroups][16]: sum x
    unsigned char* wave_lds = reinterpret_cast<unsigned char*>(SX + kFxMaxGroups * 16);
    // the wave index as a uniform (scalar) value, so the tile loop is a scalar loop
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane & 15, g = lane >> 4;
    const int ntiles = N >> 4, stride = gridDim.x * 4;
    constexpr uint32_t row_bytes = K / 2;
    const auto wr = buffer_rsrc(const_cast<uint32_t*>(W), (uint32_t)ntiles * 16u * row_bytes);
    const bool low8 = (rl & 8) == 0;
    const int offg = (g & 1) * 32 + (g >> 1) * 8;  // this lane's k within a group-pure k-step

    auto load_tile = [&](FxTile<NB>& t, int tile) {
        const bool live = tile < ntiles;
        const int n0 = min(tile, ntiles - 1) * 16;
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t off = (uint32_t)(n0 + (rl & 7) + 8 * h) * row_bytes + 128 * p + 16 * g + 64 * ((rl >> 3) ^ h);
                t.w[p][h] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, live ? off : kBufferDrop, 0, 2));
            }
        if constexpr (NB & 1) {
            const uint32_t off = (uint32_t)(n0 + rl) * row_bytes + 64 * (NB - 1) + 16 * g;
            t.tail = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, live ? off : kBufferDrop, 0, 2));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const size_t gi = (size_t)(n0 + rl) * G + min(4 * g + j, G - 1);
            t.s[j] = load_raw<SBT>(S, gi);
            t.b[j] = load_raw<SBT>(Bz, gi);
        }
    };

    int tile = blockIdx.x * 4 + wave;
    FxTile<NB> ta, tb;
    load_tile(ta, tile);  // in flight while X is staged

    // ---- X: rows 0..M-1 hi parts, M..2M-1 lo parts, 2M..15 zero; per (row, group) 2^-sh
    // and the group's sum of x (zero for lo and padding rows).
    for (int i = threadIdx.x; i < (16 - 2 * M) * (astride >> 3); i += kFxThreads)
        reinterpret_cast<u4_t*>(A + (size_t)2 * M * astride)[i] = u4_t{0u, 0u, 0u, 0u};
    for (int i = threadIdx.x; i < kFxMaxGroups * 16; i += kFxThreads) {
        if ((i & 15) >= 2 * M) {
            P2[i] = 0.0f;
            SX[i] = 0.0f;
        }
    }
    {
        constexpr int words = K / 8;
        const int total = M * words;  // a multiple of 8: K % 64 == 0
        for (int base = 0; base < total; base += kFxThreads) {
            const int i = base + threadIdx.x, ic = min(i, total - 1);
            const int m = ic / words, c = ic - m * words;
            const f4_t* src = reinterpret_cast<const f4_t*>(X + (size_t)m * K + 8 * c);
            const f4_t v0 = src[0], v1 = src[1];
            float xv[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            float mx = 0.0f, xs = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                mx = fmaxf(mx, fabsf(xv[j]));
                xs += xv[j];
            }
            // eight consecutive lanes hold one group of 64 (aligned: words per row % 8 == 0)
            mx = group_max<8>(mx);
            xs = group_sum<8>(xs);
            int e = 0;
            (void)__builtin_frexpf(mx, &e);
            const int sh = (mx > 0.0f && mx <= 3.402823466e38f) ? min(14 - e, 126) : 0;
            h8_t hi, lo;
            constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};  // q4_word_exact's order
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float xp = __builtin_ldexpf(xv[order[j]], sh);
                hi[j] = (_Float16)xp;
                lo[j] = (_Float16)(xp - (float)hi[j]);
            }
            if (i < total) {
                *reinterpret_cast<h8_t*>(A + (size_t)m * astride + 8 * c) = hi;
                *reinterpret_cast<h8_t*>(A + (size_t)(M + m) * astride + 8 * c) = lo;
                if ((c & 7) == 0) {
                    const int grp = c >> 3;
                    const float p2 = __builtin_ldexpf(1.0f, -sh);
                    P2[grp * 16 + m] = p2;
                    P2[grp * 16 + M + m] = p2;
                    SX[grp * 16 + m] = xs;
                    SX[grp * 16 + M + m] = 0.0f;
                }
            }
        }
    }
    __syncthreads();
    if (tile >= ntiles) return;

    float2* sbw = reinterpret_cast<float2*>(wave_lds + wave * kFxWaveLds);  // [16 rows][16 groups]
    float* otw = reinterpret_cast<float*>(wave_lds + wave * kFxWaveLds);    // [16][16], after the folds

    auto compute = [&](const FxTile<NB>& t, int n0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sbw[rl * 16 + 4 * g + j] = make_float2(raw_to_f32<SBT>(t.s[j]), raw_to_f32<SBT>(t.b[j]));
        f4_t y = {0.f, 0.f, 0.f, 0.f};
        auto fold = [&](const f4_t& acc, int grp) {
            const f4_t pv = *reinterpret_cast<const f4_t*>(P2 + grp * 16 + 4 * g);
            const f4_t sx = *reinterpret_cast<const f4_t*>(SX + grp * 16 + 4 * g);
            const float2 sb = sbw[rl * 16 + grp];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = fmaf(acc[e] * pv[e], sb.x, fmaf(sb.y, sx[e], y[e]));
        };
        auto do_block = [&](const u4_t& w, int b) {
            const auto s01 = __builtin_amdgcn_permlane32_swap(w[0], w[1], false, false);
            const auto s23 = __builtin_amdgcn_permlane32_swap(w[2], w[3], false, false);
            const _Float16* arow = A + (size_t)rl * astride + 128 * b + offg;
            const h8_t a0 = *reinterpret_cast<const h8_t*>(arow);
            const h8_t a2 = *reinterpret_cast<const h8_t*>(arow + 16);
            const h8_t a1 = *reinterpret_cast<const h8_t*>(arow + 64);
            const h8_t a3 = *reinterpret_cast<const h8_t*>(arow + 80);
            const f4_t z = {0.f, 0.f, 0.f, 0.f};
            f4_t ce = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, q4_word_exact(s01[0]), z, 0, 0, 0);
            ce = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, q4_word_exact(s23[0]), ce, 0, 0, 0);
            f4_t co = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, q4_word_exact(s01[1]), z, 0, 0, 0);
            co = __builtin_amdgcn_mfma_f32_16x16x32_f16(a3, q4_word_exact(s23[1]), co, 0, 0, 0);
            fold(ce, 2 * b);
            fold(co, 2 * b + 1);
        };
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            u4_t w0, w1;
            const u4_t a = t.w[p][0], b = t.w[p][1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w0[j] = low8 ? a[j] : b[j];
                w1[j] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(low8 ? b[j] : a[j]), 0x128, 0xF, 0xF, false);
            }
            do_block(w0, 2 * p);
            do_block(w1, 2 * p + 1);
        }
        if constexpr (NB & 1) do_block(t.tail, NB - 1);

        // rows m (hi) and M + m (lo) of column n0 + rl: through the wave's LDS tile
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the table reads above are done
#pragma unroll
        for (int e = 0; e < 4; ++e) otw[(4 * g + e) * 16 + rl] = y[e];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (g < M) Y[(size_t)g * N + n0 + rl] = otw[g * 16 + rl] + otw[(M + g) * 16 + rl];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // before the next tile's table writes
    };

    for (;;) {
        load_tile(tb, tile + stride);
        compute(ta, tile * 16);
        tile += stride;
        if (tile >= ntiles) break;
        load_tile(ta, tile + stride);
        compute(tb, tile * 16);
        tile += stride;
        if (tile >= ntiles) break;
    }
}

int fx_device_cus()
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

template <int SBT, int NB>
hipError_t launch_fx_nb(const uint32_t* wq, const void* S, const void* B, const float* x, float* y, int M, int N,
                        hipStream_t st)
{
    auto kern = qgemv_q4_f32x_mfma_kernel<SBT, NB>;
    const size_t lds = (size_t)16 * (NB * 128 + kFxAPad) * 2 + (size_t)2 * kFxMaxGroups * 16 * 4 + 4 * kFxWaveLds;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kFxThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    // as few rounds of tiles as the resident waves allow, spread evenly: every wave then takes
    // that many tiles or one fewer
    const int ntiles = N / 16, waves = per_cu * fx_device_cus() * 4;
    const int rounds = (ntiles + waves - 1) / waves;
    const int grid = std::max(1, ((ntiles + rounds - 1) / rounds + 3) / 4);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kFxThreads), lds, st, wq, S, B, x, y, M, N);
    return hipGetLastError();
}

template <int SBT>
hipError_t launch_fx(const uint32_t* wq, const void* S, const void* B, const float* x, float* y, int M, int N, int K,
                     hipStream_t st)
{
    switch (K / 128) {
    case 1: return launch_fx_nb<SBT, 1>(wq, S, B, x, y, M, N, st);
    case 2: return launch_fx_nb<SBT, 2>(wq, S, B, x, y, M, N, st);
    case 3: return launch_fx_nb<SBT, 3>(wq, S, B, x, y, M, N, st);
    case 4: return launch_fx_nb<SBT, 4>(wq, S, B, x, y, M, N, st);
    case 5: return launch_fx_nb<SBT, 5>(wq, S, B, x, y, M, N, st);
    case 6: return launch_fx_nb<SBT, 6>(wq, S, B, x, y, M, N, st);
    case 7: return launch_fx_nb<SBT, 7>(wq, S, B, x, y, M, N, st);
    default: return launch_fx_nb<SBT, 8>(wq, S, B, x, y, M, N, st);
    }
}

}  // namespace

bool qgemv_q4_f32x_mfma_supported(int M, int N, int K, int group_size)
{
    // the weights' buffer range (N * K / 2 bytes) stays below 2^31
    return M >= 1 && M <= 4 && N >= 16 && N % 16 == 0 && K >= 128 && K <= kFxMaxK && K % 128 == 0 &&
           group_size == 64 && (size_t)N * K / 2 < ((size_t)1 << 31);
}

hipError_t launch_qgemv_q4_f32x_mfma(const uint32_t* wq, const void* S, const void* B, int sbt, const float* x,
                                     float* y, int M, int N, int K, hipStream_t st)
{
    if (sbt == DT_F16) return launch_fx<DT_F16>(wq, S, B, x, y, M, N, K, st);
    if (sbt == DT_F32) return launch_fx<DT_F32>(wq, S, B, x, y, M, N, K, st);
    return launch_fx<DT_BF16>(wq, S, B, x, y, M, N, K, st);
}

}  // namespace cellm
