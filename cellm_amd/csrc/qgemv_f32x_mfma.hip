// q4 affine GEMV with f32 activations on MFMA, exact in the nibbles (M <= 4 rows, long N).
//
// The reference dequantizes each weight to f32 and multiplies the f32 x
// (crates/cellm-model/src/lfm.rs:985-1066; the affine lm_head lfm.rs:700-741):
//   y[m,n] = sum_k (q[n,k] s[n,g(k)] + b[n,g(k)]) x[m,k].
// Per group of 64 k the scale and bias factor out of the dot product:
//   y[m,n] = sum_g ( s[n,g] * sum_{k in g} q[n,k] x[m,k]  +  b[n,g] * sum_{k in g} x[m,k] ).
// The inner sums run on v_mfma_i32_16x16x64_i8: the nibbles are the B bytes as they are,
// and each x row becomes three signed 8-bit digits.  x' = rint(x * 2^sh), one power of two
// per row chosen from the row's largest |x| so that |x'| <= 2^20, and
//   x' = d0 * 2^14 + d1 * 2^7 + d2,   |d0|, |d1|, |d2| <= 64,
// in A rows m, M + m and 2M + m.  Each group's integer sum is exact; it is folded in f32 as
// Y_d += s * acc_d (plus b * sum(x) on the d0 rows, pre-divided by 2^(14 - sh), a power of
// two), and y = 2^-sh * (2^14 Y_0 + 2^7 Y_1 + Y_2).  x is carried to 2^-20 of the row's
// largest |x| (the f32-x VALU kernels carry each element to about 22 bits through two f16
// parts); the reference order is matched to well within 3e-5 normwise.
//
// MFMA k-slots and groups: a lane (row n = lane%16, slot group g = lane/16) loads 16
// bytes of its row per 128-k block, k = 32g .. 32g+31, i.e. words w0..w3 of 8 nibbles.
// A 64-k step over the four lanes' data would mix the block's two groups;
// v_permlane32_swap of (w0, w1) and of (w2, w3) moves words between the lane halves so
// that each step holds one group:
//   R0 = swap(w0,w1).first : g = 0,1,2,3 -> k 0, 32, 8, 40 (+0..7)     group 0 of the block
//   R1 = swap(w0,w1).second: g = 0,1,2,3 -> k 64, 96, 72, 104           group 1
//   R2 = swap(w2,w3).first : k 16, 48, 24, 56                           group 0
//   R3 = swap(w2,w3).second: k 80, 112, 88, 120                         group 1
// A lane's B operand for a group is (nibbles 0,2,4,6 | 1,3,5,7) of its first word, then of
// its second; X is staged in LDS in exactly that order per (row, block, group, lane group),
// so the A operand is one 16-byte LDS read.  (The MFMA contracts A and B over the same
// register positions, whatever k those hold.)
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "launch_util.hpp"

namespace cellm {

namespace {

// eight waves per block (measured 4 % faster than four and than sixteen at 896->151936)
constexpr int kFxThreads = 512;
constexpr int kFxWaves = kFxThreads / 64;
constexpr int kFxMaxK = 1024;
constexpr int kFxMaxGroups = kFxMaxK / 64;
constexpr int kFxAPad = 16;       // bytes after each staged digit row (rows then start 4 banks apart)
constexpr int kFxWaveLds = 2048;  // per wave: the tile's (scale, bias) table, then its output tile

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

// Eight waves per block; wave w of block b takes tiles b*8 + w, += gridDim.x*8, a tile being
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
    int8_t* A = reinterpret_cast<int8_t*>(smem);                          // [16 digit rows][astride] bytes
    float* SX = reinterpret_cast<float*>(smem + (size_t)16 * astride);   // [kFxMaxGroups][16]: d0 rows' sum x
    float* P2 = SX + kFxMaxGroups * 16;                                   // [4]: 2^-sh per x row
    uint32_t* RMAX = reinterpret_cast<uint32_t*>(P2 + 4);                 // [4]: bits of the row's max |x|
    unsigned char* wave_lds = reinterpret_cast<unsigned char*>(RMAX + 4);
    // the wave index as a uniform (scalar) value, so the tile loop is a scalar loop
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane & 15, g = lane >> 4;
    const int ntiles = N >> 4, stride = gridDim.x * kFxWaves;
    constexpr uint32_t row_bytes = K / 2;
    const auto wr = buffer_rsrc(const_cast<uint32_t*>(W), (uint32_t)ntiles * 16u * row_bytes);
    const bool low8 = (rl & 8) == 0;

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

    int tile = blockIdx.x * kFxWaves + wave;
    FxTile<NB> ta, tb;
    load_tile(ta, tile);  // in flight while X is staged

    // ---- X as digit rows.  Item i = ((m * NB + b) * 2 + h) * 4 + g is the 16 k that lane group
    // g supplies for group h of block b: two words of 8 k at kb = 128b + 64h + {0,32,8,40}[g]
    // and kb + 16, each in the order 0,2,4,6,1,3,5,7.  One item per thread (M * K / 16 <= 256).
    for (int i = threadIdx.x; i < (16 - 3 * M) * (astride >> 4); i += kFxThreads)
        reinterpret_cast<u4_t*>(A + (size_t)3 * M * astride)[i] = u4_t{0u, 0u, 0u, 0u};
    for (int i = threadIdx.x; i < kFxMaxGroups * 16; i += kFxThreads) SX[i] = 0.0f;
    if (threadIdx.x < 4) RMAX[threadIdx.x] = 0u;
    const int items = M * (K / 16), it = min((int)threadIdx.x, items - 1);
    const int im = it / (K / 16), ir = it - im * (K / 16);
    const int ib = ir >> 3, ih = (ir >> 2) & 1, ig = ir & 3;
    const int kb = 128 * ib + 64 * ih + (ig & 1) * 32 + (ig >> 1) * 8;
    float xv[16];
    {
        const f4_t* r0 = reinterpret_cast<const f4_t*>(X + (size_t)im * K + kb);
        const f4_t* r1 = reinterpret_cast<const f4_t*>(X + (size_t)im * K + kb + 16);
        const f4_t a0 = r0[0], a1 = r0[1], c0 = r1[0], c1 = r1[1];
        constexpr int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
        const float w0[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const float w1[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xv[j] = w0[order[j]];
            xv[8 + j] = w1[order[j]];
        }
    }
    float mx = 0.0f, xs = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        mx = fmaxf(mx, fabsf(xv[j]));
        xs += xv[j];
    }
    xs = group_sum<4>(xs);  // the group's 64 k: four consecutive items (items % 4 == 0)
    __syncthreads();        // RMAX cleared
    if ((int)threadIdx.x < items) atomicMax(&RMAX[im], __builtin_bit_cast(uint32_t, mx));  // |x| >= 0: bits order as values
    __syncthreads();
    if ((int)threadIdx.x < items) {
        const float rmax = __builtin_bit_cast(float, RMAX[im]);
        int e = 0;
        (void)__builtin_frexpf(rmax, &e);
        const int sh = (rmax > 0.0f && rmax <= 3.402823466e38f) ? min(20 - e, 140) : 0;
        uint32_t dw[3][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xp = rintf(__builtin_ldexpf(xv[4 * q + j], sh));  // |xp| <= 2^20
                const float d0 = rintf(xp * 0.00006103515625f);             // / 2^14
                const float r = xp - d0 * 16384.0f;                          // |r| <= 2^13
                const float d1 = rintf(r * 0.0078125f);                      // / 2^7
                const float d2 = r - d1 * 128.0f;
                b0 |= ((uint32_t)(int)d0 & 0xFFu) << (8 * j);
                b1 |= ((uint32_t)(int)d1 & 0xFFu) << (8 * j);
                b2 |= ((uint32_t)(int)d2 & 0xFFu) << (8 * j);
            }
            dw[0][q] = b0;
            dw[1][q] = b1;
            dw[2][q] = b2;
        }
#pragma unroll
        for (int d = 0; d < 3; ++d)
            *reinterpret_cast<u4_t*>(A + (size_t)(d * M + im) * astride + 16 * ir) = u4_t{dw[d][0], dw[d][1], dw[d][2], dw[d][3]};
        if (ig == 0) SX[(2 * ib + ih) * 16 + im] = __builtin_ldexpf(xs, sh - 14);  // exact: a power of two
        if (ir == 0) P2[im] = __builtin_ldexpf(1.0f, -sh);
    }
    __syncthreads();
    if (tile >= ntiles) return;

    float2* sbw = reinterpret_cast<float2*>(wave_lds + wave * kFxWaveLds);  // [16 groups][16 rows]: no bank conflicts
    float* otw = reinterpret_cast<float*>(wave_lds + wave * kFxWaveLds);    // [16][16], after the folds

    auto compute = [&](const FxTile<NB>& t, int n0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sbw[(4 * g + j) * 16 + rl] = make_float2(raw_to_f32<SBT>(t.s[j]), raw_to_f32<SBT>(t.b[j]));
        f4_t y = {0.f, 0.f, 0.f, 0.f};
        // one group's integer sums of rows 4g..4g+3 (digit rows) for column rl
        auto fold = [&](const i4_t& acc, int grp) {
            const f4_t sx = *reinterpret_cast<const f4_t*>(SX + grp * 16 + 4 * g);
            const float2 sb = sbw[grp * 16 + rl];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = fmaf((float)acc[e], sb.x, fmaf(sb.y, sx[e], y[e]));
        };
        auto do_block = [&](const u4_t& w, int b) {
            const auto s01 = __builtin_amdgcn_permlane32_swap(w[0], w[1], false, false);
            const auto s23 = __builtin_amdgcn_permlane32_swap(w[2], w[3], false, false);
            const uint32_t m4 = 0x0F0F0F0Fu;
            const i4_t b0 = {(int)(s01[0] & m4), (int)((s01[0] >> 4) & m4), (int)(s23[0] & m4), (int)((s23[0] >> 4) & m4)};
            const i4_t b1 = {(int)(s01[1] & m4), (int)((s01[1] >> 4) & m4), (int)(s23[1] & m4), (int)((s23[1] >> 4) & m4)};
            const int8_t* arow = A + (size_t)rl * astride + 128 * b + 16 * g;
            const i4_t a0 = *reinterpret_cast<const i4_t*>(arow);
            const i4_t a1 = *reinterpret_cast<const i4_t*>(arow + 64);
            const i4_t z = {0, 0, 0, 0};
            fold(__builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, z, 0, 0, 0), 2 * b);
            fold(__builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, z, 0, 0, 0), 2 * b + 1);
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

        // digit rows m, M + m and 2M + m of column n0 + rl: through the wave's LDS tile
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the table reads above are done
#pragma unroll
        for (int e = 0; e < 4; ++e) otw[(4 * g + e) * 16 + rl] = y[e];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (g < M)
            Y[(size_t)g * N + n0 + rl] =
                P2[g] * (16384.0f * otw[g * 16 + rl] + (128.0f * otw[(M + g) * 16 + rl] + otw[(2 * M + g) * 16 + rl]));
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

// ---- int8 rows, f32 x: y[m,n] = (sum_k w[n,k] x[m,k]) * s[n] (+ bias[n])
// (crates/cellm-kernels/src/cpu_kernels.rs:66-133, matmul_i8_f32 per row; the Llama lm_head loop
// llama.rs:602-643 at several sessions).  The same three-digit x rows as above, and the int8
// weights are the B bytes as they are: a lane (column n = lane%16, slot group g = lane/16) holds
// 16 bytes of its row per 64-k block, k = 64b + 16g .. +15 in natural order, and A is staged in
// that order.  No group scale splits the sum, so each digit row accumulates over the whole K in
// one i32 accumulator: |d| <= 64, |w| <= 127, K <= 1024 keep every partial sum below 2^23, so it
// converts to f32 exactly, and the row scale is applied once, after the sum, as the reference
// does.  y = s * 2^-sh * (2^14 Y_0 + 2^7 Y_1 + Y_2).
constexpr int kI8FxMaxK = 1024;

template <int NB>
struct I8FxTile {
    u4_t w[NB / 2 > 0 ? NB / 2 : 1][2];
    u4_t tail;
    uint32_t s;
    float bias;
};

template <int SBT, int NB>
__global__ __launch_bounds__(kFxThreads) void qgemv_i8_f32x_mfma_kernel(const int8_t* __restrict__ W,
                                                                        const void* __restrict__ S, int per_channel,
                                                                        const float* __restrict__ bias,
                                                                        const float* __restrict__ X,
                                                                        float* __restrict__ Y, int M, int N)
{
    constexpr int K = NB * 64, NP = NB / 2, astride = K + kFxAPad;
    extern __shared__ __align__(16) unsigned char smem[];
    int8_t* A = reinterpret_cast<int8_t*>(smem);                         // [16 digit rows][astride] bytes
    float* P2 = reinterpret_cast<float*>(smem + (size_t)16 * astride);  // [4]: 2^-sh per x row
    uint32_t* RMAX = reinterpret_cast<uint32_t*>(P2 + 4);                // [4]: bits of the row's max |x|
    float* wave_out = reinterpret_cast<float*>(RMAX + 4);                // [waves][16][16]: a tile's digit sums
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rl = lane & 15, g = lane >> 4;
    const int ntiles = N >> 4, stride = gridDim.x * kFxWaves;
    constexpr uint32_t row_bytes = K;
    const auto wr = buffer_rsrc(const_cast<int8_t*>(W), (uint32_t)ntiles * 16u * row_bytes);
    const bool low8 = (rl & 8) == 0;

    // a tile's loads: 16 rows as full 128-byte row segments (two 64-k blocks; load h covers rows
    // 8h..8h+7, lane (rl, g) taking row (rl & 7) + 8h at byte 16g + 64((rl >> 3) ^ h)), the odd
    // last block, the row's scale and bias; a tile past the end loads through an out-of-range
    // buffer offset (zeros, no traffic) so every iteration issues the same loads
    auto load_tile = [&](I8FxTile<NB>& t, int tile) {
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
        t.s = load_raw<SBT>(S, per_channel ? (size_t)(n0 + rl) : 0);
        const float b = *(bias ? bias + n0 + rl : X);  // unconditional load (X when there is no bias)
        t.bias = bias ? b : 0.0f;
    };

    int tile = blockIdx.x * kFxWaves + wave;
    I8FxTile<NB> ta, tb;
    load_tile(ta, tile);  // in flight while X is staged

    // ---- X as digit rows in natural k order: item i = m * (K / 16) + r is 16 k of row m
    for (int i = threadIdx.x; i < (16 - 3 * M) * (astride >> 4); i += kFxThreads)
        reinterpret_cast<u4_t*>(A + (size_t)3 * M * astride)[i] = u4_t{0u, 0u, 0u, 0u};
    if (threadIdx.x < 4) RMAX[threadIdx.x] = 0u;
    const int items = M * (K / 16), it = min((int)threadIdx.x, items - 1);
    const int im = it / (K / 16), ir = it - im * (K / 16);
    float xv[16];
    {
        const f4_t* r0 = reinterpret_cast<const f4_t*>(X + (size_t)im * K + 16 * ir);
        const f4_t a0 = r0[0], a1 = r0[1], a2 = r0[2], a3 = r0[3];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[j] = a0[j];
            xv[4 + j] = a1[j];
            xv[8 + j] = a2[j];
            xv[12 + j] = a3[j];
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(xv[j]));
    __syncthreads();  // RMAX cleared
    if ((int)threadIdx.x < items) atomicMax(&RMAX[im], __builtin_bit_cast(uint32_t, mx));  // |x| >= 0: bits order as values
    __syncthreads();
    if ((int)threadIdx.x < items) {
        const float rmax = __builtin_bit_cast(float, RMAX[im]);
        int e = 0;
        (void)__builtin_frexpf(rmax, &e);
        const int sh = (rmax > 0.0f && rmax <= 3.402823466e38f) ? min(20 - e, 140) : 0;
        uint32_t dw[3][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xp = rintf(__builtin_ldexpf(xv[4 * q + j], sh));  // |xp| <= 2^20
                const float d0 = rintf(xp * 0.00006103515625f);             // / 2^14
                const float r = xp - d0 * 16384.0f;                          // |r| <= 2^13
                const float d1 = rintf(r * 0.0078125f);                      // / 2^7
                const float d2 = r - d1 * 128.0f;
                b0 |= ((uint32_t)(int)d0 & 0xFFu) << (8 * j);
                b1 |= ((uint32_t)(int)d1 & 0xFFu) << (8 * j);
                b2 |= ((uint32_t)(int)d2 & 0xFFu) << (8 * j);
            }
            dw[0][q] = b0;
            dw[1][q] = b1;
            dw[2][q] = b2;
        }
#pragma unroll
        for (int d = 0; d < 3; ++d)
            *reinterpret_cast<u4_t*>(A + (size_t)(d * M + im) * astride + 16 * ir) = u4_t{dw[d][0], dw[d][1], dw[d][2], dw[d][3]};
        if (ir == 0) P2[im] = __builtin_ldexpf(1.0f, -sh);
    }
    __syncthreads();
    if (tile >= ntiles) return;

    float* otw = wave_out + wave * 256;  // [16 digit rows][16 columns]
    const int8_t* arow = A + (size_t)rl * astride + 16 * g;

    auto compute = [&](const I8FxTile<NB>& t, int n0) {
        i4_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            u4_t w0, w1;
            const u4_t a = t.w[p][0], b = t.w[p][1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w0[j] = low8 ? a[j] : b[j];
                w1[j] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(low8 ? b[j] : a[j]), 0x128, 0xF, 0xF, false);
            }
            const i4_t x0 = *reinterpret_cast<const i4_t*>(arow + 128 * p);
            const i4_t x1 = *reinterpret_cast<const i4_t*>(arow + 128 * p + 64);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, __builtin_bit_cast(i4_t, w0), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, __builtin_bit_cast(i4_t, w1), acc, 0, 0, 0);
        }
        if constexpr (NB & 1) {
            const i4_t x0 = *reinterpret_cast<const i4_t*>(arow + 64 * (NB - 1));
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, __builtin_bit_cast(i4_t, t.tail), acc, 0, 0, 0);
        }
        // lane (rl, g) holds digit rows 4g..4g+3 of column n0 + rl; the three digits of x row m
        // meet through the wave's LDS tile
#pragma unroll
        for (int e = 0; e < 4; ++e) otw[(4 * g + e) * 16 + rl] = (float)acc[e];  // exact: |acc| < 2^23
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (g < M) {
            const float v = P2[g] * (16384.0f * otw[g * 16 + rl] + (128.0f * otw[(M + g) * 16 + rl] + otw[(2 * M + g) * 16 + rl]));
            Y[(size_t)g * N + n0 + rl] = v * raw_to_f32<SBT>(t.s) + t.bias;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // before the next tile's writes
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
    const size_t lds = (size_t)16 * (NB * 128 + kFxAPad) + (size_t)kFxMaxGroups * 16 * 4 + 32 + kFxWaves * kFxWaveLds;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kFxThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    // as few rounds of tiles as the resident waves allow, spread evenly: every wave then takes
    // that many tiles or one fewer
    const int ntiles = N / 16, waves = per_cu * fx_device_cus() * kFxWaves;
    const int rounds = (ntiles + waves - 1) / waves;
    const int grid = std::max(1, ((ntiles + rounds - 1) / rounds + kFxWaves - 1) / kFxWaves);
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

template <int SBT, int NB>
hipError_t launch_i8fx_nb(const int8_t* w, const void* S, int per_channel, const float* bias, const float* x, float* y,
                          int M, int N, hipStream_t st)
{
    auto kern = qgemv_i8_f32x_mfma_kernel<SBT, NB>;
    const size_t lds = (size_t)16 * (NB * 64 + kFxAPad) + 32 + (size_t)kFxWaves * 256 * 4;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kFxThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int ntiles = N / 16, waves = per_cu * fx_device_cus() * kFxWaves;
    const int rounds = (ntiles + waves - 1) / waves;
    const int grid = std::max(1, ((ntiles + rounds - 1) / rounds + kFxWaves - 1) / kFxWaves);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kFxThreads), lds, st, w, S, per_channel, bias, x, y, M, N);
    return hipGetLastError();
}

template <int SBT>
hipError_t launch_i8fx(const int8_t* w, const void* S, int per_channel, const float* bias, const float* x, float* y,
                       int M, int N, int K, hipStream_t st)
{
    switch (K / 64) {
    case 2: return launch_i8fx_nb<SBT, 2>(w, S, per_channel, bias, x, y, M, N, st);
    case 3: return launch_i8fx_nb<SBT, 3>(w, S, per_channel, bias, x, y, M, N, st);
    case 4: return launch_i8fx_nb<SBT, 4>(w, S, per_channel, bias, x, y, M, N, st);
    case 5: return launch_i8fx_nb<SBT, 5>(w, S, per_channel, bias, x, y, M, N, st);
    case 6: return launch_i8fx_nb<SBT, 6>(w, S, per_channel, bias, x, y, M, N, st);
    case 7: return launch_i8fx_nb<SBT, 7>(w, S, per_channel, bias, x, y, M, N, st);
    case 8: return launch_i8fx_nb<SBT, 8>(w, S, per_channel, bias, x, y, M, N, st);
    case 9: return launch_i8fx_nb<SBT, 9>(w, S, per_channel, bias, x, y, M, N, st);
    case 10: return launch_i8fx_nb<SBT, 10>(w, S, per_channel, bias, x, y, M, N, st);
    case 11: return launch_i8fx_nb<SBT, 11>(w, S, per_channel, bias, x, y, M, N, st);
    case 12: return launch_i8fx_nb<SBT, 12>(w, S, per_channel, bias, x, y, M, N, st);
    case 13: return launch_i8fx_nb<SBT, 13>(w, S, per_channel, bias, x, y, M, N, st);
    case 14: return launch_i8fx_nb<SBT, 14>(w, S, per_channel, bias, x, y, M, N, st);
    case 15: return launch_i8fx_nb<SBT, 15>(w, S, per_channel, bias, x, y, M, N, st);
    default: return launch_i8fx_nb<SBT, 16>(w, S, per_channel, bias, x, y, M, N, st);
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

bool qgemv_i8_f32x_mfma_supported(int M, int N, int K)
{
    // one X item per thread (M * K / 16 <= 512 threads) and the weights' buffer range below 2^31
    return M >= 1 && M <= 4 && N >= 16 && N % 16 == 0 && K >= 128 && K <= kI8FxMaxK && K % 64 == 0 &&
           (size_t)N * K < ((size_t)1 << 31);
}

hipError_t launch_qgemv_i8_f32x_mfma(const int8_t* w, const void* S, int sdt, int per_channel, const float* bias,
                                     const float* x, float* y, int M, int N, int K, hipStream_t st)
{
    if (!qgemv_i8_f32x_mfma_supported(M, N, K)) return hipErrorInvalidValue;
    if (sdt == DT_F16) return launch_i8fx<DT_F16>(w, S, per_channel, bias, x, y, M, N, K, st);
    if (sdt == DT_F32) return launch_i8fx<DT_F32>(w, S, per_channel, bias, x, y, M, N, K, st);
    return launch_i8fx<DT_BF16>(w, S, per_channel, bias, x, y, M, N, K, st);
}

}  // namespace cellm
