// Row GEMVs for the remaining .cellm weight formats (gfx950):
//
//   f16        W [N][K] f16                         cpu_kernels.rs:135-214 (matmul_f16_f32)
//   i2         W [N][ceil(K/4)] u8, 2-bit codes low bits first, one f16 scale per row;
//              value = centroid(code) in {-1.5, -0.5, 0.5, 1.5}
//                scale mode 0 (Qwen, qwen.rs:1591-1606):   y = (sum x * c) * s
//                scale mode 1 (Gemma, gemma.rs:1673-1687): y = sum x * (c * s)
//   q1_0_g128  W [N][K/128 blocks of 18 B]: f16 d (little endian) + 128 sign bits,
//              element 8b+j = bit j of byte b, value d if set else -d
//              (qwen.rs:1004-1022, metal.rs:542-570)
//
// Layout of the fast kernel: a team of LPR lanes per output row; each lane
// streams whole units of the row (16 bytes: 8 f16 or 64 i2 codes; one 18-byte
// q1 block of 128 elements) and multiplies them with the matching activations
// staged in LDS as f32 for up to MT activation rows.  The lanes of a team read
// x at a stride of one unit (64 or 128 elements for i2 / q1), which would put
// every lane on the same LDS banks, so each unit of x is followed by 4 floats
// of padding.  Sums are per-lane then a team butterfly, compared with the
// reference's sequential sums at a relative tolerance.  Shapes the fast kernel
// does not take (unaligned rows, K that is not a whole number of units, rows
// too long for LDS) use a one-wave-per-row kernel that reads x from memory.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace cellm {

namespace {

constexpr int kBlock = 256;
constexpr int kPad = 4;  // floats of LDS padding after each unit of x

struct Q1Block {
    uint16_t h[9];  // f16 d, then 8 words of sign bits (little endian)
};

template <int FMT>
struct LowbitFmt;
template <>
struct LowbitFmt<LB_F16> {
    static constexpr int kElems = 8;  // elements per 16-byte unit
    using unit_t = u4_t;
    __device__ __forceinline__ static unit_t load(const uint8_t* row, int u)
    {
        return *reinterpret_cast<const u4_t*>(row + (size_t)u * 16);
    }
};
template <>
struct LowbitFmt<LB_I2> {
    static constexpr int kElems = 64;
    using unit_t = u4_t;
    __device__ __forceinline__ static unit_t load(const uint8_t* row, int u)
    {
        return *reinterpret_cast<const u4_t*>(row + (size_t)u * 16);
    }
};
template <>
struct LowbitFmt<LB_Q1> {
    static constexpr int kElems = 128;  // one 18-byte block, 2-byte aligned
    using unit_t = Q1Block;
    __device__ __forceinline__ static unit_t load(const uint8_t* row, int u)
    {
        const uint16_t* b = reinterpret_cast<const uint16_t*>(row + (size_t)u * 18);
        Q1Block q;
#pragma unroll
        for (int i = 0; i < 9; ++i) q.h[i] = b[i];
        return q;
    }
};

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// i2 centroid table: t[c] for code c (mode 1 folds the row scale in)
struct I2Table {
    float t0, t1, t2, t3;
    __device__ __forceinline__ float operator()(uint32_t c) const
    {
        const float lo = (c & 1u) ? t1 : t0;
        const float hi = (c & 1u) ? t3 : t2;
        return (c & 2u) ? hi : lo;
    }
};

__device__ __forceinline__ I2Table i2_table(float s, int mode)
{
    if (mode == 0) return I2Table{-1.5f, -0.5f, 0.5f, 1.5f};
    return I2Table{-1.5f * s, -0.5f * s, 0.5f * s, 1.5f * s};
}

template <int FMT, int LPR, int MT, int XT>
__global__ __launch_bounds__(kBlock) void lowbit_gemv_kernel(const uint8_t* __restrict__ w,
                                                             const uint16_t* __restrict__ S, int scale_mode,
                                                             const void* __restrict__ x, float* __restrict__ y, int M,
                                                             int N, int K, size_t row_bytes)
{
    constexpr int UE = LowbitFmt<FMT>::kElems;
    extern __shared__ __align__(16) float xs[];  // [MT][units][UE + kPad]
    const int units = K / UE;
    const int xstride = units * (UE + kPad);
    const int team = threadIdx.x / LPR, lane = threadIdx.x % LPR;
    const int n = blockIdx.x * (kBlock / LPR) + team;
    const bool active = n < N;
    const uint8_t* row = w + (size_t)min(n, N - 1) * row_bytes;
    float scale = 1.0f;
    if constexpr (FMT == LB_I2) scale = h2f(S[min(n, N - 1)]);

    // the lane's first two units are loaded before x is staged (one memory latency for both)
    using unit_t = typename LowbitFmt<FMT>::unit_t;
    unit_t pre[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int u = min(lane + p * LPR, units - 1);
        pre[p] = LowbitFmt<FMT>::load(row, u);
    }

    for (int m0 = 0; m0 < M; m0 += MT) {
        const int mt = min(MT, M - m0);
        for (int i = threadIdx.x; i < mt * K; i += kBlock) {
            const int m = i / K, k = i - m * K;
            xs[m * xstride + (k / UE) * (UE + kPad) + k % UE] = load_f32<XT>(x, (size_t)(m0 + m) * K + k);
        }
        __syncthreads();
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        if (active) {
            int p = 0;
            for (int u = lane; u < units; u += LPR, ++p) {
                const unit_t raw = (m0 == 0 && p < 2) ? (p == 0 ? pre[0] : pre[1]) : LowbitFmt<FMT>::load(row, u);
                const float* xu = xs + u * (UE + kPad);
                if constexpr (FMT == LB_F16) {
                    const h8_t wh = __builtin_bit_cast(h8_t, raw);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const f4_t a = *reinterpret_cast<const f4_t*>(xu + m * xstride);
                        const f4_t b = *reinterpret_cast<const f4_t*>(xu + m * xstride + 4);
                        float s = acc[m];
                        s = __builtin_fmaf((float)wh[0], a[0], s);
                        s = __builtin_fmaf((float)wh[1], a[1], s);
                        s = __builtin_fmaf((float)wh[2], a[2], s);
                        s = __builtin_fmaf((float)wh[3], a[3], s);
                        s = __builtin_fmaf((float)wh[4], b[0], s);
                        s = __builtin_fmaf((float)wh[5], b[1], s);
                        s = __builtin_fmaf((float)wh[6], b[2], s);
                        s = __builtin_fmaf((float)wh[7], b[3], s);
                        acc[m] = s;
                    }
                } else if constexpr (FMT == LB_I2) {
                    const I2Table tab = i2_table(scale, scale_mode);
#pragma unroll
                    for (int wd = 0; wd < 4; ++wd) {
                        const uint32_t word = raw[wd];
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) {
                            float v[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = tab((word >> (2 * (4 * q4 + e))) & 3u);
#pragma unroll
                            for (int m = 0; m < MT; ++m) {
                                const f4_t a = *reinterpret_cast<const f4_t*>(xu + m * xstride + wd * 16 + q4 * 4);
                                float s = acc[m];
                                s = __builtin_fmaf(v[0], a[0], s);
                                s = __builtin_fmaf(v[1], a[1], s);
                                s = __builtin_fmaf(v[2], a[2], s);
                                s = __builtin_fmaf(v[3], a[3], s);
                                acc[m] = s;
                            }
                        }
                    }
                } else {
                    const float d = h2f(raw.h[0]);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const uint32_t bits = raw.h[1 + t];
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) {
                            float v[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = (bits >> (4 * q4 + e)) & 1u ? d : -d;
#pragma unroll
                            for (int m = 0; m < MT; ++m) {
                                const f4_t a = *reinterpret_cast<const f4_t*>(xu + m * xstride + t * 16 + q4 * 4);
                                float s = acc[m];
                                s = __builtin_fmaf(v[0], a[0], s);
                                s = __builtin_fmaf(v[1], a[1], s);
                                s = __builtin_fmaf(v[2], a[2], s);
                                s = __builtin_fmaf(v[3], a[3], s);
                                acc[m] = s;
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = group_sum<LPR>(acc[m]);
        if (active && lane == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m < mt) {
                    float v = acc[m];
                    if (FMT == LB_I2 && scale_mode == 0) v = v * scale;
                    y[(size_t)(m0 + m) * N + n] = v;
                }
        }
        __syncthreads();
    }
}

// f16 x, i2 / q1 weights: the pair-packed form.  x is staged in LDS as half
// pairs in the order the weight bits meet them, with a per-unit correction,
// and each pair of weights becomes a half pair for v_dot2_f32_f16 (products
// of halves are exact in the f32 accumulate):
//   i2: word W of a unit holds codes 16w..16w+15; v_and_or(W >> 2j, 0x00030003,
//       0x64006400) = (1024 + q_j, 1024 + q_{j+8}).  Since the centroid is
//       q - 1.5, the unit's dot starts at -1025.5 * sum(x of the unit).
//   q1: word W = sign bits of elements 32w..32w+31;
//       ((~W << (15 - k)) & 0x80008000) | 0x3C003C00 = (+-1, +-1) for
//       elements k and k + 16 (sign set when the bit is clear); the block's
//       dot starts at 0 and is scaled by d.
// About 1.5 instructions per element instead of 4-6; the products are
// exact, the sums are f32 trees, and the i2 row scale is applied to the row
// sum in both scale modes (the modes differ only in rounding).
template <int FMT>
struct PairFmt;
template <>
struct PairFmt<LB_I2> {
    static constexpr int kPairs = 32;             // half pairs per unit (64 elements)
    static constexpr int kStride = 36;            // dwords per unit in LDS: 32 pairs + corr + pad (36 % 32 = 4)
    __device__ __forceinline__ static int pair_of(int e) { return (e >> 4) * 8 + (e & 7); }   // element -> pair
    __device__ __forceinline__ static int half_of(int e) { return (e >> 3) & 1; }              // low / high half
    static constexpr float kCorr = 1025.5f;
};
template <>
struct PairFmt<LB_Q1> {
    static constexpr int kPairs = 64;             // 128 elements
    static constexpr int kStride = 68;
    __device__ __forceinline__ static int pair_of(int e) { return (e >> 5) * 16 + (e & 15); }
    __device__ __forceinline__ static int half_of(int e) { return (e >> 4) & 1; }
    static constexpr float kCorr = 0.0f;
};

__device__ __forceinline__ float dot2h(uint32_t a, uint32_t b, float c)
{
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

template <int FMT, int LPR, int MT>
__global__ __launch_bounds__(kBlock) void lowbit_pair_kernel(const uint8_t* __restrict__ w,
                                                             const uint16_t* __restrict__ S,
                                                             const _Float16* __restrict__ x, float* __restrict__ y,
                                                             int M, int N, int K, size_t row_bytes, int rows_per_team)
{
    using P = PairFmt<FMT>;
    constexpr int UE = LowbitFmt<FMT>::kElems;
    constexpr int kTeams = kBlock / LPR;
    extern __shared__ __align__(16) uint32_t xl[];  // [MT][units][kStride]: pairs, then the correction
    const int units = K / UE;
    const int xstride = units * P::kStride;
    const int team = threadIdx.x / LPR, lane = threadIdx.x % LPR;
    // the block's rows: base + team + r * kTeams for r < rows_per_team (staging x once for all of them)
    const int base = blockIdx.x * kTeams * rows_per_team;
    using unit_t = typename LowbitFmt<FMT>::unit_t;
    unit_t pre[2];
    {
        const uint8_t* row0 = w + (size_t)min(base + team, N - 1) * row_bytes;
#pragma unroll
        for (int p = 0; p < 2; ++p) pre[p] = LowbitFmt<FMT>::load(row0, min(lane + p * LPR, units - 1));
    }

    for (int m0 = 0; m0 < M; m0 += MT) {
        const int mt = min(MT, M - m0);
        // pairs: thread -> one half of one pair
        uint16_t* xh = reinterpret_cast<uint16_t*>(xl);
        for (int i = threadIdx.x; i < mt * K; i += kBlock) {
            const int m = i / K, k = i - m * K, u = k / UE, e = k - u * UE;
            xh[2 * (m * xstride + u * P::kStride + P::pair_of(e)) + P::half_of(e)] =
                __builtin_bit_cast(uint16_t, x[(size_t)(m0 + m) * K + k]);
        }
        __syncthreads();
        // the correction: -kCorr * sum of the unit's x (f32), from the staged pairs
        if constexpr (FMT == LB_I2) {
            for (int j = threadIdx.x; j < mt * units; j += kBlock) {
                const int m = j / units, u = j - m * units;
                const uint32_t* xu = xl + m * xstride + u * P::kStride;
                float sum = 0.0f;
#pragma unroll 8
                for (int q = 0; q < P::kPairs; ++q) {
                    const h2_t h = __builtin_bit_cast(h2_t, xu[q]);
                    sum += (float)h[0] + (float)h[1];
                }
                reinterpret_cast<float*>(xl)[m * xstride + u * P::kStride + P::kPairs] = -P::kCorr * sum;
            }
            __syncthreads();
        }
        for (int r = 0; r < rows_per_team; ++r) {
        const int n = base + team + r * kTeams;
        if (n >= N) break;  // the same for the whole team
        const uint8_t* row = w + (size_t)n * row_bytes;
        float scale = 1.0f;
        if constexpr (FMT == LB_I2) scale = h2f(S[n]);
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        {
            int p = 0;
            for (int u = lane; u < units; u += LPR, ++p) {
                const unit_t raw = (m0 == 0 && r == 0 && p < 2) ? (p == 0 ? pre[0] : pre[1])
                                                                : LowbitFmt<FMT>::load(row, u);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m >= mt) break;
                    const uint32_t* xu = xl + m * xstride + u * P::kStride;
                    if constexpr (FMT == LB_I2) {
                        float d = reinterpret_cast<const float*>(xu)[P::kPairs];
#pragma unroll
                        for (int wd = 0; wd < 4; ++wd) {
                            const u4_t xa = *reinterpret_cast<const u4_t*>(xu + wd * 8);
                            const u4_t xb = *reinterpret_cast<const u4_t*>(xu + wd * 8 + 4);
                            const uint32_t W = raw[wd];
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const uint32_t h = ((W >> (2 * j)) & 0x00030003u) | 0x64006400u;
                                d = dot2h(h, j < 4 ? xa[j] : xb[j - 4], d);
                            }
                        }
                        acc[m] += d;
                    } else {
                        const float dscale = h2f(raw.h[0]);
                        float d = 0.0f;
#pragma unroll
                        for (int wd = 0; wd < 4; ++wd) {
                            const uint32_t Wn = ~((uint32_t)raw.h[1 + 2 * wd] | ((uint32_t)raw.h[2 + 2 * wd] << 16));
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const u4_t xq = *reinterpret_cast<const u4_t*>(xu + wd * 16 + q * 4);
#pragma unroll
                                for (int j = 0; j < 4; ++j) {
                                    const int k = q * 4 + j;
                                    const uint32_t h = ((Wn << (15 - k)) & 0x80008000u) | 0x3C003C00u;
                                    d = dot2h(h, xq[j], d);
                                }
                            }
                        }
                        acc[m] = __builtin_fmaf(dscale, d, acc[m]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = group_sum<LPR>(acc[m]);
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m < mt) y[(size_t)(m0 + m) * N + n] = FMT == LB_I2 ? acc[m] * scale : acc[m];
        }
        }
        __syncthreads();
    }
}

// Any shape: one wave per output row, x read from memory, elements strided
// over the lanes.
template <int FMT, int XT>
__global__ __launch_bounds__(kBlock) void lowbit_gemv_generic_kernel(const uint8_t* __restrict__ w,
                                                                     const uint16_t* __restrict__ S, int scale_mode,
                                                                     const void* __restrict__ x,
                                                                     float* __restrict__ y, int M, int N, int K,
                                                                     size_t row_bytes)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * (kBlock / 64) + wave;
    if (n >= N) return;
    const uint8_t* row = w + (size_t)n * row_bytes;
    float scale = 1.0f;
    if constexpr (FMT == LB_I2) scale = h2f(S[n]);
    const I2Table tab = i2_table(scale, scale_mode);
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int j = lane; j < K; j += 64) {
            float v;
            if constexpr (FMT == LB_F16) {
                v = h2f(reinterpret_cast<const uint16_t*>(row)[j]);
            } else if constexpr (FMT == LB_I2) {
                v = tab((row[j >> 2] >> (2 * (j & 3))) & 3u);
            } else {
                const uint8_t* blk = row + (size_t)(j >> 7) * 18;
                const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
                const int e = j & 127;
                v = (blk[2 + (e >> 3)] >> (e & 7)) & 1u ? d : -d;
            }
            acc = __builtin_fmaf(v, load_f32<XT>(x, (size_t)m * K + j), acc);
        }
        acc = group_sum<64>(acc);
        if (lane == 0) y[(size_t)m * N + n] = (FMT == LB_I2 && scale_mode == 0) ? acc * scale : acc;
    }
}

template <int FMT, int LPR, int MT>
hipError_t launch_fast(const uint8_t* w, const uint16_t* S, int mode, const void* x, int xdt, float* y, int M, int N,
                       int K, size_t row_bytes, size_t lds, hipStream_t st)
{
    const dim3 grid((N + kBlock / LPR - 1) / (kBlock / LPR));
    if (xdt == DT_F32)
        hipLaunchKernelGGL((lowbit_gemv_kernel<FMT, LPR, MT, DT_F32>), grid, dim3(kBlock), lds, st, w, S, mode, x, y,
                           M, N, K, row_bytes);
    else if (xdt == DT_F16)
        hipLaunchKernelGGL((lowbit_gemv_kernel<FMT, LPR, MT, DT_F16>), grid, dim3(kBlock), lds, st, w, S, mode, x, y,
                           M, N, K, row_bytes);
    else
        hipLaunchKernelGGL((lowbit_gemv_kernel<FMT, LPR, MT, DT_BF16>), grid, dim3(kBlock), lds, st, w, S, mode, x, y,
                           M, N, K, row_bytes);
    return hipGetLastError();
}

template <int FMT, int MT>
hipError_t launch_fast_lpr(int lpr, const uint8_t* w, const uint16_t* S, int mode, const void* x, int xdt, float* y,
                           int M, int N, int K, size_t row_bytes, size_t lds, hipStream_t st)
{
    switch (lpr) {
    case 4: return launch_fast<FMT, 4, MT>(w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    case 8: return launch_fast<FMT, 8, MT>(w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    case 16: return launch_fast<FMT, 16, MT>(w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    case 32: return launch_fast<FMT, 32, MT>(w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    default: return launch_fast<FMT, 64, MT>(w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    }
}

template <int FMT, int LPR, int MT>
hipError_t launch_pair(const uint8_t* w, const uint16_t* S, const void* x, float* y, int M, int N, int K,
                       size_t row_bytes, size_t lds, hipStream_t st)
{
    // rows per team: as many as keep about 1024 blocks (the x staging of a block is shared by all its rows)
    constexpr int kTeams = kBlock / LPR;
    const int rpt = std::max(1, std::min(16, N / (kTeams * 1024)));
    const dim3 grid((N + kTeams * rpt - 1) / (kTeams * rpt));
    hipLaunchKernelGGL((lowbit_pair_kernel<FMT, LPR, MT>), grid, dim3(kBlock), lds, st, w, S,
                       reinterpret_cast<const _Float16*>(x), y, M, N, K, row_bytes, rpt);
    return hipGetLastError();
}

template <int FMT, int MT>
hipError_t launch_pair_lpr(int lpr, const uint8_t* w, const uint16_t* S, const void* x, float* y, int M, int N, int K,
                           size_t row_bytes, size_t lds, hipStream_t st)
{
    switch (lpr) {
    case 4: return launch_pair<FMT, 4, MT>(w, S, x, y, M, N, K, row_bytes, lds, st);
    case 8: return launch_pair<FMT, 8, MT>(w, S, x, y, M, N, K, row_bytes, lds, st);
    case 16: return launch_pair<FMT, 16, MT>(w, S, x, y, M, N, K, row_bytes, lds, st);
    case 32: return launch_pair<FMT, 32, MT>(w, S, x, y, M, N, K, row_bytes, lds, st);
    default: return launch_pair<FMT, 64, MT>(w, S, x, y, M, N, K, row_bytes, lds, st);
    }
}

// ---------------------------------------------------------------------------
// q1_0_g128 with one activation row and long outputs: a sign-sum table.
//
// Byte j of block b holds the signs of elements 8 (16 b + j) + 0..7, so the
// byte's contribution to the row is T[16 b + j][byte] with
// T[g][v] = sum_i (bit i of v ? x[8 g + i] : -x[8 g + i]).  Each CU builds T
// for all K / 8 groups once (256 floats per group, 144 KB at K = 1152) and
// then spends one LDS lookup and one add per 8 weights, instead of building
// +-1 pairs and a dot2 per 2 weights.  T[g][v] = A[v & 15] + B[v >> 4], with
// A and B the 16 signed sums of elements 0..3 and 4..7 of the group.
// Lane = (row, block): a wave takes 64 / blocks-per-row rows at a time (7 at
// K = 1152, 63 of 64 lanes busy), each lane one 18-byte block (nine 2-byte
// loads, the next row group's issued before the current one is used); the
// blocks of a row meet in a per-wave LDS slot.
// ---------------------------------------------------------------------------
constexpr int kLutThreads = 512;
constexpr int kQ1Depth = 4;  // row groups in flight per wave
constexpr size_t kLutMaxBytes = (size_t)(1152 / 8) * 256 * 4;  // K <= 1152 (at most 9 blocks per row)

template <int XT>
__global__ __launch_bounds__(kLutThreads) void q1_lut_kernel(const uint8_t* __restrict__ w, const void* __restrict__ x,
                                                            float* __restrict__ y, int N, int K, int row_bytes,
                                                            int park_per_wave)
{
    extern __shared__ __align__(16) float lut[];  // [K / 8][256], 64 floats per wave, parked row sums
    const int G = K >> 3, nblk = K >> 7;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* slot = lut + (size_t)G * 256 + wave * 64;
    // the table: four threads per group, 64 entries each
    for (int u = tid; u < G * 4; u += kLutThreads) {
        const int g = u >> 2, part = u & 3;
        float xv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = load_f32<XT>(x, (size_t)g * 8 + i);
        float a[16], b[4];
#pragma unroll
        for (int c = 0; c < 16; ++c)
            a[c] = (((c & 1) ? xv[0] : -xv[0]) + ((c & 2) ? xv[1] : -xv[1])) + (((c & 4) ? xv[2] : -xv[2]) + ((c & 8) ? xv[3] : -xv[3]));
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int c = part * 4 + h;
            b[h] = (((c & 1) ? xv[4] : -xv[4]) + ((c & 2) ? xv[5] : -xv[5])) + (((c & 4) ? xv[6] : -xv[6]) + ((c & 8) ? xv[7] : -xv[7]));
        }
        float4* dst = reinterpret_cast<float4*>(lut + (size_t)g * 256 + part * 64);
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dst[h * 4 + q] = make_float4(a[4 * q] + b[h], a[4 * q + 1] + b[h], a[4 * q + 2] + b[h], a[4 * q + 3] + b[h]);
    }
    __syncthreads();

    const int R = 64 / nblk;  // rows per wave step
    const int r = lane / nblk, bk = lane - r * nblk;
    const int ngroups = (N + R - 1) / R;
    const int gw = blockIdx.x * (kLutThreads / 64) + wave, GW = gridDim.x * (kLutThreads / 64);
    const int my_groups = gw < ngroups ? (ngroups - 1 - gw) / GW + 1 : 0;
    float* park = lut + (size_t)G * 256 + (kLutThreads / 64) * 64 + (size_t)wave * park_per_wave;
    auto load = [&](int i, uint16_t (&dst)[9]) {
        // clamped: idle lanes and rows past N read a valid block whose result is never stored
        const int grp = min(gw + i * GW, ngroups - 1);
        const int row = min(grp * R + min(r, R - 1), N - 1);
        const uint16_t* p = reinterpret_cast<const uint16_t*>(w + (size_t)row * row_bytes + (size_t)bk * 18);
#pragma unroll
        for (int k = 0; k < 9; ++k) dst[k] = p[k];
    };
    const float* tb = lut + (size_t)bk * 16 * 256;
    auto group = [&](int i, const uint16_t (&c)[9]) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (c[1 + (j >> 1)] >> (8 * (j & 1))) & 0xFFu;
            sum += tb[j * 256 + byte];
        }
        slot[lane] = raw_to_f32<DT_F16>(c[0]) * sum;
        __builtin_amdgcn_wave_barrier();  // LDS operations of a wave complete in order
        if (lane < R) {
            // all (up to 9) block sums read at once, clamped, then added in block order
            float v9[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) v9[k] = slot[lane * nblk + min(k, nblk - 1)];
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < 9; ++k) t += k < nblk ? v9[k] : 0.0f;
            park[i * R + lane] = t;
        }
        __builtin_amdgcn_wave_barrier();
    };
    // kQ1Depth row groups in flight per wave; results parked in LDS until the end (a store in the loop
    // would turn every load wait into a full vmcnt(0) drain)
    uint16_t h[kQ1Depth][9];
#pragma unroll
    for (int p = 0; p < kQ1Depth; ++p) load(p, h[p]);
    for (int i0 = 0; i0 < my_groups; i0 += kQ1Depth) {
        // uniform control flow: every slot reloads (clamped past the end) and only the work is guarded;
        // an early exit from the unrolled slots made the compiler's merged waits full drains
#pragma unroll
        for (int p = 0; p < kQ1Depth; ++p) {
            const int i = i0 + p;
            uint16_t c[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) c[k] = h[p][k];
            load(i + kQ1Depth, h[p]);
            if (i < my_groups) group(i, c);
        }
    }
    for (int k = lane; k < my_groups * R; k += 64) {
        const int row = (gw + (k / R) * GW) * R + k % R;
        if (row < N) y[row] = park[k];
    }
}

// CU count of the current device, cached per device id (any id; guarded by a mutex).
static int lut_cus()
{
    static std::mutex mu;
    static std::vector<std::pair<int, int>> cached;  // (device, CUs)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const std::lock_guard<std::mutex> lk(mu);
    for (const auto& e : cached)
        if (e.first == dev) return e.second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    cached.emplace_back(dev, cus);
    return cus;
}

// LDS of the table kernel: the table, a 64-float slot per wave and each wave's parked row sums
// (0 if it exceeds one CU's 160 KB)
static size_t q1_lut_lds(int N, int K, int* park_per_wave)
{
    const int nblk = K >> 7, R = 64 / nblk;
    const int ngroups = (N + R - 1) / R, GW = lut_cus() * (kLutThreads / 64);
    *park_per_wave = ((ngroups + GW - 1) / GW) * R;
    const size_t lds = ((size_t)(K >> 3) * 256 + (kLutThreads / 64) * 64 + (size_t)(kLutThreads / 64) * *park_per_wave) * 4;
    return lds <= 160 * 1024 ? lds : 0;
}

template <int XT>
hipError_t launch_q1_lut(const uint8_t* w, const void* x, float* y, int N, int K, int row_bytes, size_t lds,
                         int park_per_wave, hipStream_t st)
{
    auto kern = q1_lut_kernel<XT>;
    // the dynamic LDS limit is raised once per device and kernel
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(done.load(std::memory_order_acquire) & bit)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        done.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL(kern, dim3(lut_cus()), dim3(kLutThreads), lds, st, w, x, y, N, K, row_bytes, park_per_wave);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_fmt(const uint8_t* w, const uint16_t* S, int mode, const void* x, int xdt, float* y, int M, int N,
                      int K, size_t row_bytes, hipStream_t st)
{
    constexpr int UE = LowbitFmt<FMT>::kElems;
    if constexpr (FMT == LB_Q1) {
        int park = 0;
        const size_t lut_lds = M == 1 && N >= 32768 && K % 128 == 0 && K > 0 &&
                                       (size_t)(K >> 3) * 256 * 4 <= kLutMaxBytes &&
                                       (reinterpret_cast<uintptr_t>(w) & 1u) == 0
                                   ? q1_lut_lds(N, K, &park)
                                   : 0;
        if (lut_lds > 0) {
            if (xdt == DT_F16) return launch_q1_lut<DT_F16>(w, x, y, N, K, (int)row_bytes, lut_lds, park, st);
            if (xdt == DT_F32) return launch_q1_lut<DT_F32>(w, x, y, N, K, (int)row_bytes, lut_lds, park, st);
            return launch_q1_lut<DT_BF16>(w, x, y, N, K, (int)row_bytes, lut_lds, park, st);
        }
    }
    if constexpr (FMT != LB_F16) {
        // f16 x: the pair-packed dot2 kernel (the i2 scale is applied to the row sum in both modes)
        const bool unit_ok = K > 0 && K % UE == 0 &&
                             (reinterpret_cast<uintptr_t>(w) & (FMT == LB_Q1 ? 1u : 15u)) == 0;
        const size_t per_row = (size_t)(K / UE) * PairFmt<FMT>::kStride * 4;
        if (xdt == DT_F16 && unit_ok && per_row <= 64 * 1024) {
            // q1 keeps its 64 sign pairs of a block live across the rows: at most 2 rows per pass
            int MT = M >= 4 && FMT == LB_I2 ? 4 : (M >= 2 ? 2 : 1);
            while (MT > 1 && MT * per_row > 64 * 1024) MT >>= 1;
            int lpr = 4;
            while (lpr < 64 && lpr < K / UE) lpr <<= 1;
            const size_t lds = (size_t)MT * per_row;
            if constexpr (FMT == LB_I2)
                if (MT == 4) return launch_pair_lpr<FMT, 4>(lpr, w, S, x, y, M, N, K, row_bytes, lds, st);
            if (MT == 2) return launch_pair_lpr<FMT, 2>(lpr, w, S, x, y, M, N, K, row_bytes, lds, st);
            return launch_pair_lpr<FMT, 1>(lpr, w, S, x, y, M, N, K, row_bytes, lds, st);
        }
    }
    const bool unit_ok =
        K % UE == 0 && (reinterpret_cast<uintptr_t>(w) & (FMT == LB_Q1 ? 1u : 15u)) == 0;
    const size_t per_row = (size_t)(K / UE) * (UE + kPad) * sizeof(float);
    int MT = M >= 4 ? 4 : (M >= 2 ? 2 : 1);
    while (MT > 1 && MT * per_row > 64 * 1024) MT >>= 1;
    if (unit_ok && K > 0 && per_row <= 64 * 1024) {
        const int units = K / UE;
        int lpr = 4;
        while (lpr < 64 && lpr < units) lpr <<= 1;
        const size_t lds = (size_t)MT * per_row;
        if (MT == 4) return launch_fast_lpr<FMT, 4>(lpr, w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
        if (MT == 2) return launch_fast_lpr<FMT, 2>(lpr, w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
        return launch_fast_lpr<FMT, 1>(lpr, w, S, mode, x, xdt, y, M, N, K, row_bytes, lds, st);
    }
    const dim3 grid((N + 3) / 4);
    if (xdt == DT_F32)
        hipLaunchKernelGGL((lowbit_gemv_generic_kernel<FMT, DT_F32>), grid, dim3(kBlock), 0, st, w, S, mode, x, y, M,
                           N, K, row_bytes);
    else if (xdt == DT_F16)
        hipLaunchKernelGGL((lowbit_gemv_generic_kernel<FMT, DT_F16>), grid, dim3(kBlock), 0, st, w, S, mode, x, y, M,
                           N, K, row_bytes);
    else
        hipLaunchKernelGGL((lowbit_gemv_generic_kernel<FMT, DT_BF16>), grid, dim3(kBlock), 0, st, w, S, mode, x, y, M,
                           N, K, row_bytes);
    return hipGetLastError();
}

}  // namespace

size_t lowbit_row_bytes(int fmt, int K)
{
    if (fmt == LB_F16) return (size_t)K * 2;
    if (fmt == LB_I2) return (size_t)(K + 3) / 4;
    return (size_t)(K / 128) * 18;
}

hipError_t launch_qgemv_lowbit(int fmt, const void* w, const uint16_t* S, int scale_mode, const void* x, int xdt,
                               float* y, int M, int N, int K, hipStream_t st)
{
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(w);
    const size_t rb = lowbit_row_bytes(fmt, K);
    if (fmt == LB_F16) return launch_fmt<LB_F16>(wb, S, scale_mode, x, xdt, y, M, N, K, rb, st);
    if (fmt == LB_I2) return launch_fmt<LB_I2>(wb, S, scale_mode, x, xdt, y, M, N, K, rb, st);
    return launch_fmt<LB_Q1>(wb, S, scale_mode, x, xdt, y, M, N, K, rb, st);
}

}  // namespace cellm
