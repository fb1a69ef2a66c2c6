// Quantized-weight decode GEMV for gfx950 (wave64, 256-thread workgroups).
//
//   int8 per-row:   y[m,n] = (sum_k W[n,k] * x[m,k]) * s[n] (+ bias[n])
//                   crates/cellm-kernels/src/cpu_kernels.rs:66-133 (matmul_i8_f32),
//                   crates/cellm-kernels/src/metal.rs:365-385 (mv_i8)
//   MLX q4 affine:  y[m,n] = sum_k (q[n,k] * S[n,k/64] + B[n,k/64]) * x[m,k]
//                   crates/cellm-model/src/lfm.rs:985-1066 (linear_i4_out_in)
//
// Work decomposition.  A "team" of LPR lanes (8..64, always inside one wave)
// owns R consecutive output rows.  The packed row is cut into 16-byte chunks
// (32 nibbles for q4, 16 bytes for int8); lane l of a team reads chunks
// l, l+LPR, ... with one global_load_dwordx4 each, so a team streams its rows
// as contiguous 16-byte segments and a wave reads whole rows back to back.
// All weight loads of a lane are issued before the activation vector is staged
// into LDS, so the x staging overlaps the HBM round trip.
//
// Activations live in LDS, pre-arranged as the half2 pairs the unpacked
// weights meet in v_dot2_f32_f16:
//   q4:   v_and_or_b32(w, 0x000F000F, 0x64006400) gives the half pair
//         (1024+q0, 1024+q4); the same mask on the 0x00F0 nibbles gives
//         (1024+16*q1, 1024+16*q5), met by (x1/16, x5/16).  One shift by 8
//         covers nibbles 2,6 and 3,7.  The 1024 offsets are removed by
//         starting each chunk's dot at -corr, corr = 1024 * sum(staged x),
//         so a 32-element chunk costs 4 shifts + 16 and_or + 16 dot2 per row.
//   int8: w ^ 0x80808080 turns int8 into u8 = w+128; v_and_or_b32 with
//         0x00FF00FF / 0x64006400 gives (1152+w0, 1152+w2) and, after a
//         shift, (1152+w1, 1152+w3); corr = 1152 * sum(x).
// Products of f16 values are exact in f32 and every sum is f32, so the only
// difference from the reference is summation order (checked to 1e-3 relative
// against the reference CPU order in tests/).
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
#ifndef CELLM_GEMV_UNROLL
#define CELLM_GEMV_UNROLL 4
#endif
constexpr int kUnroll = CELLM_GEMV_UNROLL;  // chunks per lane held in registers per pass

// Load order inside every kernel below: (1) this thread's activation words,
// (2) all weight chunks and their scale/bias bits for the first pass, (3)
// stage the activations into LDS.  Loads retire in issue order, so (3) waits
// only for (1) and the weight stream stays in flight while x is staged; the
// scale/bias bits are converted at their use, never right after the load.

// ---------------------------------------------------------------------------
// q4 affine, f16 activations
// ---------------------------------------------------------------------------

// One 8-element activation word -> LDS as the pairs (x0,x4), (x1/16,x5/16),
// (x2,x6), (x3/16,x7/16), plus per-chunk (corr, xsum) summed over the four
// words of a chunk, which sit in four adjacent lanes.
// xq layout: [MT][CPR][16] uint32; cx layout: [MT][CPR] float2.
__device__ __forceinline__ void stage_word_q4(u4_t raw, int idx, bool valid, uint32_t* xq, float2* cx)
{
    h8_t v = __builtin_bit_cast(h8_t, raw);
    const _Float16 inv16 = (_Float16)0.0625f;
    h2_t p0 = {v[0], v[4]};
    h2_t p1 = {v[1] * inv16, v[5] * inv16};
    h2_t p2 = {v[2], v[6]};
    h2_t p3 = {v[3] * inv16, v[7] * inv16};
    float corr = ((float)p0[0] + (float)p0[1]) + ((float)p1[0] + (float)p1[1]) +
                 ((float)p2[0] + (float)p2[1]) + ((float)p3[0] + (float)p3[1]);
    float xs = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) xs += (float)v[i];
    if (valid) *reinterpret_cast<u4_t*>(xq + (size_t)idx * 4) = u4_t{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
    corr = quad_sum(corr);
    xs = quad_sum(xs);
    if (valid && (idx & 3) == 0) cx[idx >> 2] = make_float2(1024.0f * corr, xs);
}

// f32 activations (the LFM runner's and the .cellm u32 runner's x) as two f16 parts.  Each
// 32-element chunk (4 words, in 4 adjacent lanes) is scaled by a power of two, x' = x * 2^sh, sh
// chosen from the chunk's largest |x| so that it lies in [2^13, 2^14): hi = RNE_f16(x') never
// overflows (|x| > 65504 alone would give hi = inf, lo = -inf and a NaN row sum) and small values
// stay clear of f16 subnormals, where hi, lo and lo / 16 lose bits.  Then x' = hi + lo with
// lo = RNE_f16(x' - hi): a nibble value times either part is exact in f32, so the dot over both
// parts keeps x to about 22 bits where one f16 rounding would keep 11.  Every product and partial
// sum of the chunk carries the exact factor 2^sh, and p2 = 2^-sh takes it out of the chunk's
// contribution (compute_pass_q4): bit for bit the unscaled sum wherever that stays in f16 normal
// range.  A chunk of zeros or with an infinite value keeps sh = 0 (fmaxf ignores NaN, which then
// propagates through the dot as it would unscaled).
// Eight f32 values -> the hi pairs at xq, the lo pairs at xq_lo (the layout of stage_word_q4),
// cx = (1024 * the pairs' sum over both parts, sum of the scaled x) and p2 per chunk.
__device__ __forceinline__ void stage_word_q4_x32(f4_t a, f4_t b, int idx, bool valid, uint32_t* xq, uint32_t* xq_lo,
                                                  float2* cx, float* p2)
{
    float xv[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(xv[i]));
    mx = group_max<4>(mx);
    int e = 0;
    (void)__builtin_frexpf(mx, &e);
    const int sh = (mx > 0.0f && mx <= 3.402823466e38f) ? min(14 - e, 126) : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = __builtin_ldexpf(xv[i], sh);
    h8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = (_Float16)xv[i];
        lo[i] = (_Float16)(xv[i] - (float)hi[i]);
    }
    const _Float16 inv16 = (_Float16)0.0625f;
    float corr = 0.0f;
    auto pack = [&](const h8_t& v, uint32_t* dst) {
        const h2_t q0 = {v[0], v[4]}, q1 = {v[1] * inv16, v[5] * inv16};
        const h2_t q2 = {v[2], v[6]}, q3 = {v[3] * inv16, v[7] * inv16};
        corr += ((float)q0[0] + (float)q0[1]) + ((float)q1[0] + (float)q1[1]) + ((float)q2[0] + (float)q2[1]) +
                ((float)q3[0] + (float)q3[1]);
        if (valid) *reinterpret_cast<u4_t*>(dst + (size_t)idx * 4) = u4_t{as_u32(q0), as_u32(q1), as_u32(q2), as_u32(q3)};
    };
    pack(hi, xq);
    pack(lo, xq_lo);
    float xs = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) xs += xv[i];
    corr = quad_sum(corr);
    xs = quad_sum(xs);
    if (valid && (idx & 3) == 0) {
        cx[idx >> 2] = make_float2(1024.0f * corr, xs);
        p2[idx >> 2] = __builtin_ldexpf(1.0f, -sh);
    }
}

// All MT * K / 8 words of f32 x -> LDS through stage_word_q4_x32, two 16-byte loads per word, in
// rounds of XW words per thread whose loads all issue before the round's first store (clamped,
// branch-free: padding rows and words past `total` read valid data whose results are never stored).
template <int XW>
__device__ __forceinline__ void stage_x_q4_x32(const float* __restrict__ x, int M, int K, int total, uint32_t* xq,
                                               uint32_t* xq_lo, float2* cx, float* p2)
{
    const int words = K >> 3;
    for (int base = 0; base < total; base += XW * kBlock) {
        f4_t ra[XW], rb[XW];
#pragma unroll
        for (int j = 0; j < XW; ++j) {
            // x rows are contiguous: word idx of row idx / words sits at x + 8 idx (rows past M
            // read the last real word; their results are never stored)
            const int idx = min(base + j * kBlock + (int)threadIdx.x, M * words - 1);
            const f4_t* p = reinterpret_cast<const f4_t*>(x + (size_t)idx * 8);
            ra[j] = p[0];
            rb[j] = p[1];
        }
#pragma unroll
        for (int j = 0; j < XW; ++j) {
            const int idx = base + j * kBlock + (int)threadIdx.x;
            stage_word_q4_x32(ra[j], rb[j], idx, idx < total, xq, xq_lo, cx, p2);
        }
    }
}

template <int XW>
__device__ __forceinline__ void load_x_words(const _Float16* __restrict__ x, int M, int K, int total, u4_t (&xr)[XW])
{
    const int words = K >> 3;
#pragma unroll
    for (int j = 0; j < XW; ++j) {
        // clamped, branch-free: padding rows m >= M and words past `total`
        // read valid data whose results are never stored
        // (x rows are contiguous: word idx sits at x + 8 idx, no division)
        const int idx = min((int)threadIdx.x + j * kBlock, min(total, M * words) - 1);
        xr[j] = *reinterpret_cast<const u4_t*>(x + (size_t)idx * 8);
    }
}

// The words of load_x_words -> LDS (stage_word_q4), then any further words of a large M*K.
template <int XW>
__device__ __forceinline__ void stage_x_q4(const u4_t (&xr)[XW], const _Float16* __restrict__ x, int M, int K,
                                           int total, uint32_t* xq, float2* cx)
{
#pragma unroll
    for (int j = 0; j < XW; ++j) {
        const int idx = (int)threadIdx.x + j * kBlock;
        stage_word_q4(xr[j], idx, idx < total, xq, cx);
    }
    for (int base = XW * kBlock; base < total; base += kBlock) {  // large M*K only
        const int idx = base + (int)threadIdx.x;
        const int words = K >> 3;
        u4_t raw = (idx < total && idx < M * words) ? *reinterpret_cast<const u4_t*>(x + (size_t)idx * 8)
                                                    : u4_t{0u, 0u, 0u, 0u};
        stage_word_q4(raw, idx, idx < total, xq, cx);
    }
}

template <int LPR, int R, int SBT, int U = kUnroll>
__device__ __forceinline__ void load_pass_q4(const u4_t* __restrict__ wq, const void* __restrict__ S,
                                             const void* __restrict__ B, int row0, int rstride, int c0, int N, int CPR,
                                             int gpr, int gshift, u4_t (&wv)[U][R], uint32_t (&sr)[U][R],
                                             uint32_t (&br)[U][R])
{
    // Addresses are clamped into the matrix instead of branching around the
    // loads: a lane whose chunk or row is out of range loads a valid element
    // and its result is never used (compute skips c >= CPR, rows >= N are not
    // stored).  Branch-free loads keep every conversion away from its load.
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * LPR, CPR - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(row0 + r * rstride, N - 1);
            wv[u][r] = __builtin_nontemporal_load(wq + (size_t)n * CPR + c);
            const size_t gi = (size_t)n * gpr + ((c << 5) >> gshift);
            sr[u][r] = load_raw<SBT>(S, gi);
            br[u][r] = load_raw<SBT>(B, gi);
        }
    }
}

template <int LPR, int R, int MT, int SBT, int U = kUnroll, bool XS = false>
__device__ __forceinline__ void compute_pass_q4(int c0, int CPR, const uint32_t* xq, const float2* cx,
                                                const u4_t (&wv)[U][R], const uint32_t (&sr)[U][R],
                                                const uint32_t (&br)[U][R], float (&acc)[R][MT],
                                                const uint32_t* xq_lo = nullptr, const float* p2 = nullptr)
{
    const uint32_t m0f = 0x000F000Fu, m1f = 0x00F000F0u, magic = 0x64006400u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = c0 + u * LPR;
        if (c < CPR) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const u4_t* xp = reinterpret_cast<const u4_t*>(xq + ((size_t)m * CPR + c) * 16);
                const u4_t xa = xp[0], xb = xp[1], xc = xp[2], xd = xp[3];
                const float2 cc = cx[(size_t)m * CPR + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const u4_t w = wv[u][r];
                    float d = -cc.x;
                    uint32_t h;
                    d = dot2(and_or(w[0], m0f, magic), xa[0], d);
                    d = dot2(and_or(w[0], m1f, magic), xa[1], d);
                    h = w[0] >> 8;
                    d = dot2(and_or(h, m0f, magic), xa[2], d);
                    d = dot2(and_or(h, m1f, magic), xa[3], d);
                    d = dot2(and_or(w[1], m0f, magic), xb[0], d);
                    d = dot2(and_or(w[1], m1f, magic), xb[1], d);
                    h = w[1] >> 8;
                    d = dot2(and_or(h, m0f, magic), xb[2], d);
                    d = dot2(and_or(h, m1f, magic), xb[3], d);
                    d = dot2(and_or(w[2], m0f, magic), xc[0], d);
                    d = dot2(and_or(w[2], m1f, magic), xc[1], d);
                    h = w[2] >> 8;
                    d = dot2(and_or(h, m0f, magic), xc[2], d);
                    d = dot2(and_or(h, m1f, magic), xc[3], d);
                    d = dot2(and_or(w[3], m0f, magic), xd[0], d);
                    d = dot2(and_or(w[3], m1f, magic), xd[1], d);
                    h = w[3] >> 8;
                    d = dot2(and_or(h, m0f, magic), xd[2], d);
                    d = dot2(and_or(h, m1f, magic), xd[3], d);
                    if constexpr (XS) {
                        // the low f16 parts of f32 x, same nibbles (the correction in cc.x covers both)
                        const u4_t* lp = reinterpret_cast<const u4_t*>(xq_lo + ((size_t)m * CPR + c) * 16);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const u4_t xl = lp[e];
                            d = dot2(and_or(w[e], m0f, magic), xl[0], d);
                            d = dot2(and_or(w[e], m1f, magic), xl[1], d);
                            h = w[e] >> 8;
                            d = dot2(and_or(h, m0f, magic), xl[2], d);
                            d = dot2(and_or(h, m1f, magic), xl[3], d);
                        }
                    }
                    if constexpr (XS)  // the chunk's x carried 2^sh: p2 = 2^-sh takes it out exactly
                        acc[r][m] += (raw_to_f32<SBT>(sr[u][r]) * d + raw_to_f32<SBT>(br[u][r]) * cc.y) *
                                     p2[(size_t)m * CPR + c];
                    else
                        acc[r][m] += raw_to_f32<SBT>(sr[u][r]) * d + raw_to_f32<SBT>(br[u][r]) * cc.y;
                }
            }
        }
    }
}

// MP: rows need more than one pass of kUnroll chunks per lane; the next pass
// is prefetched into a second register set (ping-pong) before the current one
// is consumed.  XS: x is f32, staged as hi and lo f16 parts (stage_word_q4_x32)
// and dotted with both; else x is f16.
template <int LPR, int R, int MT, int SBT, bool MP, bool XS = false>
__global__ __launch_bounds__(kBlock) void qgemv_q4_f16x_kernel(
    const u4_t* __restrict__ wq, const void* __restrict__ S, const void* __restrict__ B,
    const void* __restrict__ xv, float* __restrict__ y, int M, int N, int K, int gshift)
{
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 5;
    uint32_t* xq = lds;
    uint32_t* xq_lo = XS ? lds + (size_t)MT * CPR * 16 : nullptr;
    float2* cx = reinterpret_cast<float2*>(lds + (size_t)(XS ? 2 : 1) * MT * CPR * 16);
    float* p2 = XS ? reinterpret_cast<float*>(cx + (size_t)MT * CPR) : nullptr;  // f32 x: 2^-sh per chunk

    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * (kBlock / LPR) + team) * R;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int total = MT * (K >> 3);

    constexpr int XW = MT == 1 ? 4 : 8;
    u4_t wa[kUnroll][R];
    uint32_t sa[kUnroll][R], ba[kUnroll][R];
    if constexpr (XS) {
        // the weights first: x is a cache hit after the first blocks, the weights are not
        load_pass_q4<LPR, R, SBT>(wq, S, B, row0, 1, lane, N, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4_x32<XW / 2>(reinterpret_cast<const float*>(xv), M, K, total, xq, xq_lo, cx, p2);
    } else {
        const _Float16* x = reinterpret_cast<const _Float16*>(xv);
        u4_t xr[XW];
        load_x_words<XW>(x, M, K, total, xr);
        load_pass_q4<LPR, R, SBT>(wq, S, B, row0, 1, lane, N, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4<XW>(xr, x, M, K, total, xq, cx);
    }
    __syncthreads();
    if (row0 >= N) return;

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    if constexpr (!MP) {
        compute_pass_q4<LPR, R, MT, SBT, kUnroll, XS>(lane, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][R];
        uint32_t sb[kUnroll][R], bb[kUnroll][R];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR) load_pass_q4<LPR, R, SBT>(wq, S, B, row0, 1, c0 + P, N, CPR, gpr, gshift, wb, sb, bb);
            compute_pass_q4<LPR, R, MT, SBT, kUnroll, XS>(c0, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR)
                load_pass_q4<LPR, R, SBT>(wq, S, B, row0, 1, c0 + 2 * P, N, CPR, gpr, gshift, wa, sa, ba);
            compute_pass_q4<LPR, R, MT, SBT, kUnroll, XS>(c0 + P, CPR, xq, cx, wb, sb, bb, acc, xq_lo, p2);
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = group_sum<LPR>(acc[r][m]);
        }

    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = row0 + r;
            if (n < N) {
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m < M) y[(size_t)m * N + n] = acc[r][m];
            }
        }
    }
}

// Gate/up + SiLU (or tanh GELU) for MLX q4 in one launch (the mv2 + silu_mul
// pattern of the reference's fused graphs: metal.rs:512-541 and 232-243,
// llama_graph.rs:318-327; Gemma's gelu_tanh * up, gemma.rs:844-846).  A team owns
// output row n of both matrices: its two rows (gate, up) go through the same
// loads and dot as qgemv_q4_f16x_kernel's R = 2 rows, and lane 0 writes
// h[m, n] = act_mul(act, g, u).
template <int LPR, int SBT, int U = kUnroll>
__device__ __forceinline__ void load_pass_q4_gu(const u4_t* __restrict__ wg, const void* __restrict__ Sg,
                                                const void* __restrict__ Bg, const u4_t* __restrict__ wu,
                                                const void* __restrict__ Su, const void* __restrict__ Bu, int n, int c0,
                                                int N, int CPR, int gpr, int gshift, u4_t (&wv)[U][2],
                                                uint32_t (&sr)[U][2], uint32_t (&br)[U][2])
{
    const int nn = min(n, N - 1);  // clamped like load_pass_q4
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * LPR, CPR - 1);
        const size_t gi = (size_t)nn * gpr + ((c << 5) >> gshift);
        wv[u][0] = __builtin_nontemporal_load(wg + (size_t)nn * CPR + c);
        sr[u][0] = load_raw<SBT>(Sg, gi);
        br[u][0] = load_raw<SBT>(Bg, gi);
        wv[u][1] = __builtin_nontemporal_load(wu + (size_t)nn * CPR + c);
        sr[u][1] = load_raw<SBT>(Su, gi);
        br[u][1] = load_raw<SBT>(Bu, gi);
    }
}

template <int LPR, int MT, int SBT, bool MP, bool XS = false>
__global__ __launch_bounds__(kBlock) void qgemv_q4_gate_up_silu_kernel(
    const u4_t* __restrict__ wg, const void* __restrict__ Sg, const void* __restrict__ Bg,
    const u4_t* __restrict__ wu, const void* __restrict__ Su, const void* __restrict__ Bu,
    const void* __restrict__ xv, float* __restrict__ h, int M, int N, int K, int gshift, int act)
{
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 5;
    uint32_t* xq = lds;
    uint32_t* xq_lo = XS ? lds + (size_t)MT * CPR * 16 : nullptr;
    float2* cx = reinterpret_cast<float2*>(lds + (size_t)(XS ? 2 : 1) * MT * CPR * 16);
    float* p2 = XS ? reinterpret_cast<float*>(cx + (size_t)MT * CPR) : nullptr;  // f32 x: 2^-sh per chunk

    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int n = blockIdx.x * (kBlock / LPR) + team;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int total = MT * (K >> 3);

    constexpr int XW = MT == 1 ? 4 : 8;
    u4_t wa[kUnroll][2];
    uint32_t sa[kUnroll][2], ba[kUnroll][2];
    if constexpr (XS) {
        // f32 x as hi + lo f16 parts (stage_word_q4_x32); the weights first
        load_pass_q4_gu<LPR, SBT>(wg, Sg, Bg, wu, Su, Bu, n, lane, N, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4_x32<XW / 2>(reinterpret_cast<const float*>(xv), M, K, total, xq, xq_lo, cx, p2);
    } else {
        const _Float16* x = reinterpret_cast<const _Float16*>(xv);
        u4_t xr[XW];
        load_x_words<XW>(x, M, K, total, xr);
        load_pass_q4_gu<LPR, SBT>(wg, Sg, Bg, wu, Su, Bu, n, lane, N, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4<XW>(xr, x, M, K, total, xq, cx);
    }
    __syncthreads();
    if (n >= N) return;

    float acc[2][MT];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
    if constexpr (!MP) {
        compute_pass_q4<LPR, 2, MT, SBT, kUnroll, XS>(lane, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][2];
        uint32_t sb[kUnroll][2], bb[kUnroll][2];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR)
                load_pass_q4_gu<LPR, SBT>(wg, Sg, Bg, wu, Su, Bu, n, c0 + P, N, CPR, gpr, gshift, wb, sb, bb);
            compute_pass_q4<LPR, 2, MT, SBT, kUnroll, XS>(c0, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR)
                load_pass_q4_gu<LPR, SBT>(wg, Sg, Bg, wu, Su, Bu, n, c0 + 2 * P, N, CPR, gpr, gshift, wa, sa, ba);
            compute_pass_q4<LPR, 2, MT, SBT, kUnroll, XS>(c0 + P, CPR, xq, cx, wb, sb, bb, acc, xq_lo, p2);
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[r][m] = group_sum<LPR>(acc[r][m]);
        }
    if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) h[(size_t)m * N + n] = act_mul(act, acc[0][m], acc[1][m]);
    }
}

// Up to three MLX q4 matrices that share x in one launch (the q, k and v
// projections of the u32 runners), each with its own scales, group biases,
// optional projection bias (f32 [n], added after the row sum, as
// add_projection_bias_if_present does, qwen.rs:1132-1139) and output.  A team
// owns one row of the concatenation [seg0 rows; seg1 rows; seg2 rows]; the rows
// past the end repeat the last row and are not stored.  XS: f32 x as hi + lo
// f16 parts (stage_word_q4_x32).
struct Q4Seg {
    const u4_t* w;
    const void* S;
    const void* B;
    const float* bias;
    float* y;
    int n;
};
struct Q4Segs {
    Q4Seg g0, g1, g2;
};

template <int LPR, int MT, int SBT, bool MP, bool XS>
__global__ __launch_bounds__(kBlock) void qgemv_q4_segs_kernel(Q4Segs segs, const void* __restrict__ xv, int M,
                                                              int total_rows, int K, int gshift)
{
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 5;
    uint32_t* xq = lds;
    uint32_t* xq_lo = XS ? lds + (size_t)MT * CPR * 16 : nullptr;
    float2* cx = reinterpret_cast<float2*>(lds + (size_t)(XS ? 2 : 1) * MT * CPR * 16);
    float* p2 = XS ? reinterpret_cast<float*>(cx + (size_t)MT * CPR) : nullptr;  // f32 x: 2^-sh per chunk
    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int row = blockIdx.x * (kBlock / LPR) + team;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int total = MT * (K >> 3);

    int v = min(row, total_rows - 1);
    Q4Seg sg = segs.g0;
    if (v >= segs.g0.n) {
        v -= segs.g0.n;
        sg = segs.g1;
        if (v >= segs.g1.n) {
            v -= segs.g1.n;
            sg = segs.g2;
        }
    }
    constexpr int XW = MT == 1 ? 4 : 8;
    u4_t wa[kUnroll][1];
    uint32_t sa[kUnroll][1], ba[kUnroll][1];
    if constexpr (XS) {
        load_pass_q4<LPR, 1, SBT>(sg.w, sg.S, sg.B, v, 1, lane, sg.n, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4_x32<XW / 2>(reinterpret_cast<const float*>(xv), M, K, total, xq, xq_lo, cx, p2);
    } else {
        const _Float16* x = reinterpret_cast<const _Float16*>(xv);
        u4_t xr[XW];
        load_x_words<XW>(x, M, K, total, xr);
        load_pass_q4<LPR, 1, SBT>(sg.w, sg.S, sg.B, v, 1, lane, sg.n, CPR, gpr, gshift, wa, sa, ba);
        stage_x_q4<XW>(xr, x, M, K, total, xq, cx);
    }
    __syncthreads();
    if (row >= total_rows) return;

    float acc[1][MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[0][m] = 0.0f;
    if constexpr (!MP) {
        compute_pass_q4<LPR, 1, MT, SBT, kUnroll, XS>(lane, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][1];
        uint32_t sb[kUnroll][1], bb[kUnroll][1];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR)
                load_pass_q4<LPR, 1, SBT>(sg.w, sg.S, sg.B, v, 1, c0 + P, sg.n, CPR, gpr, gshift, wb, sb, bb);
            compute_pass_q4<LPR, 1, MT, SBT, kUnroll, XS>(c0, CPR, xq, cx, wa, sa, ba, acc, xq_lo, p2);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR)
                load_pass_q4<LPR, 1, SBT>(sg.w, sg.S, sg.B, v, 1, c0 + 2 * P, sg.n, CPR, gpr, gshift, wa, sa, ba);
            compute_pass_q4<LPR, 1, MT, SBT, kUnroll, XS>(c0 + P, CPR, xq, cx, wb, sb, bb, acc, xq_lo, p2);
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        acc[0][m] = group_sum<LPR>(acc[0][m]);
    }
    if (lane == 0) {
        const float bv = sg.bias ? sg.bias[v] : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) sg.y[(size_t)m * sg.n + v] = sg.bias ? acc[0][m] + bv : acc[0][m];
    }
}

// Persistent single-row (M = 1) variant for long outputs (lm_head): a block
// stages x once, then walks tiles tile, tile+grid, ... of ROWS rows.  The next
// tile's weights are loaded while the current one is computed (two register
// sets, loop unrolled by two), and each team's sums go to LDS; the block
// writes them out after its last tile, so the loop holds no global store and
// the compiler's in-order load counting stays exact.  A wave's teams own rows
// interleaved by team (row = base + r*TPW + team), so one load instruction
// covers TPW consecutive rows.  Requires CPR <= U*LPR (one pass per row).
template <int LPR, int R, int U, int SBT>
__global__ __launch_bounds__(kBlock) void qgemv_q4_persist_kernel(
    const u4_t* __restrict__ wq, const void* __restrict__ S, const void* __restrict__ B,
    const _Float16* __restrict__ x, float* __restrict__ y, int N, int K, int gshift, int ntiles)
{
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int TPW = 64 / LPR;
    constexpr int ROWS = (kBlock / LPR) * R;
    const int CPR = K >> 5;
    uint32_t* xq = lds;
    float2* cx = reinterpret_cast<float2*>(lds + (size_t)CPR * 16);
    float* yl = reinterpret_cast<float*>(lds + (size_t)CPR * 16 + (size_t)CPR * 2);  // [tiles of this block][ROWS]
    const int lane = threadIdx.x % LPR;
    const int rbase = (int)(threadIdx.x >> 6) * TPW * R + (int)((threadIdx.x & 63) / LPR);
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int total = K >> 3;
    const int grid = gridDim.x;

    u4_t xr[4];
    load_x_words<4>(x, 1, K, total, xr);
    u4_t wa[U][R], wb[U][R];
    uint32_t sa[U][R], ba[U][R], sb[U][R], bb[U][R];
    int t = blockIdx.x;
    load_pass_q4<LPR, R, SBT, U>(wq, S, B, t * ROWS + rbase, TPW, lane, N, CPR, gpr, gshift, wa, sa, ba);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = (int)threadIdx.x + j * kBlock;
        stage_word_q4(xr[j], idx, idx < total, xq, cx);
    }
    for (int base = 4 * kBlock; base < total; base += kBlock) {
        const int idx = base + (int)threadIdx.x;
        const u4_t raw = idx < total ? *reinterpret_cast<const u4_t*>(x + (size_t)idx * 8) : u4_t{0u, 0u, 0u, 0u};
        stage_word_q4(raw, idx, idx < total, xq, cx);
    }
    __syncthreads();

    // one tile: prefetch the next into (wn, sn, bn), compute (wc, sc, bc)
    int it = 0;
    auto tile_step = [&](u4_t(&wn)[U][R], uint32_t(&sn)[U][R], uint32_t(&bn)[U][R], const u4_t(&wc)[U][R],
                         const uint32_t(&sc)[U][R], const uint32_t(&bc)[U][R]) {
        const int tn = t + grid;
        // past the last tile: re-read tile 0 (cache resident), never used
        const int tl = tn < ntiles ? tn : 0;
        load_pass_q4<LPR, R, SBT, U>(wq, S, B, tl * ROWS + rbase, TPW, lane, N, CPR, gpr, gshift, wn, sn, bn);
        float acc[R][1];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][0] = 0.0f;
        compute_pass_q4<LPR, R, 1, SBT, U>(lane, CPR, xq, cx, wc, sc, bc, acc);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(acc[r][0]);
            if (lane == 0) yl[it * ROWS + rbase + r * TPW] = v;
        }
        ++it;
        t = tn;
        return t < ntiles;
    };
    for (;;) {
        if (!tile_step(wb, sb, bb, wa, sa, ba)) break;
        if (!tile_step(wa, sa, ba, wb, sb, bb)) break;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < it * ROWS; i += kBlock) {
        const int n = (blockIdx.x + (i / ROWS) * grid) * ROWS + (i % ROWS);
        if (n < N) y[n] = yl[i];
    }
}

// Batched-row variant for long single-row outputs (M = 1, N % 16 == 0, K <= 1024).
// A wave owns batches of 16 consecutive rows, b = wave, wave + waves, ...; a
// step is one row pair (lanes 0-31 row 2s, lanes 32-63 row 2s+1, lane = 16-byte
// chunk of the row, its x chunk held in registers).  Every lane keeps the 8
// steps of the next batch in flight (a register ring), and the batch's scale
// and bias rows, contiguous in S and B, arrive with one 16-byte load per array
// a batch ahead and are parked in LDS.  The 8 per-step partial sums of a lane
// are reduced across the row's 32 lanes with a halving butterfly (9 exchanges
// per 8 rows instead of 5 per row).  Row sums are parked in LDS until the last
// batch (a store inside the loop turns every weight-load wait into vmcnt(0)).
constexpr int kRingThreads = 512;
constexpr int kRingSteps = 8;

template <int SBT>
__global__ __launch_bounds__(kRingThreads) void qgemv_q4_ring_kernel(const u4_t* __restrict__ wq,
                                                                    const void* __restrict__ S,
                                                                    const void* __restrict__ Bz,
                                                                    const _Float16* __restrict__ x,
                                                                    float* __restrict__ y, int N, int K, int gshift,
                                                                    int nbmax)
{
    constexpr int P = kRingSteps;
    constexpr int SBB = SBT == DT_F32 ? 4 : 2;
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 5;
    uint32_t* xq = lds;
    float2* cx = reinterpret_cast<float2*>(lds + (size_t)CPR * 16);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // per wave: S rows at +0, B rows at +1024 (16 rows, <= 32 bytes each), 16-byte aligned; then the
    // parked row sums (16 per batch, nbmax batches)
    unsigned char* sbw = reinterpret_cast<unsigned char*>(lds) + ((CPR * 72 + 15) & ~15) + wave * (2048 + 64 * nbmax);
    float* park = reinterpret_cast<float*>(sbw + 2048);
    const int h = lane >> 5, c = lane & 31;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int sbrow = gpr * SBB;        // bytes of S (and of B) per row
    const int sbv = sbrow;              // 16-byte vectors per batch per array: 16 rows * sbrow / 16
    const int NB = N >> 4;
    const int gw = blockIdx.x * (kRingThreads / 64) + wave, GW = gridDim.x * (kRingThreads / 64);
    const int nb = gw < NB ? (NB - 1 - gw) / GW + 1 : 0;  // batches of this wave
    const int cc = min(c, CPR - 1);  // lanes past the row re-read its last chunk; x is zero there
    const int gi = (cc << 5) >> gshift;

    u4_t wr[P];
    auto load_w = [&](int bi, int s) {
        const int b = min(gw + GW * bi, NB - 1);  // past the end: a clamped re-read, never used
        wr[s] = __builtin_nontemporal_load(wq + (size_t)(16 * b + 2 * s + h) * CPR + cc);
    };
    u4_t sbr;
    auto load_sb = [&](int bi) {
        const int b = min(gw + GW * bi, NB - 1);
        const int v = lane < sbv ? lane : min(lane - sbv, sbv - 1);
        const unsigned char* base = reinterpret_cast<const unsigned char*>(lane < sbv ? S : Bz);
        sbr = *reinterpret_cast<const u4_t*>(base + (size_t)b * 16 * sbrow + (size_t)v * 16);
    };
    // loads first, then the x staging (its wait covers them; nothing is computed before both); the
    // scale/bias load first, in the loop's order (else its wait in the loop becomes a full drain)
    load_sb(0);
#pragma unroll
    for (int s = 0; s < P; ++s) load_w(0, s);
    for (int idx = threadIdx.x; idx < (K >> 3); idx += kRingThreads) {
        const u4_t raw = *reinterpret_cast<const u4_t*>(x + idx * 8);
        stage_word_q4(raw, idx, true, xq, cx);
    }
    __syncthreads();
    u4_t xa[4];
    float2 xc = make_float2(0.f, 0.f);
    {
        const u4_t* xp = reinterpret_cast<const u4_t*>(xq + cc * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[i] = c < CPR ? xp[i] : u4_t{0u, 0u, 0u, 0u};
        if (c < CPR) xc = cx[cc];
    }
    const uint32_t m0f = 0x000F000Fu, m1f = 0x00F000F0u, magic = 0x64006400u;
    for (int bi = 0; bi < nb; ++bi) {
        // this batch's scale/bias rows -> LDS (loaded a batch ago); next batch's load
        if (lane < 2 * sbv) *reinterpret_cast<u4_t*>(sbw + (lane < sbv ? lane * 16 : 1024 + (lane - sbv) * 16)) = sbr;
        load_sb(bi + 1);
        float v[P];
#pragma unroll
        for (int s = 0; s < P; ++s) {
            const u4_t w = wr[s];
            const int row = 2 * s + h;
            float sc, bb;
            if constexpr (SBT == DT_F32) {
                sc = *reinterpret_cast<const float*>(sbw + row * sbrow + gi * 4);
                bb = *reinterpret_cast<const float*>(sbw + 1024 + row * sbrow + gi * 4);
            } else {
                sc = raw_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(sbw + row * sbrow + gi * 2));
                bb = raw_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(sbw + 1024 + row * sbrow + gi * 2));
            }
            float d = -xc.x;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                d = dot2(and_or(w[e], m0f, magic), xa[e][0], d);
                d = dot2(and_or(w[e], m1f, magic), xa[e][1], d);
                const uint32_t t = w[e] >> 8;
                d = dot2(and_or(t, m0f, magic), xa[e][2], d);
                d = dot2(and_or(t, m1f, magic), xa[e][3], d);
            }
            v[s] = sc * d + bb * xc.y;
            load_w(bi + 1, s);
        }
        // halving butterfly over the 32 lanes of a row: 8 partials -> one row sum per lane
        const bool b16 = c & 16, b8 = c & 8, b4 = c & 4;
        float a4[4], a2[2], a1;
#pragma unroll
        for (int i = 0; i < 4; ++i) a4[i] = (b16 ? v[i + 4] : v[i]) + __shfl_xor(b16 ? v[i] : v[i + 4], 16, 32);
#pragma unroll
        for (int i = 0; i < 2; ++i) a2[i] = (b8 ? a4[i + 2] : a4[i]) + lane_xor<8>(b8 ? a4[i] : a4[i + 2], 32);
        a1 = (b4 ? a2[1] : a2[0]) + lane_xor<4>(b4 ? a2[0] : a2[1], 32);
        a1 += lane_xor<2>(a1, 32);
        a1 += lane_xor<1>(a1, 32);
        // the lane now holds step s = 4*b16 + 2*b8 + b4 of the batch
        const int s = (b16 ? 4 : 0) + (b8 ? 2 : 0) + (b4 ? 1 : 0);
        if ((c & 3) == 0) park[16 * bi + 2 * s + h] = a1;
    }
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < 16 * nb; i += 64) y[16 * (gw + GW * (i >> 4)) + (i & 15)] = park[i];
}

// Flat-batch variant for rows of 4J whole 16-byte chunks (K = 128 J, J = 4..8).
// A 16-row batch is 16 * 4J = 64 J chunks, contiguous in memory, so a wave
// reads it with J full-width loads (lane l of load j takes chunk 64 j + l of
// the batch): every load covers 1 KB of whole 128-byte lines and no lane
// idles, where the row-pair steps above leave 4 of 32 lanes idle at K = 896
// and split lines between two loads.  The chunk -> (row, k chunk) map is the
// same in every batch, so each lane keeps its J x chunks in registers.  The J
// per-chunk sums of a lane go to a per-wave LDS slot (row stride 4J + 1) and
// four lanes per row add up its 4J chunks.  D batches of loads are in flight.
// Row sums are parked in LDS and stored after the last batch: on gfx9 stores
// count in vmcnt with the loads, and a store inside the loop makes every wait
// for a weight load a full drain (vmcnt(0)) of the batches in flight.
constexpr int kFlatThreads = 512;
#ifndef CELLM_Q4_FLAT_DEPTH
#define CELLM_Q4_FLAT_DEPTH 1
#endif
constexpr int kFlatDepth = CELLM_Q4_FLAT_DEPTH;

__host__ __device__ constexpr int flat_wave_bytes(int J, int nbmax) { return 1024 + 16 * (4 * J + 1) * 4 + 64 * nbmax; }

template <int SBT, int J, int D>
__global__ __launch_bounds__(kFlatThreads) void qgemv_q4_flat_kernel(const u4_t* __restrict__ wq,
                                                                    const void* __restrict__ S,
                                                                    const void* __restrict__ Bz,
                                                                    const _Float16* __restrict__ x,
                                                                    float* __restrict__ y, int N, int gshift,
                                                                    int nbmax)
{
    constexpr int CPR = 4 * J, K = 32 * CPR, RS = CPR + 1;
    constexpr int SBB = SBT == DT_F32 ? 4 : 2;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t* xq = lds;
    float2* cx = reinterpret_cast<float2*>(lds + CPR * 16);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // per wave: 16 S rows at +0, 16 B rows at +512 (<= 32 bytes each), chunk sums at +1024, then
    // the parked row sums (16 per batch, nbmax batches)
    unsigned char* sbw =
        reinterpret_cast<unsigned char*>(lds) + ((CPR * 72 + 15) & ~15) + wave * flat_wave_bytes(J, nbmax);
    float* red = reinterpret_cast<float*>(sbw + 1024);
    float* park = red + 16 * RS;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int sbrow = gpr * SBB;  // bytes of S (and of B) per row; 16 rows = sbrow 16-byte vectors
    const int NB = N >> 4;
    const int gw = blockIdx.x * (kFlatThreads / 64) + wave, GW = gridDim.x * (kFlatThreads / 64);
    const int nb = gw < NB ? (NB - 1 - gw) / GW + 1 : 0;

    u4_t wr[D][J];
    auto load_w = [&](int bi, int slot, int j) {
        const int b = min(gw + GW * bi, NB - 1);  // past the end: a clamped re-read, never used
        wr[slot][j] = __builtin_nontemporal_load(wq + (size_t)b * (64 * J) + 64 * j + lane);
    };
    u4_t sbr;
    auto load_sb = [&](int bi) {
        const int b = min(gw + GW * bi, NB - 1);
        const int v = lane < sbrow ? lane : min(lane - sbrow, sbrow - 1);
        const unsigned char* base = reinterpret_cast<const unsigned char*>(lane < sbrow ? S : Bz);
        sbr = *reinterpret_cast<const u4_t*>(base + (size_t)b * 16 * sbrow + (size_t)v * 16);
    };
    // loads first, then the x staging (its wait covers them; nothing is computed before both).  The
    // scale/bias load goes before the weights, in the order the loop issues them: were it the newest
    // load on the way into the loop, the compiler's wait for it would become a full vmcnt(0) drain.
    load_sb(0);
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int j = 0; j < J; ++j) load_w(d, d, j);
    for (int idx = threadIdx.x; idx < (K >> 3); idx += kFlatThreads) {
        const u4_t raw = *reinterpret_cast<const u4_t*>(x + idx * 8);
        stage_word_q4(raw, idx, true, xq, cx);
    }
    __syncthreads();
    u4_t xa[J][4];
    float2 xc[J];
    int soff[J], roff[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int f = 64 * j + lane, r = f / CPR, kc = f - r * CPR;
        const u4_t* xp = reinterpret_cast<const u4_t*>(xq + kc * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[j][i] = xp[i];
        xc[j] = cx[kc];
        soff[j] = r * sbrow + ((kc << 5) >> gshift) * SBB;
        roff[j] = r * RS + kc;
    }
    const uint32_t m0f = 0x000F000Fu, m1f = 0x00F000F0u, magic = 0x64006400u;
    const int rr = lane >> 2, q = lane & 3;
    // NEXT: issue the following batch's loads (every batch but a wave's last, so that no load is
    // left in flight past the loop: the stores after it reuse those registers and would wait for it)
    auto batch = [&](int bi, int slot, auto next) {
        constexpr bool NEXT = decltype(next)::value;
        // this batch's scale/bias rows -> LDS (loaded a batch ago); next batch's load.  Lanes past the
        // rows write the spare last 16 bytes of the S slot (free whenever such lanes exist): a store
        // under a branch made the compiler wait for every load in flight.
        *reinterpret_cast<u4_t*>(sbw + (lane < sbrow ? lane * 16 : (lane < 2 * sbrow ? 512 + (lane - sbrow) * 16 : 496))) =
            sbr;
        if constexpr (NEXT) load_sb(bi + 1);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < J; ++j) {
            // copy the chunk and reissue its ring slot before the arithmetic: the opaque copy lets
            // the next batch's load leave ahead of this chunk's dot instead of after it
            u4_t w = wr[slot][j];
            asm("" : "+v"(w));
            if constexpr (NEXT) load_w(bi + D, slot, j);
            float sc, bb;
            if constexpr (SBT == DT_F32) {
                sc = *reinterpret_cast<const float*>(sbw + soff[j]);
                bb = *reinterpret_cast<const float*>(sbw + 512 + soff[j]);
            } else {
                sc = raw_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(sbw + soff[j]));
                bb = raw_to_f32<SBT>(*reinterpret_cast<const uint16_t*>(sbw + 512 + soff[j]));
            }
            float d = -xc[j].x;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                d = dot2(and_or(w[e], m0f, magic), xa[j][e][0], d);
                d = dot2(and_or(w[e], m1f, magic), xa[j][e][1], d);
                const uint32_t t = w[e] >> 8;
                d = dot2(and_or(t, m0f, magic), xa[j][e][2], d);
                d = dot2(and_or(t, m1f, magic), xa[j][e][3], d);
            }
            red[roff[j]] = sc * d + bb * xc[j].y;
        }
        // LDS operations of a wave complete in order: the reads below see every lane's writes
        __builtin_amdgcn_wave_barrier();
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < J; ++t) s += red[rr * RS + q + 4 * t];
        s += lane_xor<1>(s, 64);
        s += lane_xor<2>(s, 64);
        if (q == 0) park[16 * bi + rr] = s;
        __builtin_amdgcn_wave_barrier();
    };
    static_assert(D == 1 || D == 2, "one or two batches in flight");
    using with_next = std::integral_constant<bool, true>;
    if constexpr (D == 1) {
        for (int bi = 0; bi + 1 < nb; ++bi) batch(bi, 0, with_next{});
        if (nb > 0) batch(nb - 1, 0, std::integral_constant<bool, false>{});
    } else {
        for (int bi = 0; bi < nb; bi += D) {
            batch(bi, 0, with_next{});
            if (bi + 1 < nb) batch(bi + 1, 1, with_next{});
        }
    }
    for (int i = lane; i < 16 * nb; i += 64) y[16 * (gw + GW * (i >> 4)) + (i & 15)] = park[i];
}

// ---------------------------------------------------------------------------
// int8 per-row scale
// ---------------------------------------------------------------------------

// f16 activations, 8 elements per unit: pairs (x0,x2),(x1,x3),(x4,x6),(x5,x7);
// xq [MT][CPR][8] uint32, cx [MT][CPR] = 1152*sum(x) over the 16-element chunk
// (two units in adjacent lanes).
__device__ __forceinline__ void stage_unit_i8(u4_t raw, int idx, bool valid, uint32_t* xq, float* cx)
{
    h8_t v = __builtin_bit_cast(h8_t, raw);
    h2_t p0 = {v[0], v[2]}, p1 = {v[1], v[3]}, p2 = {v[4], v[6]}, p3 = {v[5], v[7]};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += (float)v[i];
    if (valid) *reinterpret_cast<u4_t*>(xq + (size_t)idx * 4) = u4_t{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
    s = pair_sum(s);
    if (valid && (idx & 1) == 0) cx[idx >> 1] = 1152.0f * s;
}

// Same pass with one row pointer per team row (rows of different matrices).
template <int LPR, int R>
__device__ __forceinline__ void load_pass_i8_rows(const u4_t* const (&rp)[R], int c0, int CPR,
                                                  u4_t (&wv)[kUnroll][R])
{
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int c = min(c0 + u * LPR, CPR - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) wv[u][r] = __builtin_nontemporal_load(rp[r] + c);
    }
}

template <int LPR, int R>
__device__ __forceinline__ void load_pass_i8(const u4_t* __restrict__ w8, int row0, int c0, int N, int CPR,
                                             u4_t (&wv)[kUnroll][R])
{
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int c = min(c0 + u * LPR, CPR - 1);  // clamped, branch-free (see load_pass_q4)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(row0 + r, N - 1);
            wv[u][r] = __builtin_nontemporal_load(w8 + (size_t)n * CPR + c);
        }
    }
}

template <int LPR, int R, int MT>
__device__ __forceinline__ void compute_pass_i8_f16x(int c0, int CPR, const uint32_t* xq, const float* cx,
                                                     const u4_t (&wv)[kUnroll][R], float (&acc)[R][MT])
{
    const uint32_t mlo = 0x00FF00FFu, magic = 0x64006400u;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int c = c0 + u * LPR;
        if (c < CPR) {
            uint32_t lo[R][4], hi[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t b = wv[u][r][t] ^ 0x80808080u;
                    lo[r][t] = and_or(b, mlo, magic);
                    hi[r][t] = and_or(b >> 8, mlo, magic);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const u4_t* xp = reinterpret_cast<const u4_t*>(xq + ((size_t)m * CPR + c) * 8);
                const u4_t xa = xp[0], xb = xp[1];
                const float corr = cx[(size_t)m * CPR + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float d = acc[r][m] - corr;
                    d = dot2(lo[r][0], xa[0], d);
                    d = dot2(hi[r][0], xa[1], d);
                    d = dot2(lo[r][1], xa[2], d);
                    d = dot2(hi[r][1], xa[3], d);
                    d = dot2(lo[r][2], xb[0], d);
                    d = dot2(hi[r][2], xb[1], d);
                    d = dot2(lo[r][3], xb[2], d);
                    d = dot2(hi[r][3], xb[3], d);
                    acc[r][m] = d;
                }
            }
        }
    }
}

// f32 x in LDS: 4 floats of padding after every 16 (K % 16 == 0, so each row starts padded too).  A
// lane's 16-float chunk then starts 80 bytes after its neighbour's, and the 16-byte reads of 8
// lanes fall on 32 distinct banks (unpadded, 64 bytes apart, they met 4-way conflicts).
__host__ __device__ constexpr int i8_xpad(int e) { return e + (e >> 4) * 4; }

template <int LPR, int R, int MT>
__device__ __forceinline__ void compute_pass_i8_f32x(int c0, int CPR, int K, const float* xs,
                                                     const u4_t (&wv)[kUnroll][R], float (&acc)[R][MT])
{
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int c = c0 + u * LPR;
        if (c < CPR) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const f4_t* xp = reinterpret_cast<const f4_t*>(xs + i8_xpad(m * K + c * 16));
                const f4_t x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
                const float xv[16] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3],
                                      x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]};
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float d = acc[r][m];
#pragma unroll
                    for (int t = 0; t < 4; ++t)
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            d = __builtin_fmaf((float)(int8_t)(wv[u][r][t] >> (8 * b)), xv[t * 4 + b], d);
                    acc[r][m] = d;
                }
            }
        }
    }
}

// int8 kernels' activation staging.  i8_load_x issues this thread's first
// XW activation words (clamped, branch-free); i8_stage_x stores them (and any
// further words of a large M*K) into LDS: f16 x as the dot2 pairs plus the
// 1152*sum(x) offsets (stage_unit_i8), f32 x as is.
template <int MT, int XT, int XW>
__device__ __forceinline__ void i8_load_x(const void* __restrict__ xv, int M, int K, u4_t (&xr)[XW])
{
    const int unit = XT == DT_F16 ? 8 : 4;
    const int units = K / unit;
    const int total = MT * units;
#pragma unroll
    for (int j = 0; j < XW; ++j) {
        // x rows are contiguous: unit idx sits at element unit * idx (no division; padding rows read
        // the last real unit, and their results are never stored)
        const int idx = min((int)threadIdx.x + j * kBlock, min(total, M * units) - 1);
        const char* base = reinterpret_cast<const char*>(xv) + (size_t)idx * unit * (XT == DT_F16 ? 2 : 4);
        xr[j] = *reinterpret_cast<const u4_t*>(base);
    }
}

template <int MT, int XT, int XW>
__device__ __forceinline__ void i8_stage_x(const u4_t (&xr)[XW], const void* __restrict__ xv, int M, int K,
                                           uint32_t* lds)
{
    const int CPR = K >> 4;
    const int unit = XT == DT_F16 ? 8 : 4;
    const int units = K / unit;
    const int total = MT * units;
    uint32_t* xq = lds;
    if constexpr (XT == DT_F16) {
        float* cx = reinterpret_cast<float*>(lds + (size_t)MT * CPR * 8);
#pragma unroll
        for (int j = 0; j < XW; ++j) {
            const int idx = (int)threadIdx.x + j * kBlock;
            stage_unit_i8(xr[j], idx, idx < total, xq, cx);
        }
        for (int b0 = XW * kBlock; b0 < total; b0 += kBlock) {
            const int idx = b0 + (int)threadIdx.x;
            const _Float16* xh = reinterpret_cast<const _Float16*>(xv);
            u4_t raw = (idx < total && idx < M * units) ? *reinterpret_cast<const u4_t*>(xh + (size_t)idx * 8)
                                                        : u4_t{0u, 0u, 0u, 0u};
            stage_unit_i8(raw, idx, idx < total, xq, cx);
        }
    } else {
        // f32 x: element e of the [MT][K] rows at e + 4 (e / 16) (i8_xpad)
#pragma unroll
        for (int j = 0; j < XW; ++j) {
            const int idx = (int)threadIdx.x + j * kBlock;
            if (idx < total) *reinterpret_cast<u4_t*>(xq + i8_xpad(idx * 4)) = xr[j];
        }
        for (int b0 = XW * kBlock; b0 < total; b0 += kBlock) {
            const int idx = b0 + (int)threadIdx.x;
            const float* xf = reinterpret_cast<const float*>(xv);
            if (idx < total)
                *reinterpret_cast<u4_t*>(xq + i8_xpad(idx * 4)) =
                    idx < M * units ? *reinterpret_cast<const u4_t*>(xf + (size_t)idx * 4) : u4_t{0u, 0u, 0u, 0u};
        }
    }
}

// XT: DT_F16 (dot2 path) or DT_F32 (exact int8->f32 conversion + f32 FMA).  BX: 12 x words per
// thread instead of 8 in the first staging round (4 rows of f32 x over K up to 3072 in one round).
template <int LPR, int R, int MT, int XT, bool MP, bool BX = false>
__global__ __launch_bounds__(kBlock) void qgemv_i8_kernel(
    const u4_t* __restrict__ w8, const void* __restrict__ S, int sdt, int per_channel,
    const void* __restrict__ xv, const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K)
{
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 4;
    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * (kBlock / LPR) + team) * R;

    // (1) activations: f16 in 8-element units, f32 in 4-element units
    constexpr int XW = MT == 1 ? 4 : (BX ? 12 : 8);
    u4_t xr[XW];
    i8_load_x<MT, XT, XW>(xv, M, K, xr);
    // (2) weights for the first pass and this team's per-row scale / bias
    u4_t wa[kUnroll][R];
    load_pass_i8<LPR, R>(w8, row0, lane, N, CPR, wa);
    uint32_t sraw[R];
    float bv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(row0 + r, N - 1);
        const size_t si = per_channel ? (size_t)n : 0;
        sraw[r] = sdt == DT_F32 ? load_raw<DT_F32>(S, si) : load_raw<DT_F16>(S, si);
        bv[r] = bias ? bias[n] : 0.0f;
    }
    // (3) stage activations
    i8_stage_x<MT, XT, XW>(xr, xv, M, K, lds);
    __syncthreads();
    if (row0 >= N) return;

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    auto compute = [&](int c0, const u4_t(&wv)[kUnroll][R]) {
        if constexpr (XT == DT_F16)
            compute_pass_i8_f16x<LPR, R, MT>(c0, CPR, lds, reinterpret_cast<const float*>(lds + (size_t)MT * CPR * 8),
                                             wv, acc);
        else
            compute_pass_i8_f32x<LPR, R, MT>(c0, CPR, K, reinterpret_cast<const float*>(lds), wv, acc);
    };
    if constexpr (!MP) {
        compute(lane, wa);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][R];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR) load_pass_i8<LPR, R>(w8, row0, c0 + P, N, CPR, wb);
            compute(c0, wa);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR) load_pass_i8<LPR, R>(w8, row0, c0 + 2 * P, N, CPR, wa);
            compute(c0 + P, wb);
        }
    }

    // the team's R * MT sums reduced transposed: lane l ends with value team_sum_t_index(l), and
    // one lane per value applies the row's scale (and bias) and stores
    static_assert(R * MT <= LPR, "one value per lane at most");
    constexpr int V = R * MT;
    float a[V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) a[r * MT + m] = acc[r][m];
    const float tot = team_sum_t<LPR, V>(a);
    const int vi = team_sum_t_index<LPR, V>(lane), r = vi / MT, m = vi % MT, n = row0 + r;
    if ((lane & (LPR / V - 1)) == 0 && m < M && n < N) {
        uint32_t sr = sraw[0];
        float bvr = bv[0];
#pragma unroll
        for (int k = 1; k < R; ++k) {
            sr = r == k ? sraw[k] : sr;
            bvr = r == k ? bv[k] : bvr;
        }
        const float s = sdt == DT_F32 ? raw_to_f32<DT_F32>(sr)
                      : sdt == DT_F16 ? raw_to_f32<DT_F16>(sr)
                                      : raw_to_f32<DT_BF16>(sr);
        float v = tot * s;
        if (bias) v += bvr;
        y[(size_t)m * N + n] = v;
    }
}

// ---------------------------------------------------------------------------
// Symmetric i4: y[m,n] = sum_k (nib[n,k] - 8) * s[n, k / gs] * x[m,k]
// (cpu_kernels.rs:219-243 matmul_i4_f32, gemma.rs:1446-1471 with gs = in_dim).
// A row is K/2 bytes, element 2b in the low nibble of byte b and 2b+1 in the
// high one, so a little-endian u32 holds elements 0..7 in nibble order.  A
// 16-byte chunk is 32 elements and chunks go to team lanes as in the int8
// kernel.  x is staged in LDS as f32 (f16 x widened exactly) together with
// 8 * sum(x) per chunk.  A chunk's dot is sum(nib * x) - 8 * sum(x): the
// 0x0F0F0F0F-masked word and its 4-bit shift give the nibbles as bytes, and
// v_cvt_f32_ubyteN turns each into f32 (3 ops per 8 nibbles); nib * x is exact
// and every sum is f32, so the difference from the reference is its summation
// order.  One scale per row (gs >= K) scales the row sum once; smaller groups
// (gs % 32 == 0) scale each chunk sum by its group's scale.
// ---------------------------------------------------------------------------

// x words of i8_load_x -> LDS: xs [MT][K] f32, cx [MT][K/32] = 8 * sum over the chunk.
// Units past the first XW per thread are moved in rounds of XW: all loads of a
// round are issued before any is stored, so a round costs one L2 round trip.
template <int MT, int XT, int XW>
__device__ __forceinline__ void i4_stage_x(const u4_t (&xr)[XW], const void* __restrict__ xv, int M, int K,
                                           float* xs, float* cx)
{
    constexpr int unit = XT == DT_F16 ? 8 : 4;
    constexpr int upc = 32 / unit;  // units per chunk, in adjacent lanes
    const int units = K / unit;
    const int total = MT * units;
    auto put = [&](const u4_t raw, int idx) {
        const bool valid = idx < total;
        float s = 0.0f;
        if constexpr (XT == DT_F16) {
            const h8_t v = __builtin_bit_cast(h8_t, raw);
            const f4_t a = {(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
            const f4_t b = {(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
            s = ((a[0] + a[1]) + (a[2] + a[3])) + ((b[0] + b[1]) + (b[2] + b[3]));
            if (valid) {
                *reinterpret_cast<f4_t*>(xs + (size_t)idx * 8) = a;
                *reinterpret_cast<f4_t*>(xs + (size_t)idx * 8 + 4) = b;
            }
        } else {
            const f4_t a = __builtin_bit_cast(f4_t, raw);
            s = (a[0] + a[1]) + (a[2] + a[3]);
            if (valid) *reinterpret_cast<f4_t*>(xs + (size_t)idx * 4) = a;
        }
        if constexpr (upc == 8)
            s = oct_sum(s);
        else
            s = quad_sum(s);
        if (valid && idx % upc == 0) cx[idx / upc] = 8.0f * s;
    };
#pragma unroll
    for (int j = 0; j < XW; ++j) put(xr[j], (int)threadIdx.x + j * kBlock);
    for (int b0 = XW * kBlock; b0 < total; b0 += XW * kBlock) {
        u4_t rr[XW];
#pragma unroll
        for (int j = 0; j < XW; ++j) {
            // contiguous rows: unit ic at element unit * ic (padding rows read the last real unit)
            const int ic = min(b0 + j * kBlock + (int)threadIdx.x, min(total, M * units) - 1);
            const char* base = reinterpret_cast<const char*>(xv) + (size_t)ic * unit * (XT == DT_F16 ? 2 : 4);
            rr[j] = *reinterpret_cast<const u4_t*>(base);
        }
#pragma unroll
        for (int j = 0; j < XW; ++j) put(rr[j], b0 + j * kBlock + (int)threadIdx.x);
    }
}

// sum over one chunk of nib * x (32 elements, x at xp)
__device__ __forceinline__ float i4_chunk_dot(const u4_t w, const float* xp, float d)
{
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const f4_t xa = *reinterpret_cast<const f4_t*>(xp + 8 * t);
        const f4_t xb = *reinterpret_cast<const f4_t*>(xp + 8 * t + 4);
        const uint32_t lo = w[t] & 0x0F0F0F0Fu, hi = (w[t] >> 4) & 0x0F0F0F0Fu;
        d = __builtin_fmaf(cvt_ubyte<0>(lo), xa[0], d);
        d = __builtin_fmaf(cvt_ubyte<0>(hi), xa[1], d);
        d = __builtin_fmaf(cvt_ubyte<1>(lo), xa[2], d);
        d = __builtin_fmaf(cvt_ubyte<1>(hi), xa[3], d);
        d = __builtin_fmaf(cvt_ubyte<2>(lo), xb[0], d);
        d = __builtin_fmaf(cvt_ubyte<2>(hi), xb[1], d);
        d = __builtin_fmaf(cvt_ubyte<3>(lo), xb[2], d);
        d = __builtin_fmaf(cvt_ubyte<3>(hi), xb[3], d);
    }
    return d;
}

// cpg = 0: one scale per row (the row's first); else chunk c is scaled by S[n * spr + c / cpg],
// cpg = gs / 32 chunks per group.
template <int LPR, int R, int MT, int XT, bool MP>
__global__ __launch_bounds__(kBlock) void qgemv_i4_kernel(const u4_t* __restrict__ w4, const uint16_t* __restrict__ S,
                                                          int spr, int cpg, const void* __restrict__ xv,
                                                          float* __restrict__ y, int M, int N, int K)
{
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 5;
    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * (kBlock / LPR) + team) * R;
    float* xs = reinterpret_cast<float*>(lds);
    float* cx = xs + (size_t)MT * K;

    constexpr int XW = MT == 1 ? 4 : 8;
    u4_t xr[XW];
    i8_load_x<MT, XT, XW>(xv, M, K, xr);
    u4_t wa[kUnroll][R];
    load_pass_i8<LPR, R>(w4, row0, lane, N, CPR, wa);
    const uint16_t* rs[R];
    uint32_t s0[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rs[r] = S + (size_t)min(row0 + r, N - 1) * spr;
        s0[r] = load_raw<DT_F16>(rs[r], 0);
    }
    i4_stage_x<MT, XT, XW>(xr, xv, M, K, xs, cx);
    __syncthreads();
    if (row0 >= N) return;

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
    auto compute = [&](int c0, const u4_t(&wv)[kUnroll][R]) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * LPR;
            if (c < CPR) {
                if (cpg == 0) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const float* xp = xs + (size_t)m * K + (size_t)c * 32;
                        const float corr = cx[(size_t)m * CPR + c];
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[r][m] = i4_chunk_dot(wv[u][r], xp, acc[r][m] - corr);
                    }
                } else {
                    float sg[R];
#pragma unroll
                    for (int r = 0; r < R; ++r) sg[r] = raw_to_f32<DT_F16>(load_raw<DT_F16>(rs[r], (size_t)(c / cpg)));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const float* xp = xs + (size_t)m * K + (size_t)c * 32;
                        const float corr = cx[(size_t)m * CPR + c];
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[r][m] = __builtin_fmaf(sg[r], i4_chunk_dot(wv[u][r], xp, -corr), acc[r][m]);
                    }
                }
            }
        }
    };
    if constexpr (!MP) {
        compute(lane, wa);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][R];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR) load_pass_i8<LPR, R>(w4, row0, c0 + P, N, CPR, wb);
            compute(c0, wa);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR) load_pass_i8<LPR, R>(w4, row0, c0 + 2 * P, N, CPR, wa);
            compute(c0 + P, wb);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = group_sum<LPR>(acc[r][m]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = row0 + r;
            if (n < N) {
                const float sc = cpg == 0 ? raw_to_f32<DT_F16>(s0[r]) : 1.0f;
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m < M) y[(size_t)m * N + n] = acc[r][m] * sc;
            }
        }
    }
}

// Any shape, any gs: one wave per output row, one byte per lane and step.
template <int XT>
__global__ __launch_bounds__(kBlock) void qgemv_i4_generic_kernel(const uint8_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ S, int spr, int gs,
                                                                  const void* __restrict__ x, float* __restrict__ y,
                                                                  int M, int N, int K)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * (kBlock / 64) + wave;
    if (n >= N) return;
    const int row_stride = (K + 1) >> 1;
    const uint8_t* row = w + (size_t)n * row_stride;
    const uint16_t* rs = S + (size_t)n * spr;
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int bi = lane; bi < row_stride; bi += 64) {
            const uint32_t byte = row[bi];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = 2 * bi + h;
                if (j < K) {
                    const int q = (int)((byte >> (4 * h)) & 0xFu) - 8;
                    const float s = load_f32<DT_F16>(rs, (size_t)(j / gs));
                    acc = __builtin_fmaf((float)q * s, load_f32<XT>(x, (size_t)m * K + j), acc);
                }
            }
        }
        acc = group_sum<64>(acc);
        if (lane == 0) y[(size_t)m * N + n] = acc;
    }
}

// ---------------------------------------------------------------------------
// Fused multi-output int8 GEMV: up to three int8 matrices that share x in one
// launch (QKV, metal.rs:387-439 mv_qkv_i8), or gate and up with the SiLU * up
// epilogue (llama_graph.rs:320-327: mv_i8 x2 + silu_mul_f32_inplace,
// metal.rs:235-245).  Each team holds R = 2 rows:
//   * segments (SILU = false): consecutive rows of the concatenation
//     [seg0 rows; seg1 rows; seg2 rows], each row reading its own matrix,
//     scale, bias and output;
//   * SILU: row n of seg0 (gate) and row n of seg1 (up);
//     h[n] = act(g) * u with g, u the scaled (and biased) row results and
//     act silu(g) = g / (1 + exp(-g)) or the tanh GELU (act_mul, segs.act),
//     written to seg0's output.
// ---------------------------------------------------------------------------
using I8Seg = I8FusedSeg;

struct I8Segs {
    I8Seg g0, g1, g2;
    int act;  // gate/up epilogue (SILU = true): ACT_SILU or ACT_GELU_TANH
};

__device__ __forceinline__ I8Seg seg_of(const I8Segs& t, int i)
{
    I8Seg r = t.g0;
    if (i == 1) r = t.g1;
    if (i == 2) r = t.g2;
    return r;
}

template <int LPR, int MT, int XT, bool MP, bool SILU>
__global__ __launch_bounds__(kBlock) void qgemv_i8_fused_kernel(I8Segs segs, int sdt, const void* __restrict__ xv,
                                                                int M, int total_rows, int K)
{
    constexpr int R = 2;
    extern __shared__ __align__(16) uint32_t lds[];
    const int CPR = K >> 4;
    const int team = threadIdx.x / LPR;
    const int lane = threadIdx.x % LPR;
    // SILU: team -> one row index of both matrices; else two consecutive rows
    const int first = SILU ? blockIdx.x * (kBlock / LPR) + team : (blockIdx.x * (kBlock / LPR) + team) * R;

    constexpr int XW = MT == 1 ? 4 : 8;
    u4_t xr[XW];
    i8_load_x<MT, XT, XW>(xv, M, K, xr);

    // row -> (segment, local row); rows past the end repeat the last row and are not stored
    int segi[R], loc[R];
    const u4_t* rp[R];
    uint32_t sraw[R];
    float bv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if constexpr (SILU) {
            segi[r] = r;
            loc[r] = min(first, total_rows - 1);
        } else {
            int v = min(first + r, total_rows - 1);
            int i = 0;
            if (v >= segs.g0.n) {
                v -= segs.g0.n;
                i = 1;
                if (v >= segs.g1.n) {
                    v -= segs.g1.n;
                    i = 2;
                }
            }
            segi[r] = i;
            loc[r] = v;
        }
        const I8Seg sg = seg_of(segs, segi[r]);
        rp[r] = reinterpret_cast<const u4_t*>(sg.w) + (size_t)loc[r] * CPR;
        const size_t si = sg.per_channel ? (size_t)loc[r] : 0;
        sraw[r] = sdt == DT_F32 ? load_raw<DT_F32>(sg.s, si) : load_raw<DT_F16>(sg.s, si);
        bv[r] = sg.bias ? sg.bias[loc[r]] : 0.0f;
    }
    u4_t wa[kUnroll][R];
    load_pass_i8_rows<LPR, R>(rp, lane, CPR, wa);
    i8_stage_x<MT, XT, XW>(xr, xv, M, K, lds);
    __syncthreads();
    if (first >= total_rows) return;

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
    auto compute = [&](int c0, const u4_t(&wv)[kUnroll][R]) {
        if constexpr (XT == DT_F16)
            compute_pass_i8_f16x<LPR, R, MT>(c0, CPR, lds, reinterpret_cast<const float*>(lds + (size_t)MT * CPR * 8),
                                             wv, acc);
        else
            compute_pass_i8_f32x<LPR, R, MT>(c0, CPR, K, reinterpret_cast<const float*>(lds), wv, acc);
    };
    if constexpr (!MP) {
        compute(lane, wa);
    } else {
        constexpr int P = kUnroll * LPR;
        u4_t wb[kUnroll][R];
        for (int c0 = lane; c0 < CPR + lane; c0 += 2 * P) {
            if (c0 - lane + P < CPR) load_pass_i8_rows<LPR, R>(rp, c0 + P, CPR, wb);
            compute(c0, wa);
            if (c0 - lane + P >= CPR) break;
            if (c0 - lane + 2 * P < CPR) load_pass_i8_rows<LPR, R>(rp, c0 + 2 * P, CPR, wa);
            compute(c0 + P, wb);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = group_sum<LPR>(acc[r][m]);
    if (lane != 0) return;

    float val[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float s = sdt == DT_F32 ? raw_to_f32<DT_F32>(sraw[r])
                      : sdt == DT_F16 ? raw_to_f32<DT_F16>(sraw[r])
                                      : raw_to_f32<DT_BF16>(sraw[r]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[r][m] * s;
            if (seg_of(segs, segi[r]).bias) v += bv[r];
            val[r][m] = v;
        }
    }
    if constexpr (SILU) {
        float* h = segs.g0.y;
        const int n = segs.g0.n;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < M) h[(size_t)m * n + first] = act_mul(segs.act, val[0][m], val[1][m]);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (first + r >= total_rows) continue;
            const I8Seg sg = seg_of(segs, segi[r]);
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m < M) sg.y[(size_t)m * sg.n + loc[r]] = val[r][m];
        }
    }
}

// ---------------------------------------------------------------------------
// Generic fallback: any K % 8 == 0, any activation dtype, one wave per row.
// Same element formulas as the reference, f32 arithmetic throughout.
// ---------------------------------------------------------------------------

template <int XT, int SBT>
__global__ __launch_bounds__(kBlock) void qgemv_q4_generic_kernel(
    const uint32_t* __restrict__ wq, const void* __restrict__ S, const void* __restrict__ B, const void* __restrict__ x,
    float* __restrict__ y, int M, int N, int K, int gshift)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * (kBlock / 64) + wave;
    if (n >= N) return;
    const int P = K >> 3;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int p = lane; p < P; p += 64) {
            const uint32_t w = wq[(size_t)n * P + p];
            const int g = (p << 3) >> gshift;
            const float s = load_f32<SBT>(S, (size_t)n * gpr + g);
            const float b = load_f32<SBT>(B, (size_t)n * gpr + g);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float wv = __fadd_rn(__fmul_rn((float)((w >> (4 * k)) & 0xFu), s), b);
                acc = __builtin_fmaf(wv, load_f32<XT>(x, (size_t)m * K + (size_t)p * 8 + k), acc);
            }
        }
        acc = group_sum<64>(acc);
        if (lane == 0) y[(size_t)m * N + n] = acc;
    }
}

template <int XT>
__global__ __launch_bounds__(kBlock) void qgemv_i8_generic_kernel(
    const int8_t* __restrict__ w, const void* __restrict__ S, int sdt, int per_channel, const void* __restrict__ x,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * (kBlock / 64) + wave;
    if (n >= N) return;
    const size_t si = per_channel ? (size_t)n : 0;
    const float s = sdt == DT_F32 ? load_f32<DT_F32>(S, si) : sdt == DT_F16 ? load_f32<DT_F16>(S, si)
                                                                            : load_f32<DT_BF16>(S, si);
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int k = lane; k < K; k += 64)
            acc = __builtin_fmaf((float)w[(size_t)n * K + k], load_f32<XT>(x, (size_t)m * K + k), acc);
        acc = group_sum<64>(acc);
        if (lane == 0) {
            float v = acc * s;
            if (bias) v += bias[n];
            y[(size_t)m * N + n] = v;
        }
    }
}

// Launch shape (lanes per row, rows per team).  Chosen from a sweep on
// MI355X (4-byte and 16-byte chunk rows, M=1):
//   * large N (>= 32768 rows): 8 lanes per row; weight streaming dominates and
//     narrow teams minimise reduction and staging cost per byte; rows longer
//     than one pass use the ping-pong multi-pass kernel;
//   * otherwise: the narrowest team whose row fits in one pass while keeping
//     >= 512 waves in flight, weighted by lane utilisation.
struct GemvShape {
    int lpr;
    int rows;
};

int gemv_device_cus()
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

GemvShape pick_shape(int cpr, int n_rows, bool q4)
{
    if (n_rows >= 32768) return {8, q4 && cpr <= 4 * 8 ? 2 : 1};
    const int cand[4] = {8, 16, 32, 64};
    int best = 64;
    double best_score = -1.0;
    for (int i = 0; i < 4; ++i) {
        const int lpr = cand[i];
        const int c = (cpr + lpr - 1) / lpr;
        if (c > kUnroll && lpr != 64) continue;
        const double eff = (double)cpr / ((double)lpr * c);
        const double waves = (double)n_rows * lpr / 64.0;
        const double fill = waves >= 512.0 ? 1.0 : waves / 512.0;
        const double score = eff * fill;
        if (score > best_score + 1e-9) {
            best_score = score;
            best = lpr;
        }
    }
    return {best, 1};
}

template <int LPR, int R, int MT, bool MP, bool XS>
hipError_t launch_q4_f16x_sbt(int sbt, const uint32_t* wq, const void* S, const void* B, const void* x, float* y,
                              int M, int N, int K, int gshift, hipStream_t st)
{
    const int CPR = K >> 5;
    const size_t lds = (size_t)(XS ? 2 : 1) * MT * CPR * 16 * 4 + (size_t)MT * CPR * (XS ? 12 : 8);
    const int rows_per_block = (kBlock / LPR) * R;
    const dim3 grid((N + rows_per_block - 1) / rows_per_block);
    const u4_t* w4 = reinterpret_cast<const u4_t*>(wq);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, w4, S, B, x, y, M, N, K, gshift);
        return hipGetLastError();
    };
    if (sbt == DT_F16) return go(qgemv_q4_f16x_kernel<LPR, R, MT, DT_F16, MP, XS>);
    if (sbt == DT_F32) return go(qgemv_q4_f16x_kernel<LPR, R, MT, DT_F32, MP, XS>);
    return go(qgemv_q4_f16x_kernel<LPR, R, MT, DT_BF16, MP, XS>);
}

template <int LPR, int R, int MT, bool XS>
hipError_t launch_q4_f16x_mp(int sbt, const uint32_t* wq, const void* S, const void* B, const void* x, float* y,
                             int M, int N, int K, int gshift, hipStream_t st)
{
    if ((K >> 5) > kUnroll * LPR)
        return launch_q4_f16x_sbt<LPR, R, MT, true, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
    return launch_q4_f16x_sbt<LPR, R, MT, false, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
}

template <int R, int MT, bool XS = false>
hipError_t launch_q4_f16x_lpr(int lpr, int sbt, const uint32_t* wq, const void* S, const void* B, const void* x,
                              float* y, int M, int N, int K, int gshift, hipStream_t st)
{
    switch (lpr) {
    case 8: return launch_q4_f16x_mp<8, R, MT, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
    case 16: return launch_q4_f16x_mp<16, R, MT, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
    case 32: return launch_q4_f16x_mp<32, R, MT, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
    default: return launch_q4_f16x_mp<64, R, MT, XS>(sbt, wq, S, B, x, y, M, N, K, gshift, st);
    }
}

template <int LPR, int R, int MT, int XT>
hipError_t launch_i8_xt(const int8_t* w, const void* S, int sdt, int per_channel, const void* x, const float* bias,
                        float* y, int M, int N, int K, hipStream_t st)
{
    const int CPR = K >> 4;
    const int rows_per_block = (kBlock / LPR) * R;
    const dim3 grid((N + rows_per_block - 1) / rows_per_block);
    const u4_t* w4 = reinterpret_cast<const u4_t*>(w);
    const size_t lds = XT == DT_F16 ? (size_t)MT * CPR * 8 * 4 + (size_t)MT * CPR * 4 : (size_t)i8_xpad(MT * K) * 4;
    auto go = [&](auto kern) {
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, w4, S, sdt, per_channel, x, bias, y, M, N, K);
        return hipGetLastError();
    };
    // 4 rows of f32 x past one round of 8 words per thread (K > 2048): 12 words, one round up to
    // K = 3072 (2560->960 at 4 rows 4.57 -> 4.32 us on MI355X; shorter rows run slower with 12,
    // the extra words being clamped re-reads)
    if constexpr (MT == 4 && XT == DT_F32) {
        if ((size_t)MT * (K / 4) > (size_t)kBlock * 8) {
            if (CPR > kUnroll * LPR) return go(qgemv_i8_kernel<LPR, R, MT, XT, true, true>);
            return go(qgemv_i8_kernel<LPR, R, MT, XT, false, true>);
        }
    }
    if (CPR > kUnroll * LPR) return go(qgemv_i8_kernel<LPR, R, MT, XT, true>);
    return go(qgemv_i8_kernel<LPR, R, MT, XT, false>);
}

template <int LPR, int R, int MT>
hipError_t launch_i8_lpr_fixed(int xdt, const int8_t* w, const void* S, int sdt, int per_channel, const void* x,
                               const float* bias, float* y, int M, int N, int K, hipStream_t st)
{
    if (xdt == DT_F16) return launch_i8_xt<LPR, R, MT, DT_F16>(w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    return launch_i8_xt<LPR, R, MT, DT_F32>(w, S, sdt, per_channel, x, bias, y, M, N, K, st);
}

template <int R, int MT>
hipError_t launch_i8_lpr(int lpr, int xdt, const int8_t* w, const void* S, int sdt, int per_channel, const void* x,
                         const float* bias, float* y, int M, int N, int K, hipStream_t st)
{
    switch (lpr) {
    case 8: return launch_i8_lpr_fixed<8, R, MT>(xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    case 16: return launch_i8_lpr_fixed<16, R, MT>(xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    case 32: return launch_i8_lpr_fixed<32, R, MT>(xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    default: return launch_i8_lpr_fixed<64, R, MT>(xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    }
}

template <int LPR, int MT, int XT, bool SILU>
hipError_t launch_i8_fused_lpr(const I8Segs& t, int total_rows, int sdt, const void* x, int M, int K, hipStream_t st)
{
    const int CPR = K >> 4;
    const int rows_per_block = (kBlock / LPR) * (SILU ? 1 : 2);
    const dim3 grid((total_rows + rows_per_block - 1) / rows_per_block);
    const size_t lds = XT == DT_F16 ? (size_t)MT * CPR * 8 * 4 + (size_t)MT * CPR * 4 : (size_t)i8_xpad(MT * K) * 4;
    if (CPR > kUnroll * LPR)
        hipLaunchKernelGGL((qgemv_i8_fused_kernel<LPR, MT, XT, true, SILU>), grid, dim3(kBlock), lds, st, t, sdt, x, M,
                           total_rows, K);
    else
        hipLaunchKernelGGL((qgemv_i8_fused_kernel<LPR, MT, XT, false, SILU>), grid, dim3(kBlock), lds, st, t, sdt, x,
                           M, total_rows, K);
    return hipGetLastError();
}

template <int MT, int XT, bool SILU>
hipError_t launch_i8_fused_mt(int lpr, const I8Segs& t, int total_rows, int sdt, const void* x, int M, int K,
                              hipStream_t st)
{
    switch (lpr) {
    case 8: return launch_i8_fused_lpr<8, MT, XT, SILU>(t, total_rows, sdt, x, M, K, st);
    case 16: return launch_i8_fused_lpr<16, MT, XT, SILU>(t, total_rows, sdt, x, M, K, st);
    case 32: return launch_i8_fused_lpr<32, MT, XT, SILU>(t, total_rows, sdt, x, M, K, st);
    default: return launch_i8_fused_lpr<64, MT, XT, SILU>(t, total_rows, sdt, x, M, K, st);
    }
}

template <int XT, bool SILU>
hipError_t launch_i8_fused_xt(int lpr, const I8Segs& t, int total_rows, int sdt, const void* x, int M, int K,
                              hipStream_t st)
{
    if (M == 1) return launch_i8_fused_mt<1, XT, SILU>(lpr, t, total_rows, sdt, x, M, K, st);
    if (M == 2) return launch_i8_fused_mt<2, XT, SILU>(lpr, t, total_rows, sdt, x, M, K, st);
    return launch_i8_fused_mt<4, XT, SILU>(lpr, t, total_rows, sdt, x, M, K, st);
}

template <int LPR, int MT, bool MP, bool XS>
hipError_t launch_q4_gu_shape(int sbt, const uint32_t* wg, const void* Sg, const void* Bg, const uint32_t* wu,
                              const void* Su, const void* Bu, const void* x, float* h, int M, int N, int K,
                              int gshift, int act, hipStream_t st)
{
    const dim3 grid((N + (kBlock / LPR) - 1) / (kBlock / LPR));
    const size_t lds = (size_t)qgemv_q4_lds_bytes(M, K) + (XS ? (size_t)MT * (K >> 5) * 68 : 0);
    const u4_t* g4 = reinterpret_cast<const u4_t*>(wg);
    const u4_t* u4 = reinterpret_cast<const u4_t*>(wu);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, g4, Sg, Bg, u4, Su, Bu, x, h, M, N, K, gshift, act);
        return hipGetLastError();
    };
    if (sbt == DT_F16) return go(qgemv_q4_gate_up_silu_kernel<LPR, MT, DT_F16, MP, XS>);
    if (sbt == DT_F32) return go(qgemv_q4_gate_up_silu_kernel<LPR, MT, DT_F32, MP, XS>);
    return go(qgemv_q4_gate_up_silu_kernel<LPR, MT, DT_BF16, MP, XS>);
}

template <int MT, bool XS>
hipError_t launch_q4_gu_mt(int sbt, const uint32_t* wg, const void* Sg, const void* Bg, const uint32_t* wu,
                           const void* Su, const void* Bu, const void* x, float* h, int M, int N, int K, int gshift,
                           int act, hipStream_t st)
{
    const int CPR = K >> 5;
    const int lpr = pick_shape(CPR, 2 * N, false).lpr;
#define CELLM_GU_L(L_)                                                                                               \
    return CPR > kUnroll * L_                                                                                      \
               ? launch_q4_gu_shape<L_, MT, true, XS>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st)  \
               : launch_q4_gu_shape<L_, MT, false, XS>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st)
    switch (lpr) {
    case 8: CELLM_GU_L(8);
    case 16: CELLM_GU_L(16);
    case 32: CELLM_GU_L(32);
    default: CELLM_GU_L(64);
    }
#undef CELLM_GU_L
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int LPR, int R, int MT, int XT>
hipError_t launch_i4_shape(const uint8_t* w, const uint16_t* S, int spr, int cpg, const void* x, float* y, int M, int N,
                           int K, hipStream_t st)
{
    const int CPR = K >> 5;
    const int rows_per_block = (kBlock / LPR) * R;
    const dim3 grid((N + rows_per_block - 1) / rows_per_block);
    const size_t lds = (size_t)MT * K * 4 + (size_t)MT * CPR * 4;
    const u4_t* w4 = reinterpret_cast<const u4_t*>(w);
    if (CPR > kUnroll * LPR) {
        auto kern = qgemv_i4_kernel<LPR, R, MT, XT, true>;
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, w4, S, spr, cpg, x, y, M, N, K);
    } else {
        auto kern = qgemv_i4_kernel<LPR, R, MT, XT, false>;
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, w4, S, spr, cpg, x, y, M, N, K);
    }
    return hipGetLastError();
}

// Team shapes (measured on the Gemma-3-1B MLP shapes): rows of up to 64
// chunks (K <= 2048) with enough of them take 16-lane teams of two rows, so
// each x read from LDS serves two rows (1152->6912: 4.5 us against 5.2 us for
// one row per team); longer rows at M = 4 take 64-lane teams of two rows
// (6912->1152: 14.0 us, against 19.4 us for 32-lane teams of one row and 16.8
// us for 64-lane teams of four), and pick_shape's single-row teams otherwise.
template <int MT, int XT>
hipError_t launch_i4_mt(const uint8_t* w, const uint16_t* S, int spr, int cpg, const void* x, float* y, int M, int N,
                        int K, hipStream_t st)
{
    const int CPR = K >> 5;
    if (CPR <= 64 && N >= 4096) return launch_i4_shape<16, 2, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    if (MT == 4 && CPR > 64) return launch_i4_shape<64, 2, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    const int lpr = pick_shape(CPR, N, false).lpr;
    switch (lpr) {
    case 8: return launch_i4_shape<8, 1, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    case 16: return launch_i4_shape<16, 1, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    case 32: return launch_i4_shape<32, 1, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    default: return launch_i4_shape<64, 1, MT, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    }
}

template <int XT>
hipError_t launch_i4_fast(const uint8_t* w, const uint16_t* S, int spr, int cpg, const void* x, float* y, int M,
                          int N, int K, hipStream_t st)
{
    if (M == 1) return launch_i4_mt<1, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    if (M == 2) return launch_i4_mt<2, XT>(w, S, spr, cpg, x, y, M, N, K, st);
    return launch_i4_mt<4, XT>(w, S, spr, cpg, x, y, M, N, K, st);
}


}  // namespace

int qgemv_q4_lds_bytes(int M, int K)
{
    const int MT = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    const int CPR = K >> 5;
    return MT * CPR * 16 * 4 + MT * CPR * 8;
}

static int persist_grid();

// Blocks for the 16-row-batch lm_head kernels: as many batches per wave as one block per CU needs,
// and only the waves that takes, so every wave gets the same count (the last round is not a
// partial one).  At 896->151936: 5 batches for 1900 waves, 238 blocks, measured 2 % faster than 256
// blocks with 4.6 batches per wave; more waves (2374 of 4 batches, 4748 of 2) were 6-10 % slower.
static int batch_grid(int NB, int waves_per_block)
{
    const int blocks = std::max(1, persist_grid() / 4), per = blocks * waves_per_block;
    const int bpw = (NB + per - 1) / per, waves = (NB + bpw - 1) / bpw;
    return std::max(1, (waves + waves_per_block - 1) / waves_per_block);
}

// The flat-batch kernel parks every row sum of a wave in LDS (64 bytes per batch).
static bool flat_lds_fits(int N, int K)
{
    const int GW = batch_grid(N >> 4, kFlatThreads / 64) * (kFlatThreads / 64), nbmax = ((N >> 4) + GW - 1) / GW;
    return (size_t)(((K >> 5) * 72 + 15) & ~15) + (size_t)(kFlatThreads / 64) * flat_wave_bytes(K >> 7, nbmax) <=
           64 * 1024;
}

// The ring kernel parks every row sum of a wave in LDS too.
static bool ring_lds_fits(int N, int K)
{
    const int GW = batch_grid(N >> 4, kRingThreads / 64) * (kRingThreads / 64), nbmax = ((N >> 4) + GW - 1) / GW;
    return (size_t)(((K >> 5) * 72 + 15) & ~15) + (size_t)(kRingThreads / 64) * (2048 + 64 * nbmax) <= 64 * 1024;
}

// Persistent grid: 4 blocks per CU (measured best for the lm_head shape).
static int persist_grid()
{
    // keyed by device, under a mutex: contexts on several threads and devices may launch at once
    static std::mutex mu;
    static std::vector<std::pair<int, int>> cached;  // (device, 4 * CUs)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const std::lock_guard<std::mutex> lk(mu);
    for (const auto& e : cached)
        if (e.first == dev) return e.second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    cached.emplace_back(dev, 4 * cus);
    return 4 * cus;
}

hipError_t launch_qgemv_q4_affine(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                  const void* x, int xdt, float* y, int M, int N, int K, hipStream_t st,
                                  int force_generic)
{
    const int gshift = __builtin_ctz((unsigned)group_size);
    const bool fast = !force_generic && xdt == DT_F16 && M <= 4 && (K % 32) == 0 && group_size >= 32 &&
                      aligned16(wq) && aligned16(x) && qgemv_q4_lds_bytes(M, K) <= 64 * 1024;
    const int sbrow = ((K + group_size - 1) / group_size) * (sbt == DT_F32 ? 4 : 2);
    if (fast && M == 1 && N >= 32768 && (N % 16) == 0 && (K % 128) == 0 && K >= 512 && K <= 1024 &&
        sbrow <= 32 && aligned16(S) && aligned16(B) && flat_lds_fits(N, K)) {
        // long single-row outputs, rows of 16..32 chunks in groups of 4: flat-batch kernel, one block per CU
        const int grid = batch_grid(N >> 4, kFlatThreads / 64);
        const int J = K >> 7;
        const int GW = grid * (kFlatThreads / 64), nbmax = ((N >> 4) + GW - 1) / GW;
        const size_t lds =
            (size_t)(((K >> 5) * 72 + 15) & ~15) + (size_t)(kFlatThreads / 64) * flat_wave_bytes(J, nbmax);
        const u4_t* w4 = reinterpret_cast<const u4_t*>(wq);
        const _Float16* xh = reinterpret_cast<const _Float16*>(x);
#define CELLM_Q4_FLAT(SBT_, J_)                                                                                   \
    hipLaunchKernelGGL((qgemv_q4_flat_kernel<SBT_, J_, kFlatDepth>), dim3(grid), dim3(kFlatThreads), lds, st, w4, S, \
                       B, xh, y, N, gshift, nbmax)
#define CELLM_Q4_FLAT_J(SBT_)                 \
    switch (J) {                              \
        case 4: CELLM_Q4_FLAT(SBT_, 4); break; \
        case 5: CELLM_Q4_FLAT(SBT_, 5); break; \
        case 6: CELLM_Q4_FLAT(SBT_, 6); break; \
        case 7: CELLM_Q4_FLAT(SBT_, 7); break; \
        default: CELLM_Q4_FLAT(SBT_, 8); break; \
    }
        if (sbt == DT_F16) {
            CELLM_Q4_FLAT_J(DT_F16)
        } else if (sbt == DT_F32) {
            CELLM_Q4_FLAT_J(DT_F32)
        } else {
            CELLM_Q4_FLAT_J(DT_BF16)
        }
#undef CELLM_Q4_FLAT_J
#undef CELLM_Q4_FLAT
        return hipGetLastError();
    }
    if (fast && M == 1 && N >= 32768 && (N % 16) == 0 && (K >> 5) <= 32 && sbrow <= 32 && aligned16(S) &&
        aligned16(B) && ring_lds_fits(N, K)) {
        // long single-row outputs, whole 16-row batches: batched-row ring kernel, one block per CU
        const int grid = batch_grid(N >> 4, kRingThreads / 64);
        const int GW = grid * (kRingThreads / 64), nbmax = ((N >> 4) + GW - 1) / GW;
        const size_t lds = (size_t)(((K >> 5) * 72 + 15) & ~15) + (size_t)(kRingThreads / 64) * (2048 + 64 * nbmax);
        const u4_t* w4 = reinterpret_cast<const u4_t*>(wq);
        const _Float16* xh = reinterpret_cast<const _Float16*>(x);
        if (sbt == DT_F16)
            hipLaunchKernelGGL((qgemv_q4_ring_kernel<DT_F16>), dim3(grid), dim3(kRingThreads), lds, st, w4, S, B, xh, y,
                               N, K, gshift, nbmax);
        else if (sbt == DT_F32)
            hipLaunchKernelGGL((qgemv_q4_ring_kernel<DT_F32>), dim3(grid), dim3(kRingThreads), lds, st, w4, S, B, xh, y,
                               N, K, gshift, nbmax);
        else
            hipLaunchKernelGGL((qgemv_q4_ring_kernel<DT_BF16>), dim3(grid), dim3(kRingThreads), lds, st, w4, S, B, xh,
                               y, N, K, gshift, nbmax);
        return hipGetLastError();
    }
    if (fast && M == 1 && N >= 32768 && (K >> 5) <= 32) {
        // long single-row outputs: persistent kernel, 32 lanes per row, 2 rows per team
        constexpr int LPR = 32, R = 2, ROWS = (kBlock / LPR) * R;
        const int ntiles = (N + ROWS - 1) / ROWS;
        const int grid = std::min(ntiles, persist_grid());
        const int tiles_per_block = (ntiles + grid - 1) / grid;
        const size_t lds = (size_t)qgemv_q4_lds_bytes(1, K) + (size_t)tiles_per_block * ROWS * 4;
        if (lds <= 64 * 1024) {
            const u4_t* w4 = reinterpret_cast<const u4_t*>(wq);
            const _Float16* xh = reinterpret_cast<const _Float16*>(x);
#define CELLM_Q4_PERSIST(SBT_)                                                                                   \
    hipLaunchKernelGGL((qgemv_q4_persist_kernel<LPR, R, 1, SBT_>), dim3(grid), dim3(kBlock), lds, st, w4, S, B, xh, y, \
                       N, K, gshift, ntiles)
            if (sbt == DT_F16) CELLM_Q4_PERSIST(DT_F16);
            else if (sbt == DT_F32) CELLM_Q4_PERSIST(DT_F32);
            else CELLM_Q4_PERSIST(DT_BF16);
#undef CELLM_Q4_PERSIST
            return hipGetLastError();
        }
    }
    if (fast) {
        const GemvShape sh = pick_shape(K >> 5, N, true);
        const _Float16* xh = reinterpret_cast<const _Float16*>(x);
        if (sh.rows == 2) {
            if (M == 1) return launch_q4_f16x_lpr<2, 1>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
            if (M == 2) return launch_q4_f16x_lpr<2, 2>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
            return launch_q4_f16x_lpr<2, 4>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
        }
        if (M == 1) return launch_q4_f16x_lpr<1, 1>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
        if (M == 2) return launch_q4_f16x_lpr<1, 2>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
        return launch_q4_f16x_lpr<1, 4>(sh.lpr, sbt, wq, S, B, xh, y, M, N, K, gshift, st);
    }
    // f32 x (the LFM runner's activations): the same team kernel over hi + lo f16 parts of x
    const int MT = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    const size_t lds32 = (size_t)2 * MT * (K >> 5) * 64 + (size_t)MT * (K >> 5) * 12;
    if (!force_generic && xdt == DT_F32 && M <= 4 && (K % 32) == 0 && group_size >= 32 && aligned16(wq) &&
        aligned16(x) && lds32 <= 160 * 1024) {
        const GemvShape sh = pick_shape(K >> 5, N, true);
        if (M == 1) return launch_q4_f16x_lpr<1, 1, true>(sh.lpr, sbt, wq, S, B, x, y, M, N, K, gshift, st);
        if (M == 2) return launch_q4_f16x_lpr<1, 2, true>(sh.lpr, sbt, wq, S, B, x, y, M, N, K, gshift, st);
        return launch_q4_f16x_lpr<1, 4, true>(sh.lpr, sbt, wq, S, B, x, y, M, N, K, gshift, st);
    }
    const dim3 grid((N + 3) / 4);
#define CELLM_Q4_GENERIC(XT_, SBT_)                                                                              \
    hipLaunchKernelGGL((qgemv_q4_generic_kernel<XT_, SBT_>), grid, dim3(kBlock), 0, st, wq, S, B, x, y, M, N, K, \
                       gshift)
    if (xdt == DT_F32) {
        if (sbt == DT_F32) CELLM_Q4_GENERIC(DT_F32, DT_F32);
        else if (sbt == DT_F16) CELLM_Q4_GENERIC(DT_F32, DT_F16);
        else CELLM_Q4_GENERIC(DT_F32, DT_BF16);
    } else if (xdt == DT_F16) {
        if (sbt == DT_F32) CELLM_Q4_GENERIC(DT_F16, DT_F32);
        else if (sbt == DT_F16) CELLM_Q4_GENERIC(DT_F16, DT_F16);
        else CELLM_Q4_GENERIC(DT_F16, DT_BF16);
    } else {
        if (sbt == DT_F32) CELLM_Q4_GENERIC(DT_BF16, DT_F32);
        else if (sbt == DT_F16) CELLM_Q4_GENERIC(DT_BF16, DT_F16);
        else CELLM_Q4_GENERIC(DT_BF16, DT_BF16);
    }
#undef CELLM_Q4_GENERIC
    return hipGetLastError();
}

hipError_t launch_qgemv_i8(const int8_t* w, const void* S, int sdt, int per_channel, const void* x, int xdt,
                           const float* bias, float* y, int M, int N, int K, hipStream_t st, int force_generic)
{
    const int MT = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    const size_t lds = xdt == DT_F16 ? (size_t)MT * (K >> 4) * 36 : (size_t)i8_xpad(MT * K) * 4;
    // x past 64 KB of LDS (f32 x of long rows at M > 1) takes the per-kernel limit raised to 160 KB
    const bool fast = !force_generic && (xdt == DT_F16 || xdt == DT_F32) && M <= 4 && (K % 16) == 0 &&
                      aligned16(w) && aligned16(x) && lds <= 160 * 1024;
    if (fast) {
        const GemvShape sh = pick_shape(K >> 4, N, false);
        if (M == 1) return launch_i8_lpr<1, 1>(sh.lpr, xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
        if (M == 2) return launch_i8_lpr<1, 2>(sh.lpr, xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
        // f32 x whose LDS leaves one block per CU (over 80 KB) and more four-row blocks than CUs:
        // two rows per team halve the blocks into one round (6912->1152 at 4 rows 18.4 -> 11.2 us
        // on MI355X; where two blocks fit a CU, two rows per team measured slower)
        if (xdt == DT_F32 && lds > 80 * 1024 && (N + 3) / 4 > gemv_device_cus())
            return launch_i8_lpr<2, 4>(sh.lpr, xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
        return launch_i8_lpr<1, 4>(sh.lpr, xdt, w, S, sdt, per_channel, x, bias, y, M, N, K, st);
    }
    const dim3 grid((N + 3) / 4);
    if (xdt == DT_F32)
        hipLaunchKernelGGL((qgemv_i8_generic_kernel<DT_F32>), grid, dim3(kBlock), 0, st, w, S, sdt, per_channel, x,
                           bias, y, M, N, K);
    else if (xdt == DT_F16)
        hipLaunchKernelGGL((qgemv_i8_generic_kernel<DT_F16>), grid, dim3(kBlock), 0, st, w, S, sdt, per_channel, x,
                           bias, y, M, N, K);
    else
        hipLaunchKernelGGL((qgemv_i8_generic_kernel<DT_BF16>), grid, dim3(kBlock), 0, st, w, S, sdt, per_channel, x,
                           bias, y, M, N, K);
    return hipGetLastError();
}

hipError_t launch_qgemv_i4_sym(const uint8_t* w, const uint16_t* S, int spr, int gs, const void* x, int xdt, float* y,
                               int M, int N, int K, hipStream_t st)
{
    const int MT = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    const size_t lds = (size_t)MT * K * 4 + (size_t)MT * (K >> 5) * 4;
    // one group per row when the row's last element still uses scale 0
    const bool per_row = K > 0 && (K - 1) / gs == 0;
    const bool fast = (xdt == DT_F16 || xdt == DT_F32) && M <= 4 && K > 0 && (K % 32) == 0 &&
                      (per_row || (gs % 32) == 0) && aligned16(w) && aligned16(x) && lds <= 160 * 1024;
    if (fast) {
        const int cpg = per_row ? 0 : gs / 32;
        if (xdt == DT_F16) return launch_i4_fast<DT_F16>(w, S, spr, cpg, x, y, M, N, K, st);
        return launch_i4_fast<DT_F32>(w, S, spr, cpg, x, y, M, N, K, st);
    }
    const dim3 grid((N + 3) / 4);
    if (xdt == DT_F32)
        hipLaunchKernelGGL((qgemv_i4_generic_kernel<DT_F32>), grid, dim3(kBlock), 0, st, w, S, spr, gs, x, y, M, N, K);
    else if (xdt == DT_F16)
        hipLaunchKernelGGL((qgemv_i4_generic_kernel<DT_F16>), grid, dim3(kBlock), 0, st, w, S, spr, gs, x, y, M, N, K);
    else
        hipLaunchKernelGGL((qgemv_i4_generic_kernel<DT_BF16>), grid, dim3(kBlock), 0, st, w, S, spr, gs, x, y, M, N,
                           K);
    return hipGetLastError();
}

bool qgemv_q4_gate_up_supported(int xdt, int M, int K, int group_size, const void* x, const void* wg, const void* wu)
{
    // f32 x (staged as hi + lo f16 parts) takes twice the x space, up to the raised 160 KB
    const bool f32x = xdt == DT_F32;
    return (xdt == DT_F16 || f32x) && M >= 1 && M <= 4 && K > 0 && (K % 32) == 0 && group_size >= 32 &&
           aligned16(x) && aligned16(wg) && aligned16(wu) &&
           (f32x ? (size_t)qgemv_q4_lds_bytes(M, K) + (size_t)(M <= 1 ? 1 : (M <= 2 ? 2 : 4)) * (K >> 5) * 68 <=
                       160 * 1024
                 : qgemv_q4_lds_bytes(M, K) <= 64 * 1024);
}

hipError_t launch_qgemv_q4_gate_up_silu(const uint32_t* wg, const void* Sg, const void* Bg, const uint32_t* wu,
                                        const void* Su, const void* Bu, int sbt, int group_size, const void* x,
                                        int xdt, float* h, int M, int N, int K, int act, hipStream_t st)
{
    const int gshift = __builtin_ctz((unsigned)group_size);
    if (xdt == DT_F32) {
        if (M == 1) return launch_q4_gu_mt<1, true>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
        if (M == 2) return launch_q4_gu_mt<2, true>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
        return launch_q4_gu_mt<4, true>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
    }
    if (M == 1) return launch_q4_gu_mt<1, false>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
    if (M == 2) return launch_q4_gu_mt<2, false>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
    return launch_q4_gu_mt<4, false>(sbt, wg, Sg, Bg, wu, Su, Bu, x, h, M, N, K, gshift, act, st);
}

bool qgemv_q4_segs_supported(int xdt, int M, int K, int group_size, const void* x, const Q4FusedSeg* segs, int nseg)
{
    if (!(xdt == DT_F16 || xdt == DT_F32) || M < 1 || M > 4 || K <= 0 || (K % 32) != 0 || group_size < 32 ||
        !aligned16(x))
        return false;
    const size_t lds = (size_t)qgemv_q4_lds_bytes(M, K) + (xdt == DT_F32 ? (size_t)(M <= 1 ? 1 : (M <= 2 ? 2 : 4)) * (K >> 5) * 68 : 0);
    if (lds > (xdt == DT_F32 ? 160 : 64) * 1024) return false;
    for (int i = 0; i < nseg; ++i)
        if (!aligned16(segs[i].w)) return false;
    return true;
}

namespace {

template <int LPR, int MT, bool MP, bool XS>
hipError_t launch_q4_segs_shape(const Q4Segs& t, int total_rows, int sbt, const void* x, int M, int K, int gshift,
                                hipStream_t st)
{
    const dim3 grid((total_rows + (kBlock / LPR) - 1) / (kBlock / LPR));
    const size_t lds = (size_t)qgemv_q4_lds_bytes(M, K) + (XS ? (size_t)MT * (K >> 5) * 68 : 0);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024)
            if (hipError_t e = allow_big_lds(kern, (int)lds); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, dim3(kBlock), lds, st, t, x, M, total_rows, K, gshift);
        return hipGetLastError();
    };
    if (sbt == DT_F16) return go(qgemv_q4_segs_kernel<LPR, MT, DT_F16, MP, XS>);
    if (sbt == DT_F32) return go(qgemv_q4_segs_kernel<LPR, MT, DT_F32, MP, XS>);
    return go(qgemv_q4_segs_kernel<LPR, MT, DT_BF16, MP, XS>);
}

template <int MT, bool XS>
hipError_t launch_q4_segs_mt(const Q4Segs& t, int total_rows, int sbt, const void* x, int M, int K, int gshift,
                             hipStream_t st)
{
    const int CPR = K >> 5;
    const int lpr = pick_shape(CPR, total_rows, true).lpr;
#define CELLM_SEGS_L(L_)                                                                                   \
    return CPR > kUnroll * L_ ? launch_q4_segs_shape<L_, MT, true, XS>(t, total_rows, sbt, x, M, K, gshift, st) \
                              : launch_q4_segs_shape<L_, MT, false, XS>(t, total_rows, sbt, x, M, K, gshift, st)
    switch (lpr) {
    case 8: CELLM_SEGS_L(8);
    case 16: CELLM_SEGS_L(16);
    case 32: CELLM_SEGS_L(32);
    default: CELLM_SEGS_L(64);
    }
#undef CELLM_SEGS_L
}

}  // namespace

hipError_t launch_qgemv_q4_segs(const Q4FusedSeg* segs, int nseg, int sbt, int group_size, const void* x, int xdt,
                                int M, int K, hipStream_t st)
{
    Q4Seg g[3] = {};
    int total = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg)
            g[i] = Q4Seg{reinterpret_cast<const u4_t*>(segs[i].w), segs[i].S, segs[i].B, segs[i].bias, segs[i].y,
                         segs[i].n};
        else
            g[i] = g[0], g[i].n = 0;
        total += g[i].n;
    }
    const Q4Segs t{g[0], g[1], g[2]};
    const int gshift = __builtin_ctz((unsigned)group_size);
    if (xdt == DT_F32) {
        if (M == 1) return launch_q4_segs_mt<1, true>(t, total, sbt, x, M, K, gshift, st);
        if (M == 2) return launch_q4_segs_mt<2, true>(t, total, sbt, x, M, K, gshift, st);
        return launch_q4_segs_mt<4, true>(t, total, sbt, x, M, K, gshift, st);
    }
    if (M == 1) return launch_q4_segs_mt<1, false>(t, total, sbt, x, M, K, gshift, st);
    if (M == 2) return launch_q4_segs_mt<2, false>(t, total, sbt, x, M, K, gshift, st);
    return launch_q4_segs_mt<4, false>(t, total, sbt, x, M, K, gshift, st);
}

bool qgemv_i8_fused_supported(int xdt, int M, int K, const void* x, const I8FusedSeg* segs, int nseg)
{
    if (!(xdt == DT_F16 || xdt == DT_F32) || M < 1 || M > 4 || K <= 0 || (K % 16) != 0 || !aligned16(x)) return false;
    const int MT = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    const size_t lds = xdt == DT_F16 ? (size_t)MT * (K >> 4) * 36 : (size_t)i8_xpad(MT * K) * 4;
    if (lds > 64 * 1024) return false;
    for (int i = 0; i < nseg; ++i)
        if (!aligned16(segs[i].w)) return false;
    return true;
}

hipError_t launch_qgemv_i8_fused(const I8FusedSeg* segs, int nseg, bool silu, int act, int sdt, const void* x, int xdt,
                                 int M, int K, hipStream_t st)
{
    I8Segs t;
    t.act = act;
    t.g0 = segs[0];
    t.g1 = nseg > 1 ? segs[1] : segs[0];
    t.g2 = nseg > 2 ? segs[2] : segs[0];
    if (nseg < 2) t.g1.n = 0;
    if (nseg < 3) t.g2.n = 0;
    const int total_rows = silu ? segs[0].n : t.g0.n + t.g1.n + t.g2.n;
    if (total_rows <= 0) return hipSuccess;
    const GemvShape sh = pick_shape(K >> 4, silu ? 2 * total_rows : total_rows, false);
    if (silu) {
        if (xdt == DT_F16) return launch_i8_fused_xt<DT_F16, true>(sh.lpr, t, total_rows, sdt, x, M, K, st);
        return launch_i8_fused_xt<DT_F32, true>(sh.lpr, t, total_rows, sdt, x, M, K, st);
    }
    if (xdt == DT_F16) return launch_i8_fused_xt<DT_F16, false>(sh.lpr, t, total_rows, sdt, x, M, K, st);
    return launch_i8_fused_xt<DT_F32, false>(sh.lpr, t, total_rows, sdt, x, M, K, st);
}

}  // namespace cellm
