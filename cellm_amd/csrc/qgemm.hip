// Quantized-weight GEMM on MFMA for prefill and batched decode (gfx950).
//
//   Y[M,N] = X[M,K] . dequant(W)[N,K]^T        (f16 X, f32 accumulate, f32 Y)
//
// Reference: there is no batched or GEMM path in cellm (prefill runs the GEMV
// token by token, crates/cellm-model/src/llama.rs:214-233).  The per-element
// oracle is cpu_kernels::matmul_f32 (cpu_kernels.rs:36-63) over the dequantized
// weight, summed over k ascending.
//
// Weights are dequantized to f16 with the converter's rounding,
// h = RNE_f16(f32(q)*s + b) (tools/convert/src/main.rs:4435-4436): into LDS
// tiles by qgemm_kernel, in registers right before each MFMA by the q4 kernel
// for K % 128 == 0.  For f16 or bf16 scales, f32(q)*s is exact in f32, so
// fma(q, s, b) rounds exactly as the reference's mul-then-add does; f32
// scales take a separate mul and add.
// int8 weights are exact in f16; their per-row scale is applied in the epilogue
// (y = acc * s, cpu_kernels.rs:130).
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; block tile 128x128, wave tile
// 64x64 = 4x4 v_mfma_f32_16x16x32_f16 tiles; BK = 64 per LDS stage.  The next
// stage's global data is prefetched into registers during the MFMA loop.
// Split-K over blockIdx.z writes f32 partials to a workspace that a second
// kernel sums in a fixed order (deterministic).
#include <mutex>
#include <utility>
#include <vector>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace cellm {

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // halves; 144-byte rows break LDS bank aliasing
constexpr int kThreads = 256;
constexpr int kStages = 4;  // register prefetch depth (K stages of 64 in flight)

template <int SBT>
__device__ __forceinline__ h8_t dequant_word_f16(uint32_t w, float s, float b)
{
    h8_t h;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float q = (float)((w >> (4 * k)) & 0xFu);
        float v;
        if constexpr (SBT == DT_F32) {
#pragma clang fp contract(off)
            const float t = q * s;
            v = t + b;
        } else {
            v = __builtin_fmaf(q, s, b);  // q*s exact: same bits as mul-then-add
        }
        // Keep the f32 rounding: without this barrier the compiler folds the
        // fma and the f16 narrowing into one v_fma_mix*_f16, which rounds once
        // instead of the reference's twice (f32, then f16).
        asm volatile("" : "+v"(v));
        h[k] = (_Float16)v;
    }
    return h;
}

__device__ __forceinline__ h8_t int8_to_f16x8(u2_t w)
{
    const uint32_t mlo = 0x00FF00FFu, magic = 0x64006400u;
    const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t b0 = w[0] ^ 0x80808080u, b1 = w[1] ^ 0x80808080u;
    // (1152+w0, 1152+w2), (1152+w1, 1152+w3): exact in f16; subtracting 1152 is exact
    h2_t a0 = as_h2(and_or(b0, mlo, magic)) - off;
    h2_t a1 = as_h2(and_or(b0 >> 8, mlo, magic)) - off;
    h2_t a2 = as_h2(and_or(b1, mlo, magic)) - off;
    h2_t a3 = as_h2(and_or(b1 >> 8, mlo, magic)) - off;
    h8_t h = {a0[0], a1[0], a0[1], a1[1], a2[0], a3[0], a2[1], a3[1]};
    return h;
}

// One K stage (BK = 64) of global data held in registers by one thread:
// its 32-element halves of one X row and one W row, plus the W row's scale
// and bias bits for that group (raw, converted when the tile is stored).
struct StageRegs {
    u4_t x[4];
    u4_t w0, w1;  // q4: w0 = 32 nibbles; int8: w0, w1 = 32 bytes
    uint32_t s, b;
};

// WT: 0 = q4 affine (u32 words), 1 = int8.  NS = register prefetch depth.
template <int WT, int SBT, int NS>
__global__ __launch_bounds__(kThreads) void qgemm_kernel(const void* __restrict__ W, const void* __restrict__ S,
                                                         const void* __restrict__ Bz, int group_size,
                                                         const _Float16* __restrict__ X, float* __restrict__ Y,
                                                         int M, int N, int K, int k_per_split, int per_channel)
{
    // two LDS buffers: stage s is stored into buffer s&1 while no wave can
    // still read it (every wave passed the barrier after its compute of s-2)
    __shared__ __align__(16) _Float16 xs[2][BM * LDS_STRIDE];
    __shared__ __align__(16) _Float16 ws[2][BN * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kbeg = blockIdx.z * k_per_split;
    const int kend = min(K, kbeg + k_per_split);
    const int nsteps = kend > kbeg ? (kend - kbeg) / BK : 0;  // K % 64 == 0, k_per_split % 64 == 0

    // global -> register assignment: thread = (row, 32-element half of the stage)
    const int ld_row = tid >> 1;
    const int ld_half = tid & 1;
    // Rows past M or N are clamped to the last valid row: their loads stay in
    // bounds without a branch and their results are never stored.
    const int xm = min(m0 + ld_row, M - 1), wn_row = min(n0 + ld_row, N - 1);
    const int gshift = __builtin_ctz((unsigned)group_size);
    const int gpr = (K + group_size - 1) >> gshift;
    const u4_t* w4 = reinterpret_cast<const u4_t*>(W);

    auto load_stage = [&](int step, StageRegs& r) {
        const int kc = kbeg + min(step, nsteps - 1) * BK + ld_half * 32;  // clamped: tail slots reload the last stage
#pragma unroll
        for (int i = 0; i < 4; ++i) r.x[i] = *reinterpret_cast<const u4_t*>(X + (size_t)xm * K + kc + i * 8);
        if constexpr (WT == 0) {
            r.w0 = __builtin_nontemporal_load(w4 + ((size_t)wn_row * K + kc) / 32);
            const size_t gi = (size_t)wn_row * gpr + (kc >> gshift);
            r.s = load_raw<SBT>(S, gi);
            r.b = load_raw<SBT>(Bz, gi);
        } else {
            r.w0 = __builtin_nontemporal_load(w4 + ((size_t)wn_row * K + kc) / 16);
            r.w1 = __builtin_nontemporal_load(w4 + ((size_t)wn_row * K + kc) / 16 + 1);
        }
    };

    auto store_stage = [&](const StageRegs& r, int buf) {
        _Float16* xd = xs[buf] + ld_row * LDS_STRIDE + ld_half * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u4_t*>(xd + i * 8) = r.x[i];
        _Float16* wd = ws[buf] + ld_row * LDS_STRIDE + ld_half * 32;
        if constexpr (WT == 0) {
            const float sc = raw_to_f32<SBT>(r.s), bi = raw_to_f32<SBT>(r.b);
#pragma unroll
            for (int i = 0; i < 4; ++i) *reinterpret_cast<h8_t*>(wd + i * 8) = dequant_word_f16<SBT>(r.w0[i], sc, bi);
        } else {
            *reinterpret_cast<h8_t*>(wd + 0) = int8_to_f16x8(u2_t{r.w0[0], r.w0[1]});
            *reinterpret_cast<h8_t*>(wd + 8) = int8_to_f16x8(u2_t{r.w0[2], r.w0[3]});
            *reinterpret_cast<h8_t*>(wd + 16) = int8_to_f16x8(u2_t{r.w1[0], r.w1[1]});
            *reinterpret_cast<h8_t*>(wd + 24) = int8_to_f16x8(u2_t{r.w1[2], r.w1[3]});
        }
    };

    f4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int frag_row = lane & 15;
    const int frag_k = (lane >> 4) * 8;
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            h8_t a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a[i] = *reinterpret_cast<const h8_t*>(xs[buf] + (wm * 64 + i * 16 + frag_row) * LDS_STRIDE + kk + frag_k);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                b[j] = *reinterpret_cast<const h8_t*>(ws[buf] + (wn * 64 + j * 16 + frag_row) * LDS_STRIDE + kk + frag_k);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    if (nsteps > 0) {
        // Software pipeline.  Stage s is in LDS buffer s&1 when step s starts;
        // step s dequantizes and stores stage s+1 into the other buffer while
        // its own MFMAs run (same basic block, so VALU issues in the MFMA
        // shadow), then one barrier, then the freed ring slot is refilled with
        // stage s+1+NS.  Buffer (s+1)&1 last held stage s-1, which every wave
        // finished reading before the barrier that ended step s-1.
        StageRegs ring[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) load_stage(j, ring[j]);
        store_stage(ring[0], 0);
        __syncthreads();
        load_stage(NS, ring[0]);
        for (int s0 = 0; s0 < nsteps; s0 += NS) {
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const int s = s0 + j;
                if (s < nsteps) {
                    // past the end this stores a clamped copy of the last stage
                    // into the idle buffer; nobody reads it
                    store_stage(ring[(j + 1) % NS], (s + 1) & 1);
                    compute(s & 1);
                }
                // The barrier and the reload run on every path (s is block-uniform and
                // the reload is clamped), so each unrolled step issues the same loads
                // and the compiler's vmcnt stays partial across the loop back edge.
                __syncthreads();
                load_stage(s + 1 + NS, ring[(j + 1) % NS]);
            }
        }
    }

    // C fragment: lane holds rows 4*(lane/16)+e, column lane%16 of each 16x16 tile.
    float* out = Y + (size_t)blockIdx.z * M * N;
    const int crow = (lane >> 4) * 4;
    const int ccol = lane & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + j * 16 + ccol;
        if (n >= N) continue;
        float s = 1.0f;
        if constexpr (WT == 1) s = load_f32<SBT>(S, per_channel ? (size_t)n : 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + wm * 64 + i * 16 + crow + e;
                if (m < M) out[(size_t)m * N + n] = acc[i][j][e] * s;
            }
        }
    }
}

// Sum split-K partials [splits][M*N] in split order, then add the optional bias.
__global__ void splitk_reduce_kernel(const float* __restrict__ part, float* __restrict__ y, const float* __restrict__ bias,
                                     int splits, int M, int N)
{
    const size_t total = (size_t)M * N;
    if ((N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
        // four columns of one row per thread: 16-byte loads of every split's partials
        const size_t n4 = total >> 2;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
            f4_t v = sum_splits_f4(reinterpret_cast<const f4_t*>(part) + i, n4, splits);
            if (bias) {
                const size_t n = (4 * i) % (size_t)N;
                v += f4_t{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]};
            }
            reinterpret_cast<f4_t*>(y)[i] = v;
        }
        return;
    }
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        float v = part[i];
        for (int s = 1; s < splits; ++s) v += part[(size_t)s * total + i];
        if (bias) v += bias[i % N];
        y[i] = v;
    }
}

__global__ void add_bias_kernel(float* __restrict__ y, const float* __restrict__ bias, int M, int N)
{
    const size_t total = (size_t)M * N;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x)
        y[i] += bias[i % N];
}


// ---------------------------------------------------------------------------
// Direct-to-LDS helpers for the q4 qGEMM below (K % 128 == 0): LDS tiles hold
// rows of 16 chunks of 8 halves, chunk position XOR-swizzled by (row & 15) so
// that the 16 rows a fragment read touches fall in 16 distinct 4-bank groups.
// The DMA loads are issued from inline asm with the LDS base in M0 and are
// waited for with explicit s_waitcnt counts: the compiler treats LDS DMA as
// aliasing every LDS read and would otherwise wait for all of them (including
// the stage just issued) before each fragment read.
// ---------------------------------------------------------------------------
namespace dma {

constexpr int BK = 128;
constexpr int kStageHalves = BM * BK;       // one f16 X or W tile
constexpr size_t kMaxLds = 160 * 1024;

__device__ __forceinline__ int slot(int r, int c) { return r * 16 + (c ^ (r & 15)); }

__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// 16 bytes per lane, global -> LDS; lane i lands at lds + 16 i (checked on gfx950)
__device__ __forceinline__ void dma16(const void* g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}

// Same with a uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset: a loop that only changes
// the base never rewrites the VGPR operand (the compiler's wait pass treats an asm's VGPR operands as
// pending after it, and rewriting them cost a vmcnt(0) drain per iteration).
__device__ __forceinline__ void dma16_s(uint32_t voff, const void* sbase, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---------------------------------------------------------------------------
// q4 affine qGEMM, dequant at the MFMA (K % 128 == 0).
//
// 512 threads = 8 waves, two per SIMD; block tile 128 (M) x 128 (N).  Wave
// (kh, ns) owns a 128 x 32 tile (four v_mfma_f32_32x32x16_f16 accumulators)
// over k half kh of every 128-wide k-step; the two halves are added through
// LDS after the loop.  X (f16) and the raw nibbles of W go global -> LDS by
// global_load_lds_dwordx4 through a ring of three stages (stage = one k-step:
// X 128 x 128 halves, swizzled as above, and W 128 columns x 64 bytes),
// issued two steps ahead; the f16 weights never touch LDS.  Lane
// (r32 = lane % 32, h32 = lane / 32) owns column n0 + 32 ns + r32 and the 32 k
// starting at 64 kh + 32 h32 of each step (16 bytes of nibbles, one LDS read).
// The MFMA's k order is free as long as X and W agree, so k-slot group h32 of
// substep ks is k = 64 kh + 32 h32 + 8 ks + 0..7: one nibble word of the lane,
// dequantized right before its MFMAs, and chunk 8 kh + 4 h32 + ks of the X row.
// Every weight is dequantized once, by the lane that multiplies it, and LDS
// carries no f16 weight tile.
// Dequant: bytes of (w & 0x0F0F0F0F) and ((w >> 4) & 0x0F0F0F0F) convert with
// v_cvt_f32_ubyteN, then fma(q, s, b) in f32 (mul then add for f32 scales)
// and a round-to-nearest-even pack to f16: the converter's
// RNE_f16(f32(q) * s + b).
// The loop holds no compiler-visible global access (the DMA is inline asm
// waited for by explicit counts): a register prefetch of W made the compiler
// copy the loaded registers between iterations behind a vmcnt(0), which
// drained every load in flight at each step.  Measured per k-step on the box:
// X fragment reads plus DMA (~170 KB of LDS traffic per CU) 0.48 us, with the
// MFMAs 0.82 us, everything 1.04 us; one wave per SIMD (4 waves, 128 x 32
// tiles over the whole step) took 1.36 us.
// ---------------------------------------------------------------------------
constexpr int kRegThreads = 512;
constexpr int kRegStages = 3;
constexpr int kRawStepBytes = BN * BK / 2;                           // W nibbles of one k-step
constexpr int kRegStageBytes = kStageHalves * 2 + kRawStepBytes;    // 40 KB
constexpr size_t kRegFixedLds = (size_t)kRegStages * kRegStageBytes;
constexpr size_t kRegExchangeBytes = 8 * 2 * 16 * 64 * 4;  // k-half exchange after the loop (64 KB)

template <int SBT>
__global__ __launch_bounds__(kRegThreads) void qgemm_q4_regw_kernel(const uint32_t* __restrict__ W,
                                                                   const void* __restrict__ S,
                                                                   const void* __restrict__ Bz, int gshift,
                                                                   const _Float16* __restrict__ X,
                                                                   float* __restrict__ out, int M, int N, int K,
                                                                   int k_per_split)
{
    extern __shared__ __align__(16) unsigned char smem[];
    // stage t: X tile at t * kRegStageBytes, W raw at + kStageHalves * 2; then the scales/biases
    uint32_t* sbl = reinterpret_cast<uint32_t*>(smem + kRegFixedLds);  // [BN][groups] as in the DMA kernel
    // wn through readfirstlane: the DMA's LDS bases derived from it stay scalar arithmetic.  Wave
    // wn = (kh, ns): k half kh of every step, 32-column slice ns of the tile.
    const int tid = threadIdx.x, lane = tid & 63, wn = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wn >> 2, ns = wn & 3;
    const int r32 = lane & 31, h32 = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int kbeg = blockIdx.z * k_per_split;
    const int kend = min(K, kbeg + k_per_split);
    const int nsteps = (kend - kbeg) / BK;
    float* o = out + (size_t)blockIdx.z * M * N;
    if (nsteps <= 0) return;  // the launcher never makes an empty split
    const int last = nsteps - 1;
    const int gpr = (K + (1 << gshift) - 1) >> gshift;
    const int g0 = kbeg >> gshift;
    const int ng = ((kend - 1) >> gshift) - g0 + 1;

    // X DMA: 4 per wave per stage, load j covers tile rows (wn * 4 + j) * 4 .. +4; byte offsets from
    // X + 2 kbeg (the launcher keeps M K 2 below 2^32)
    uint32_t xoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = (wn * 4 + j) * 4 + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        xoff[j] = (uint32_t)((size_t)min(m0 + r, M - 1) * K * 2 + 16 * c);
    }
    // W DMA: 1 per wave per stage, covering columns wn * 16 .. +16, 64 bytes each (columns past N
    // re-read the last one: computed, never stored); byte offsets from W + kbeg / 2
    const uint32_t woff =
        (uint32_t)((size_t)min(n0 + wn * 16 + (lane >> 2), N - 1) * (K / 2) + 16 * (lane & 3));
    const unsigned char* xbase = reinterpret_cast<const unsigned char*>(X) + (size_t)kbeg * 2;
    const unsigned char* wbase = reinterpret_cast<const unsigned char*>(W) + kbeg / 2;
    const uint32_t lds0 = lds_addr(smem);
    auto issue = [&](int step) {
        const int sc = min(step, last), st = step % kRegStages;
        const uint32_t base = lds0 + st * kRegStageBytes;
        const unsigned char* xs_ = xbase + (size_t)sc * BK * 2;
        const unsigned char* ws_ = wbase + (size_t)sc * (BK / 2);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16_s(xoff[j], xs_, base + (wn * 4 + j) * 1024);
        dma16_s(woff, ws_, base + kStageHalves * 2 + wn * 1024);
    };

    issue(0);
    {
        // scales/biases of this split's groups, loads batched before any use
        constexpr int PB = 8;
        const int total = BN * ng;
        for (int base = tid; base < total; base += PB * kRegThreads) {
            uint32_t sv[PB], bv[PB];
#pragma unroll
            for (int u = 0; u < PB; ++u) {
                const int i = min(base + u * kRegThreads, total - 1);
                const int col = i / ng, gi = i - col * ng;
                const size_t idx = (size_t)min(n0 + col, N - 1) * gpr + g0 + gi;
                sv[u] = load_raw<SBT>(S, idx);
                bv[u] = load_raw<SBT>(Bz, idx);
            }
#pragma unroll
            for (int u = 0; u < PB; ++u) {
                // unconditional (slots past the end rewrite the last one with its own value): a load
                // consumed only under a branch stays pending for the compiler on the other path, and
                // the first reuse of its register inside the k-loop became a vmcnt(0) drain per step
                const int i = min(base + u * kRegThreads, total - 1);
                if constexpr (SBT == DT_F32) {
                    sbl[2 * i] = sv[u];
                    sbl[2 * i + 1] = bv[u];
                } else {
                    sbl[i] = sv[u] | (bv[u] << 16);
                }
            }
        }
    }
    __syncthreads();
    issue(1);

    const int lcol = ns * 32 + r32;
    auto scale_bias = [&](int k) {
        const int gi = ((kbeg + k) >> gshift) - g0;
        float sc, bi;
        if constexpr (SBT == DT_F32) {
            sc = __builtin_bit_cast(float, sbl[2 * (lcol * ng + gi)]);
            bi = __builtin_bit_cast(float, sbl[2 * (lcol * ng + gi) + 1]);
        } else {
            const uint32_t sb = sbl[lcol * ng + gi];
            sc = raw_to_f32<SBT>(sb & 0xFFFFu);
            bi = raw_to_f32<SBT>(sb >> 16);
        }
        return make_float2(sc, bi);
    };

    f16v_t acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = f16v_t{};
    for (int s = 0; s < nsteps; ++s) {
        // Stage s was issued two steps ago; only stage s + 1 (5 loads per thread) may stay in flight.
        // A bare s_barrier: __syncthreads()'s release fence waits for vmcnt(0), i.e. for every DMA in
        // flight.  The asm waits carry memory clobbers, so no LDS access moves across them.
        wait_vmcnt<5>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // stage s complete everywhere; stage s - 1 no longer read
        issue(s + 2);                  // into the ring slot of stage s - 1
        const unsigned char* sbase = smem + (s % kRegStages) * kRegStageBytes;
        const _Float16* xa = reinterpret_cast<const _Float16*>(sbase);
        // this lane's 32 k of the step: k = 64 kh + 32 h32 + 8 ks + 0..7 (substep ks = 0..3)
        const u4_t w = *reinterpret_cast<const u4_t*>(sbase + kStageHalves * 2 + lcol * 64 + 32 * kh + 16 * h32);
        const float2 sb = scale_bias(s * BK + 64 * kh + 32 * h32);
        // A fragments are read one substep ahead of their MFMAs
        h8_t a[2][4];
        auto read_a = [&](int ks, h8_t (&dst)[4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dst[i] = *reinterpret_cast<const h8_t*>(xa + slot(i * 32 + r32, 8 * kh + 4 * h32 + ks) * 8);
        };
        read_a(0, a[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks + 1 < 4) read_a(ks + 1, a[(ks + 1) & 1]);
            const h8_t b = dequant_word_bytes<SBT>(w[ks], sb.x, sb.y);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks & 1][i], b, acc[i], 0, 0, 0);
        }
    }
    // drain the trailing (re-read) DMA before the stage memory is reused
    wait_vmcnt<0>();
    __syncthreads();

    // The two k halves meet through LDS: wave (kh, ns) hands the row tiles the other half keeps to
    // its partner (kh = 0 keeps rows 0..63, kh = 1 rows 64..127) and adds what it receives; lane l
    // exchanges with lane l of the partner, 8 KB per wave.  All partner values are read before any
    // add or store (one LDS round trip instead of one per store).
    float* xch = reinterpret_cast<float*>(smem);
    const int ncol = n0 + lcol;
    auto finish = [&](auto keep_c) {
        constexpr int KEEP = decltype(keep_c)::value, GIVE = 2 - KEEP;  // constant indices: no scratch
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) xch[(((wn * 2 + t) * 16 + r) * 64) + lane] = acc[GIVE + t][r];
        __syncthreads();
        float other[2][16];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) other[t][r] = xch[((((wn ^ 4) * 2 + t) * 16 + r) * 64) + lane];
        if (ncol >= N) return;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                // register r of a 32x32 tile: row (r/4)*8 + (lane/32)*4 + r%4, column lane%32
                const int m = m0 + (KEEP + t) * 32 + (r >> 2) * 8 + h32 * 4 + (r & 3);
                if (m < M) __builtin_nontemporal_store(acc[KEEP + t][r] + other[t][r], o + (size_t)m * N + ncol);
            }
    };
    if (kh == 0)
        finish(std::integral_constant<int, 0>{});
    else
        finish(std::integral_constant<int, 2>{});
}

#ifndef CELLM_QGEMM_MIN_SPLIT_STEPS
#define CELLM_QGEMM_MIN_SPLIT_STEPS 4
#endif
constexpr int kMinSplitSteps = CELLM_QGEMM_MIN_SPLIT_STEPS;  // k-steps per split at least

struct Plan {
    int splits;
    int k_per_split;
    size_t lds;
};

// Split-K so the grid covers the 256 CUs (each split >= 4 steps), and enough
// splits that a split's scales/biases fit the LDS left by the tiles.
Plan plan(int M, int N, int K, int group, int sbt, size_t fixed_lds)
{
    Plan p{0, 0, 0};
    if (K <= 0 || K % BK != 0 || group < 32) return p;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int steps = K / BK;
    int splits = 1;
    while (tiles * splits * 2 <= 256 && steps / (splits * 2) >= kMinSplitSteps) splits *= 2;
    const size_t sb_bytes = sbt == DT_F32 ? 8 : 4;
    for (;;) {
        const int sps = (steps + splits - 1) / splits;
        const int kps = sps * BK;
        const int ng = (kps + group - 1) / group + 1;  // + 1: a split may start mid-group
        const size_t lds = fixed_lds + (size_t)BN * ng * sb_bytes;
        if (lds <= kMaxLds) {
            p.splits = (steps + sps - 1) / sps;  // no empty split
            p.k_per_split = kps;
            p.lds = lds;
            return p;
        }
        if (sps == 1) return Plan{0, 0, 0};
        ++splits;
    }
}

}  // namespace dma

}  // namespace

// Choose the split-K factor so the grid covers the chip: 256 CUs.
int qgemm_splits(int M, int N, int K)
{
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int ksteps = (K + BK - 1) / BK;
    int splits = 1;
    // one round of blocks on 256 CUs; each split keeps >= 8 stages so the
    // prefetch ring has something to overlap
    while (tiles * splits * 2 <= 256 && ksteps / (splits * 2) >= 8) splits *= 2;
    return splits;
}

size_t qgemm_workspace_bytes(int wt, int M, int N, int K, int group_size, int sbt)
{
    if (wt == 0) {
        const dma::Plan p = dma::plan(M, N, K, group_size, sbt, dma::kRegFixedLds);
        if (p.splits > 0) return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
    }
    const int splits = qgemm_splits(M, N, K);
    return splits > 1 ? (size_t)splits * M * N * sizeof(float) : 0;
}

// Dynamic LDS above 64 KB needs the per-function limit raised once per device and kernel (keyed by the
// kernel itself: every instantiation of a kernel template has the same pointer type).
template <typename Kern>
static hipError_t allow_lds(Kern kern, size_t bytes)
{
    static std::mutex mu;
    static std::vector<std::pair<int, const void*>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const void* fn = reinterpret_cast<const void*>(kern);
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& d : done)
        if (d.first == dev && d.second == fn) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dma::kMaxLds);
    if (e == hipSuccess) done.emplace_back(dev, fn);
    (void)bytes;
    return e;
}

template <int SBT>
static hipError_t launch_q4_regw(const dma::Plan& p, const uint32_t* wq, const void* S, const void* B, int gshift,
                                 const _Float16* x, float* out, int M, int N, int K, hipStream_t st)
{
    auto kern = dma::qgemm_q4_regw_kernel<SBT>;
    hipError_t e = allow_lds(kern, p.lds);
    if (e != hipSuccess) return e;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, p.splits);
    hipLaunchKernelGGL(kern, grid, dim3(dma::kRegThreads), p.lds, st, wq, S, B, gshift, x, out, M, N, K,
                       p.k_per_split);
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_qgemm_common(const void* W, const void* S, const void* B, int sbt, int group_size,
                                      int per_channel, const _Float16* X, float* Y, const float* bias, int M, int N,
                                      int K, float* workspace, hipStream_t st)
{
    const int splits = workspace ? qgemm_splits(M, N, K) : 1;
    const int ksteps = (K + BK - 1) / BK;
    const int k_per_split = ((ksteps + splits - 1) / splits) * BK;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, splits);
    float* out = splits > 1 ? workspace : Y;
#define CELLM_QGEMM(SBT_)                                                                                          \
    hipLaunchKernelGGL((qgemm_kernel<WT, SBT_, kStages>), grid, dim3(kThreads), 0, st, W, S, B, group_size, X, out, M, N, K, \
                       k_per_split, per_channel)
    if (sbt == DT_F32) CELLM_QGEMM(DT_F32);
    else if (sbt == DT_F16) CELLM_QGEMM(DT_F16);
    else CELLM_QGEMM(DT_BF16);
#undef CELLM_QGEMM
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t total = (size_t)M * N;
    unsigned blocks = (unsigned)((total + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (splits > 1) {
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, workspace, Y, bias, splits, M, N);
        e = hipGetLastError();
    } else if (bias) {
        hipLaunchKernelGGL(add_bias_kernel, dim3(blocks), dim3(256), 0, st, Y, bias, M, N);
        e = hipGetLastError();
    }
    return e;
}

hipError_t launch_qgemm_q4_affine_ws(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                     const _Float16* x, float* y, int M, int N, int K, float* workspace,
                                     hipStream_t st)
{
    dma::Plan p = dma::plan(M, N, K, group_size, sbt, dma::kRegFixedLds);
    p.lds = std::max(p.lds, dma::kRegExchangeBytes);
    const bool offsets_fit = (uint64_t)M * K * 2 < (1ull << 32) && (uint64_t)N * K / 2 < (1ull << 32);
    if (p.splits > 0 && (p.splits == 1 || workspace) && offsets_fit) {
        const int gshift = __builtin_ctz((unsigned)group_size);
        float* out = p.splits > 1 ? workspace : y;
        hipError_t e = sbt == DT_F16   ? launch_q4_regw<DT_F16>(p, wq, S, B, gshift, x, out, M, N, K, st)
                       : sbt == DT_F32 ? launch_q4_regw<DT_F32>(p, wq, S, B, gshift, x, out, M, N, K, st)
                                       : launch_q4_regw<DT_BF16>(p, wq, S, B, gshift, x, out, M, N, K, st);
        if (e != hipSuccess || p.splits == 1) return e;
        const size_t total = (size_t)M * N;
        unsigned blocks = (unsigned)((total + 255) / 256);
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, workspace, y, nullptr, p.splits, M,
                           N);
        return hipGetLastError();
    }
    return launch_qgemm_common<0>(wq, S, B, sbt, group_size, 1, x, y, nullptr, M, N, K, workspace, st);
}

hipError_t launch_qgemm_i8_ws(const int8_t* w, const void* S, int sdt, int per_channel, const _Float16* x,
                              const float* bias, float* y, int M, int N, int K, float* workspace, hipStream_t st)
{
    return launch_qgemm_common<1>(w, S, nullptr, sdt, 64, per_channel, x, y, bias, M, N, K, workspace, st);
}

}  // namespace cellm
