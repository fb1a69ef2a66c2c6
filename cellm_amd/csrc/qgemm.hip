// Quantized-weight GEMM on MFMA for prefill and batched decode (gfx950).
//
//   Y[M,N] = X[M,K] . dequant(W)[N,K]^T        (f16 X, f32 accumulate, f32 Y)
//
// Reference: there is no batched or GEMM path in cellm (prefill runs the GEMV
// token by token, crates/cellm-model/src/llama.rs:214-233).  The per-element
// oracle is cpu_kernels::matmul_f32 (cpu_kernels.rs:36-63) over the dequantized
// weight, summed over k ascending.
//
// Weight tiles are dequantized into LDS as f16 with the converter's rounding,
// h = RNE_f16(f32(q)*s + b) (tools/convert/src/main.rs:4435-4436).  For f16 or
// bf16 scales, f32(q)*s is exact in f32, so fma(q, s, b) rounds exactly as the
// reference's mul-then-add does; f32 scales take a separate mul and add.
// int8 weights are exact in f16; their per-row scale is applied in the epilogue
// (y = acc * s, cpu_kernels.rs:130).
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; block tile 128x128, wave tile
// 64x64 = 4x4 v_mfma_f32_16x16x32_f16 tiles; BK = 64 per LDS stage.  The next
// stage's global data is prefetched into registers during the MFMA loop.
// Split-K over blockIdx.z writes f32 partials to a workspace that a second
// kernel sums in a fixed order (deterministic).
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

size_t qgemm_workspace_bytes(int M, int N, int K)
{
    const int splits = qgemm_splits(M, N, K);
    return splits > 1 ? (size_t)splits * M * N * sizeof(float) : 0;
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
    return launch_qgemm_common<0>(wq, S, B, sbt, group_size, 1, x, y, nullptr, M, N, K, workspace, st);
}

hipError_t launch_qgemm_i8_ws(const int8_t* w, const void* S, int sdt, int per_channel, const _Float16* x,
                              const float* bias, float* y, int M, int N, int K, float* workspace, hipStream_t st)
{
    return launch_qgemm_common<1>(w, S, nullptr, sdt, 64, per_channel, x, y, bias, M, N, K, workspace, st);
}

}  // namespace cellm
