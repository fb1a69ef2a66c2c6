// Bit-exact dequantization of MLX 4-bit affine weights, the symmetric-i4 GEMV
// and the device smoke-test kernel.
//
// Dequant semantics:
//   f32 out: w = f32(q) * s + b, multiply and add rounded separately
//            (crates/cellm-model/src/lfm.rs:1014-1025)
//   f16 out: h = RNE_f16(f32(q) * s + b)   (tools/convert/src/main.rs:4430-4436)
// Contraction into v_fma_f32 would round once instead of twice, so this file
// turns contraction off for the element formula.
#include "common.hpp"
#include "kernels.hpp"

namespace cellm {

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float affine_elem(uint32_t q, float s, float b)
{
#pragma clang fp contract(off)
    const float t = (float)q * s;
    return t + b;
}

// One thread per u32 word (8 elements).  Rows have K/8 words; groups of
// `gsize` elements share a scale/bias; g = min(i/gsize, groups-1).
template <int SBT, int OUT_F16>
__global__ __launch_bounds__(kBlock) void dequant_q4_affine_kernel(const uint32_t* __restrict__ wq,
                                                                   const void* __restrict__ S,
                                                                   const void* __restrict__ B, void* __restrict__ out,
                                                                   int N, int K, int gsize)
{
    const int P = K >> 3;
    const size_t total = (size_t)N * P;
    const int groups = (K + gsize - 1) / gsize;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (size_t)gridDim.x * kBlock) {
        const int n = (int)(i / P);
        const int p = (int)(i - (size_t)n * P);
        const uint32_t w = wq[i];
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            int g = (p * 8 + k) / gsize;
            g = g < groups - 1 ? g : groups - 1;
            const float s = load_f32<SBT>(S, (size_t)n * groups + g);
            const float b = load_f32<SBT>(B, (size_t)n * groups + g);
            v[k] = affine_elem((w >> (4 * k)) & 0xFu, s, b);
        }
        if constexpr (OUT_F16) {
            h8_t h;
#pragma unroll
            for (int k = 0; k < 8; ++k) h[k] = (_Float16)v[k];  // v_cvt_f16_f32: round to nearest even
            reinterpret_cast<h8_t*>(out)[i] = h;
        } else {
            float* o = reinterpret_cast<float*>(out) + i * 8;
            *reinterpret_cast<f4_t*>(o) = f4_t{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f4_t*>(o + 4) = f4_t{v[4], v[5], v[6], v[7]};
        }
    }
}

__global__ void fill_f32_kernel(float* __restrict__ y, float v, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) y[i] = v;
}

__global__ void add_f32_kernel(const float* a, const float* b, float* out, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// g[i] = silu(g[i]) * u[i], silu(g) = g / (1 + exp(-g)) as silu_mul_f32_inplace
// (crates/cellm-kernels/src/metal.rs:235-245) and llama.rs:477-484
__global__ void silu_mul_kernel(float* __restrict__ g, const float* __restrict__ u, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float x = g[i];
        const float sig = 1.0f / (1.0f + expf(-x));
        g[i] = (x * sig) * u[i];
    }
}

// g[i] = gelu_tanh(g[i]) * u[i]: gelu_tanh_mul_f32_inplace (metal.rs:245-257) and the CPU
// loop of gemma.rs:844-846 over gelu_tanh_f32 (gemma.rs:1689-1693), in act_mul's order
__global__ void gelu_tanh_mul_kernel(float* __restrict__ g, const float* __restrict__ u, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        g[i] = act_mul(ACT_GELU_TANH, g[i], u[i]);
}

}  // namespace

hipError_t launch_dequant_q4_affine(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                    void* out, int out_dt, int N, int K, hipStream_t st)
{
    const size_t total = (size_t)N * (size_t)(K >> 3);
    size_t blocks = (total + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)blocks);
#define CELLM_DQ(SBT_, F16_)                                                                                    \
    hipLaunchKernelGGL((dequant_q4_affine_kernel<SBT_, F16_>), grid, dim3(kBlock), 0, st, wq, S, B, out, N, K, \
                       group_size)
    const bool f16 = out_dt == DT_F16;
    if (sbt == DT_F32) { if (f16) CELLM_DQ(DT_F32, 1); else CELLM_DQ(DT_F32, 0); }
    else if (sbt == DT_F16) { if (f16) CELLM_DQ(DT_F16, 1); else CELLM_DQ(DT_F16, 0); }
    else { if (f16) CELLM_DQ(DT_BF16, 1); else CELLM_DQ(DT_BF16, 0); }
#undef CELLM_DQ
    return hipGetLastError();
}

__global__ void add_bias_rows_kernel(float* __restrict__ y, const float* __restrict__ bias, int M, int N)
{
    const size_t total = (size_t)M * N;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x)
        y[i] += bias[i % (size_t)N];
}

hipError_t launch_add_bias_rows(float* y, const float* bias, int M, int N, hipStream_t st)
{
    const size_t total = (size_t)M * N;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(add_bias_rows_kernel, dim3(blocks), dim3(256), 0, st, y, bias, M, N);
    return hipGetLastError();
}

hipError_t launch_act_mul(int act, float* g, const float* u, size_t count, hipStream_t st)
{
    if (act == ACT_SILU) return launch_silu_mul(g, u, count, st);
    if (count == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(gelu_tanh_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, u, count);
    return hipGetLastError();
}

hipError_t launch_silu_mul(float* g, const float* u, size_t count, hipStream_t st)
{
    if (count == 0) return hipSuccess;
    size_t blocks = (count + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, u, count);
    return hipGetLastError();
}

// A kernel, not hipMemsetAsync: a caller capturing the stream into a HIP graph gets a kernel node.
hipError_t launch_fill_f32(float* y, float v, size_t count, hipStream_t st)
{
    if (count == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, y, v, count);
    return hipGetLastError();
}

hipError_t launch_add_f32(const float* a, const float* b, float* out, int n, hipStream_t st)
{
    hipLaunchKernelGGL(add_f32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, a, b, out, n);
    return hipGetLastError();
}

}  // namespace cellm
