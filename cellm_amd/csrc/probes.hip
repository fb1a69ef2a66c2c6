// Measurement probes for bench.py: the box's own dense f16 MFMA rate and
// streaming HBM read rate, the ceilings the qGEMM and the GEMV rooflines are
// read against beside the published peaks.  Not part of the hot path; built
// into libcellm_probes.so, which only bench.py loads.
//
//   cellm_probe_mfma_f16:    blocks x 4 waves, each wave `iters` rounds of
//                            eight independent v_mfma_f32_32x32x16_f16 chains
//                            on register operands (no memory traffic);
//                            flop = blocks * 4 * iters * 8 * 2 * 32*32*16.
//   cellm_probe_stream_read: every 16-byte unit of `bytes` read once with
//                            non-temporal loads, four in flight per lane, a
//                            grid-stride walk over one 512-thread block per CU
//                            (the best of the shapes swept on the box).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 ph8_t __attribute__((ext_vector_type(8)));
typedef float pf16v_t __attribute__((ext_vector_type(16)));
typedef uint32_t pu4_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int kChains = 8;

__global__ __launch_bounds__(256) void mfma_f16_probe_kernel(int iters, float* __restrict__ sink)
{
    const int lane = threadIdx.x & 63;
    ph8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (float)((lane + i) & 7));
        b[i] = (_Float16)(0.002f * (float)((lane * 3 + i) & 7));
    }
    pf16v_t acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = pf16v_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    // one store per block keeps the chains live without measurable traffic
    if (threadIdx.x == 0) sink[blockIdx.x] = s;
}

__global__ __launch_bounds__(512) void stream_read_probe_kernel(const pu4_t* __restrict__ p, size_t n16,
                                                                uint32_t* __restrict__ sink)
{
    constexpr int U = 4;
    pu4_t acc = {0u, 0u, 0u, 0u};
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        pu4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= p[i];
    // a store that (almost) never happens keeps the loads from being removed
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = acc.x;
}

int cus_of_current_device()
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) return 256;
    return cus;
}

}  // namespace

extern "C" {

// Enqueue one MFMA probe launch on `stream`; `sink` holds `blocks` floats.
// Returns 0, or -1 for bad arguments, -2 for a launch error.
int32_t cellm_probe_mfma_f16(int32_t blocks, int32_t iters, float* sink, hipStream_t stream)
{
    if (blocks < 1 || iters < 1 || !sink) return -1;
    hipLaunchKernelGGL(mfma_f16_probe_kernel, dim3(blocks), dim3(256), 0, stream, iters, sink);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Flops of one cellm_probe_mfma_f16 launch.
double cellm_probe_mfma_f16_flops(int32_t blocks, int32_t iters)
{
    return (double)blocks * 4.0 * iters * kChains * 2.0 * 32.0 * 32.0 * 16.0;
}

// Enqueue one streaming read of `bytes` (a multiple of 16, 16-byte aligned) on `stream`.
int32_t cellm_probe_stream_read(const void* p, uint64_t bytes, uint32_t* sink, hipStream_t stream)
{
    if (!p || !sink || bytes == 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(p) & 15)) return -1;
    hipLaunchKernelGGL(stream_read_probe_kernel, dim3(cus_of_current_device()), dim3(512), 0, stream,
                       reinterpret_cast<const pu4_t*>(p), (size_t)(bytes >> 4), sink);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
