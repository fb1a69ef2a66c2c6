// Shared device helpers for the cellm HIP kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cellm {

// Element types understood by the kernels.  The integer values are the ABI
// values of cellm_hip_dtype_t in include/cellm_hip.h.
enum DType : int32_t { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef float f16v_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t as_u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Exact widening of one stored scale/bias/activation element to f32.
template <int DT>
__device__ __forceinline__ float load_f32(const void* p, size_t i)
{
    if constexpr (DT == DT_F32) {
        return reinterpret_cast<const float*>(p)[i];
    } else if constexpr (DT == DT_F16) {
        return (float)reinterpret_cast<const _Float16*>(p)[i];
    } else {
        uint32_t b = (uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16;
        return __builtin_bit_cast(float, b);
    }
}

// Split load/convert: load_raw issues the memory access and returns the
// stored bits; raw_to_f32 widens them at the point of use.  Keeping the
// conversion away from the load lets the compiler leave the load in flight
// (a conversion right after a load forces an s_waitcnt on every earlier load).
template <int DT>
__device__ __forceinline__ uint32_t load_raw(const void* p, size_t i)
{
    if constexpr (DT == DT_F32) {
        return reinterpret_cast<const uint32_t*>(p)[i];
    } else {
        return (uint32_t)reinterpret_cast<const uint16_t*>(p)[i];
    }
}

template <int DT>
__device__ __forceinline__ float raw_to_f32(uint32_t r)
{
    if constexpr (DT == DT_F32) {
        return __builtin_bit_cast(float, r);
    } else if constexpr (DT == DT_F16) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)r);
    } else {
        return __builtin_bit_cast(float, r << 16);
    }
}

// v_and_or_b32: (a & mask) | bits in one VOP3 op.  gfx9 VOP3 can encode
// neither a literal nor more than one SGPR operand, so the mask comes from an
// SGPR and the OR constant from a VGPR the compiler hoists out of the loops.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits)
{
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(mask), "v"(bits));
    return d;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
{
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Sum over aligned groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v)
{
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, W);
    return v;
}

}  // namespace cellm
