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
typedef int32_t i4_t __attribute__((ext_vector_type(4)));
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

// Butterfly partners on DPP (VALU moves within a 16-lane row, no LDS permute
// round trip): lane i gets the value of lane i ^ 1, i ^ 2, i ^ 4 or i ^ 8.  xor 1
// and 2 are quad permutes; xor 4 and 8 pick a row shift up or down by the lane
// bit.  Every lane read must be active.
__device__ __forceinline__ float dpp_xor1(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
// lanes with bit `B` clear read B lanes up (row_shl:B), the others B lanes down (row_shr:B)
template <int B>
__device__ __forceinline__ float dpp_xor_row(float v)
{
    const int b = __builtin_bit_cast(int, v);
    const int up = __builtin_amdgcn_update_dpp(0, b, 0x100 + B, 0xF, 0xF, false);
    const int down = __builtin_amdgcn_update_dpp(0, b, 0x110 + B, 0xF, 0xF, false);
    return __builtin_bit_cast(float, (threadIdx.x & B) ? down : up);
}
// xor 16 and 32 with the gfx950 lane swaps: v_permlane16_swap exchanges the odd
// 16-lane rows of its first operand with the even rows of its second, and
// v_permlane32_swap the upper half of the first with the lower half of the
// second; with v in both, the partner's value is in the first result for lanes
// with the bit set and in the second for the others.
template <int B>
__device__ __forceinline__ float swap_xor(float v)
{
    const int b = __builtin_bit_cast(int, v);
    if constexpr (B == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
        return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
    }
}
template <int OFF>
__device__ __forceinline__ float lane_xor(float v, int width)
{
    (void)width;  // every partner lies inside the aligned group of `width` lanes
    if constexpr (OFF == 1) return dpp_xor1(v);
    else if constexpr (OFF == 2) return dpp_xor2(v);
    else if constexpr (OFF == 4 || OFF == 8) return dpp_xor_row<OFF>(v);
    else return swap_xor<OFF>(v);
}

// Sum over aligned groups of W lanes (W a power of two <= 64): the butterfly
// v += partner(v ^ off) for off = W/2 .. 1, every step a VALU lane move (DPP
// below 16, the lane swaps at 16 and 32).  Every lane of a group must be active.
template <int W>
__device__ __forceinline__ float group_sum(float v)
{
    if constexpr (W >= 64) v += lane_xor<32>(v, W);
    if constexpr (W >= 32) v += lane_xor<16>(v, W);
    if constexpr (W >= 16) v += lane_xor<8>(v, W);
    if constexpr (W >= 8) v += lane_xor<4>(v, W);
    if constexpr (W >= 4) v += lane_xor<2>(v, W);
    if constexpr (W >= 2) v += lane_xor<1>(v, W);
    return v;
}
// Maximum over aligned groups of W lanes (the butterfly of group_sum with fmaxf).
template <int W>
__device__ __forceinline__ float group_max(float v)
{
    if constexpr (W >= 64) v = fmaxf(v, lane_xor<32>(v, W));
    if constexpr (W >= 32) v = fmaxf(v, lane_xor<16>(v, W));
    if constexpr (W >= 16) v = fmaxf(v, lane_xor<8>(v, W));
    if constexpr (W >= 8) v = fmaxf(v, lane_xor<4>(v, W));
    if constexpr (W >= 4) v = fmaxf(v, lane_xor<2>(v, W));
    if constexpr (W >= 2) v = fmaxf(v, lane_xor<1>(v, W));
    return v;
}
// Sums of V values over aligned teams of W lanes, transposed (V <= W, both powers
// of two): log2(V) halving steps, each at offset O = W/2, W/4, ..., leave every
// lane with one value, and plain butterfly steps finish the sum over the team.
// In a halving step a lane keeps the low half of its values when its lane bit O
// is clear and the high half when set, adding the partner's copy of that half:
// one lane swap per pair of values at O = 16 and 32 (the swap hands each side
// the half it keeps), two DPP adds and a select below.  Lane l ends with the
// team total of value index  sum_s bit(l, W >> (s + 1)) * V / 2^(s + 1)
// (team_sum_t_index), against one full butterfly per value otherwise.
template <int O>
__device__ __forceinline__ float half_step(float lo, float hi)
{
    if constexpr (O >= 16) {
        const int a = __builtin_bit_cast(int, lo), b = __builtin_bit_cast(int, hi);
        const auto r = O == 32 ? __builtin_amdgcn_permlane32_swap(a, b, false, false)
                               : __builtin_amdgcn_permlane16_swap(a, b, false, false);
        // ROCm 7.2's compiler folds r[0] + r[1] of one lane swap into r[0] + r[0] (checked in
        // the gfx950 assembly); an empty asm on both results keeps them apart
        uint32_t x = r[0], y = r[1];
        asm("" : "+v"(x), "+v"(y));
        return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
    } else {
        float l, h;
        if constexpr (O == 8 || O == 4) {
            l = lo + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, lo), 0x100 + O,
                                                                          0xF, 0xF, false));  // lane + O
            h = hi + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, hi), 0x110 + O,
                                                                          0xF, 0xF, false));  // lane - O
        } else if constexpr (O == 2) {
            l = lo + dpp_xor2(lo);
            h = hi + dpp_xor2(hi);
        } else {
            l = lo + dpp_xor1(lo);
            h = hi + dpp_xor1(hi);
        }
        return (threadIdx.x & O) ? h : l;
    }
}
template <int W, int V>
__device__ __forceinline__ float team_sum_t(const float (&a)[V])
{
    static_assert(V >= 1 && V <= W && (V & (V - 1)) == 0 && (W & (W - 1)) == 0, "V <= W, powers of two");
    if constexpr (V == 1) {
        return group_sum<W>(a[0]);
    } else {
        float b[V / 2];
#pragma unroll
        for (int i = 0; i < V / 2; ++i) b[i] = half_step<W / 2>(a[i], a[V / 2 + i]);
        return team_sum_t<W / 2, V / 2>(b);
    }
}
// The value index team_sum_t<W, V> leaves in lane `lane` (lanes of one team that
// differ only below bit W / V hold the same total).
template <int W, int V>
__device__ __forceinline__ int team_sum_t_index(int lane)
{
    int idx = 0;
#pragma unroll
    for (int o = W / 2, v = V / 2; v >= 1; o >>= 1, v >>= 1) idx += (lane & o) ? v : 0;
    return idx;
}

// Raw buffer resource over [base, base + bytes), bytes < 2^31.  A buffer store whose byte
// offset falls outside it is dropped by the hardware, so a masked store is one instruction
// with an out-of-range offset (kBufferDrop) in the lanes that must not write -- no branch,
// and the same number of memory instructions on every path.
constexpr uint32_t kBufferDrop = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}
// NT: non-temporal (streaming) store
template <bool NT>
__device__ __forceinline__ void buffer_store_f32(float v, __amdgpu_buffer_rsrc_t r, uint32_t byte_off)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)byte_off, 0, NT ? 2 : 0);
}
// Sum of the nsplit split-K partials p4[s * stride], s = 0, 1, ..., added in split order (a fixed
// order: deterministic), with eight splits' 16-byte loads in flight at a time (slots past the last
// split re-read it and are not added).
__device__ __forceinline__ f4_t sum_splits_f4(const f4_t* __restrict__ p4, size_t stride, int nsplit)
{
    f4_t a = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
        f4_t b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = p4[(size_t)min(s0 + j, nsplit - 1) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < nsplit) a = s0 + j == 0 ? b[j] : a + b[j];
    }
    return a;
}
__device__ __forceinline__ float quad_sum(float v) { return group_sum<4>(v); }
__device__ __forceinline__ float pair_sum(float v) { return group_sum<2>(v); }
__device__ __forceinline__ float oct_sum(float v) { return group_sum<8>(v); }


// ---- gate/up activation epilogues -------------------------------------------
// ACT_SILU: silu(g) * u with silu(g) = g * (1 / (1 + exp(-g))), the order of
// silu_mul_f32_inplace (metal.rs:232-243) and llama.rs:477-484.
// ACT_GELU_TANH: gelu_tanh(g) * u with gelu_tanh(x) = 0.5 x (1 + tanh(k (x + c x^3))),
// k = 0.7978846, c = 0.044715, evaluated in the reference's order
// (crates/cellm-model/src/gemma.rs:1689-1693, applied at :844-846;
// gelu_tanh_mul_f32_inplace, metal.rs:245-257): c*x*x*x as ((c*x)*x)*x, every
// product and sum rounded in f32 (no contraction).
enum Act : int32_t { ACT_SILU = 0, ACT_GELU_TANH = 1 };

__device__ __forceinline__ float act_mul(int act, float g, float u)
{
#pragma clang fp contract(off)
    if (act == ACT_GELU_TANH) {
        const float k = 0.7978846f, c = 0.044715f;
        const float inner = k * (g + ((c * g) * g) * g);
        return ((0.5f * g) * (1.0f + tanhf(inner))) * u;
    }
    const float sig = 1.0f / (1.0f + expf(-g));
    return (g * sig) * u;
}

// ---- MLX affine dequant of one u32 word of nibbles to f16, as the converter
// rounds it (tools/convert/src/main.rs:4435-4436): RNE_f16(f32(q) * s + b),
// the product and the sum rounded in f32 (one fma when s is f16/bf16: q * s is
// then exact), then one round-to-nearest-even to f16.  Output in natural
// order: element j = nibble j of the word.  Shared by the prefill qGEMM and
// the batched decode tiles.
// v_cvt_f32_ubyteN: byte N of a register to f32.  Spelled out because the compiler folds
// (float)((x >> 8N) & 0xFF) of a masked word back into one v_bfe_u32 per nibble plus a convert.
template <int N>
__device__ __forceinline__ float cvt_ubyte(uint32_t x)
{
    float f;
    if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(x));
    else if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(x));
    else if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(x));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(x));
    return f;
}

template <int SBT>
__device__ __forceinline__ h8_t dequant_word_bytes(uint32_t w, float s, float b)
{
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const float q[8] = {cvt_ubyte<0>(lo), cvt_ubyte<0>(hi), cvt_ubyte<1>(lo), cvt_ubyte<1>(hi),
                        cvt_ubyte<2>(lo), cvt_ubyte<2>(hi), cvt_ubyte<3>(lo), cvt_ubyte<3>(hi)};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float q0 = q[2 * i], q1 = q[2 * i + 1];  // nibbles 2i, 2i + 1
        if constexpr (SBT == DT_F32) {
#pragma clang fp contract(off)
            const float t0 = q0 * s, t1 = q1 * s;
            v[2 * i] = t0 + b;
            v[2 * i + 1] = t1 + b;
        } else {
            v[2 * i] = __builtin_fmaf(q0, s, b);  // q*s exact: same bits as mul-then-add
            v[2 * i + 1] = __builtin_fmaf(q1, s, b);
        }
    }
    h8_t h;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        // Keep the f32 rounding (no fused v_fma_mix*_f16 with a single rounding).  Not volatile: a
        // volatile asm is a scheduling barrier.
        asm("" : "+v"(v[k]));
        h[k] = (_Float16)v[k];
    }
    return h;
}

}  // namespace cellm
