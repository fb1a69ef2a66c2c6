/*
 * cellm_oracle.c -- CPU restatement of cellm's quantized-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library under cellm_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * The reference (jeffasante/cellm) is Rust and cannot be built here, so each
 * function restates the reference arithmetic in C, in the same operation
 * order, and cites the reference file:line it follows.  Build flags
 * (oracle/Makefile): -O3 -ffp-contract=off -fno-fast-math, so that every
 * f32 multiply and add rounds separately and no sum is reassociated, which
 * is what rustc/LLVM does for Rust f32 code.
 *
 * Parity pins (tests/test_oracle.py): every function below is checked against
 * closed forms, IEEE conversions from numpy, exhaustive nibble/byte sweeps,
 * fp64 error bounds and brute-force tiny cases.  The config-5 decode-step
 * helpers at the bottom (rms_norm, RoPE in both layouts, attention, softmax,
 * SiLU, tanh GELU) are pinned by closed forms (RoPE at pos 0 is the identity,
 * rotation preserves the norm of each pair and the two layouts are one
 * permutation apart, softmax of equal scores is uniform, attention over one
 * token returns v, gelu(0) = 0 and gelu(x) - gelu(-x) = x, the tanh GELU
 * within its published distance of the erf GELU).
 * Their glibc expf/sinf/cosf/powf calls are not bit-pinned across machines;
 * that is why the decode step is compared by greedy token id.
 *
 * Parallelism: row loops carry "#pragma omp parallel for schedule(static)",
 * mirroring rayon's par_iter over output rows (cpu_kernels.rs:78).  Rows are
 * independent, so the thread count never changes a result bit.
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>
#include <float.h>

#define ORACLE_F32 0
#define ORACLE_F16 1
#define ORACLE_BF16 2

/* ------------------------------------------------------------------------ */
/* IEEE-754 binary16 / bfloat16 conversions (the `half` crate, v2.4).        */
/* ------------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* f16::from_bits(h).to_f32(): exact widening (cpu_kernels.rs:80,212,238). */
float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return bits_to_f32(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) {
        return bits_to_f32(sign | 0x7f800000u | (man << 13));
    }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* f16::from_f32(f): IEEE round-to-nearest-even narrowing
 * (tools/convert/src/main.rs:3925,4436; crates/cellm-cache/src/kvcache.rs:611-612). */
uint16_t oracle_f32_to_f16(float f)
{
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13)); /* quiet NaN, keep payload top */
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {
        /* subnormal or zero in f16 */
        if (e < -10) return (uint16_t)sign; /* rounds to zero (below half the min subnormal) */
        uint32_t m = man | 0x800000u;       /* implicit bit */
        uint32_t shift = (uint32_t)(14 - e); /* 24-bit significand -> 10-bit subnormal field */
        uint32_t half_bit = 1u << (shift - 1);
        uint32_t rest = m & ((1u << shift) - 1u);
        uint32_t r = m >> shift;
        if (rest > half_bit || (rest == half_bit && (r & 1u))) r += 1u;
        return (uint16_t)(sign | r); /* r may carry into the min normal: still correct */
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) r += 1u; /* carry may reach inf: correct */
    return (uint16_t)(sign | r);
}

/* bf16 -> f32 widening (converter bf16_bytes_to_f32_slice, main.rs:4374-4401). */
float oracle_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

static inline float load_as_f32(const void* p, int dtype, size_t i)
{
    switch (dtype) {
    case ORACLE_F16: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    case ORACLE_BF16: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Deterministic generator: the reference test LCG                          */
/* (crates/cellm-kernels/tests/metal_parity.rs:17-26).                      */
/* ------------------------------------------------------------------------ */

static inline uint64_t lcg_next(uint64_t s) { return s * 6364136223846793005ull + 1ull; }
/* ((s >> 32) as u32) as f32 / (u32::MAX as f32) */
static inline float lcg_unit(uint64_t s) { return (float)(uint32_t)(s >> 32) / (float)UINT32_MAX; }

/* lcg_fill(len, seed, scale): v = (x*2 - 1) * scale, metal_parity.rs:17-26. */
void oracle_lcg_fill(float* out, size_t n, uint64_t seed, float scale)
{
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = lcg_next(s);
        float x = lcg_unit(s);
        out[i] = (x * 2.0f - 1.0f) * scale;
    }
}

/* U(0,1) draws from the same LCG, as float in [0,1]. */
void oracle_lcg_unit(float* out, size_t n, uint64_t seed)
{
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) { s = lcg_next(s); out[i] = lcg_unit(s); }
}

/* int8 weights uniform in [-127,127]: q = min(floor(u*255), 254) - 127. */
void oracle_gen_i8(int8_t* out, size_t n, uint64_t seed)
{
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = lcg_next(s);
        int q = (int)floorf(lcg_unit(s) * 255.0f);
        if (q > 254) q = 254;
        out[i] = (int8_t)(q - 127);
    }
}

/* nibbles uniform in [0,15], packed 8 per u32 along K (nibble k of word p is element 8p+k). */
void oracle_gen_q4_words(uint32_t* out, size_t nwords, uint64_t seed)
{
    uint64_t s = seed;
    for (size_t i = 0; i < nwords; ++i) {
        uint32_t w = 0;
        for (int k = 0; k < 8; ++k) {
            s = lcg_next(s);
            uint32_t q = (uint32_t)floorf(lcg_unit(s) * 16.0f);
            if (q > 15u) q = 15u;
            w |= q << (4 * k);
        }
        out[i] = w;
    }
}

/* uniform in [lo, hi) as f32. */
void oracle_gen_uniform(float* out, size_t n, uint64_t seed, float lo, float hi)
{
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) { s = lcg_next(s); out[i] = lo + lcg_unit(s) * (hi - lo); }
}

/* N(mu, sigma) by Box-Muller on pairs of LCG draws; if positive_only, redraw until > 0. */
void oracle_gen_normal(float* out, size_t n, uint64_t seed, float mu, float sigma, int positive_only)
{
    uint64_t s = seed;
    size_t i = 0;
    while (i < n) {
        s = lcg_next(s);
        double u1 = (double)lcg_unit(s);
        s = lcg_next(s);
        double u2 = (double)lcg_unit(s);
        if (u1 < 1e-12) u1 = 1e-12;
        double r = sqrt(-2.0 * log(u1));
        double z0 = r * cos(6.283185307179586 * u2);
        double z1 = r * sin(6.283185307179586 * u2);
        float v0 = (float)(mu + sigma * z0);
        float v1 = (float)(mu + sigma * z1);
        if (!positive_only || v0 > 0.0f) out[i++] = v0;
        if (i < n && (!positive_only || v1 > 0.0f)) out[i++] = v1;
    }
}

/* ------------------------------------------------------------------------ */
/* int8 per-output-row scaled GEMV.                                         */
/* ------------------------------------------------------------------------ */

/* cpu_kernels::matmul_i8_f32, x86 branch (crates/cellm-kernels/src/cpu_kernels.rs:66-80,124-131):
 * acc = 0; for kk: acc += (row[kk] as f32) * b[kk];  *o = acc * scale (scale = f16 -> f32). */
void oracle_matmul_i8_f32(const int8_t* a_i8, const uint16_t* a_scales_f16, size_t m, size_t k,
                          const float* b, float* out)
{
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < m; ++i) {
        const int8_t* row = a_i8 + i * k;
        float scale = oracle_f16_to_f32(a_scales_f16[i]);
        float acc = 0.0f;
        for (size_t kk = 0; kk < k; ++kk) acc += (float)row[kk] * b[kk];
        out[i] = acc * scale;
    }
}

/* Batched form of the int8 GEMV for M activation rows and the config dtypes: the scale
 * (f32/f16/bf16) and x (f32/f16) are widened exactly to f32, then each output
 * y[mi, n] is the reference row GEMV above on activation row mi.
 * This is what the reference computes when called once per row (one session
 * at a time, crates/cellm-sdk/src/lib.rs:622-680). */
void oracle_qgemv_i8(const int8_t* w, const void* scales, int scale_dtype, const void* x, int x_dtype,
                     size_t M, size_t N, size_t K, float* y)
{
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            const int8_t* row = w + n * K;
            float scale = load_as_f32(scales, scale_dtype, n);
            float acc = 0.0f;
            for (size_t kk = 0; kk < K; ++kk) acc += (float)row[kk] * load_as_f32(x, x_dtype, mi * K + kk);
            y[mi * N + n] = acc * scale;
        }
    }
}

/* Llama CPU lm_head over i8 weights (crates/cellm-model/src/llama.rs:602-643):
 * serial over vocab, scale applied per element: acc += x[i] * ((w as f32) * scale);
 * non-finite -> -inf. */
void oracle_llama_lm_head_i8(const float* x, const int8_t* w, const uint16_t* scales_f16, size_t vocab,
                             size_t hidden, float* out)
{
    for (size_t vid = 0; vid < vocab; ++vid) {
        const int8_t* row = w + vid * hidden;
        float scale = oracle_f16_to_f32(scales_f16[vid]);
        float acc = 0.0f;
        for (size_t i = 0; i < hidden; ++i) acc += x[i] * ((float)row[i] * scale);
        if (!isfinite(acc)) acc = -INFINITY;
        out[vid] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* cellm symmetric i4 (u8 bytes, low nibble = even element).                */
/* ------------------------------------------------------------------------ */

/* LlamaRunner::embed_token (crates/cellm-model/src/llama.rs:676-726), one
 * row per token, t = token % vocab (:684):
 *   "f16": out[i] = f16::from_bits(row[i]).to_f32()                (:687-693)
 *   "i8":  out[i] = (row[i] as f32) * scale[t]                      (:694-702)
 *   "i4":  out[i] = ((nibble as i8 - 8) as f32) * scale[t], low nibble even,
 *          ceil(hidden/2) bytes per row                              (:703-718) */
void oracle_embed(int kind, const uint32_t* tokens, size_t rows, const void* w, const uint16_t* scales_f16,
                  size_t vocab, size_t hidden, float* out)
{
    for (size_t r = 0; r < rows; ++r) {
        const size_t t = (size_t)tokens[r] % vocab;
        float* o = out + r * hidden;
        if (kind == 0) {
            const uint16_t* row = (const uint16_t*)w + t * hidden;
            for (size_t i = 0; i < hidden; ++i) o[i] = oracle_f16_to_f32(row[i]);
        } else if (kind == 1) {
            const int8_t* row = (const int8_t*)w + t * hidden;
            const float scale = oracle_f16_to_f32(scales_f16[t]);
            for (size_t i = 0; i < hidden; ++i) o[i] = (float)row[i] * scale;
        } else {
            const size_t stride = (hidden + 1) / 2;
            const uint8_t* row = (const uint8_t*)w + t * stride;
            const float scale = oracle_f16_to_f32(scales_f16[t]);
            for (size_t i = 0; i < hidden; ++i) {
                const uint8_t b = row[i / 2];
                const int v = (i % 2 == 0) ? (int)(b & 0x0F) - 8 : (int)(b >> 4) - 8;
                o[i] = (float)v * scale;
            }
        }
    }
}

/* The CPU lm_head loop of LlamaRunner::step_inner for an f16 or i4 source
 * (llama.rs:576-646; the i8 one is oracle_llama_lm_head_i8), serial over the
 * vocabulary, non-finite logits -> -inf (:641-643):
 *   f16: acc += x[i] * f16_to_f32(row[i])                           (:602-608)
 *   i4:  acc += x[i] * val * scale, left to right: (x[i] * val) * scale (:619-634) */
void oracle_llama_lm_head_f16_i4(int kind, const float* x, const void* w, const uint16_t* scales_f16, size_t vocab,
                                 size_t hidden, float* out)
{
    for (size_t vid = 0; vid < vocab; ++vid) {
        float acc = 0.0f;
        if (kind == 0) {
            const uint16_t* row = (const uint16_t*)w + vid * hidden;
            for (size_t i = 0; i < hidden; ++i) acc += x[i] * oracle_f16_to_f32(row[i]);
        } else {
            const size_t stride = (hidden + 1) / 2;
            const uint8_t* row = (const uint8_t*)w + vid * stride;
            const float scale = oracle_f16_to_f32(scales_f16[vid]);
            for (size_t i = 0; i < hidden; ++i) {
                const uint8_t b = row[i / 2];
                const float val = (float)((i % 2 == 0) ? (int)(b & 0x0F) - 8 : (int)(b >> 4) - 8);
                acc += x[i] * val * scale;
            }
        }
        if (!isfinite(acc)) acc = -INFINITY;
        out[vid] = acc;
    }
}

/* cpu_kernels::matmul_i4_f32 (cpu_kernels.rs:219-243):
 * row_stride = ceil(k/2), spr = len(scales)/m,
 * dot += (q as f32) * scale * b[j]   i.e. ((q*scale)*x) then add. */
void oracle_matmul_i4_f32(const uint8_t* a_i4, const uint16_t* a_scales_f16, size_t n_scales, size_t m,
                          size_t k, size_t gs, const float* b, float* out)
{
    size_t row_stride = (k + 1) / 2;
    size_t spr = n_scales / m;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < m; ++i) {
        const uint8_t* row = a_i4 + i * row_stride;
        const uint16_t* rs = a_scales_f16 + i * spr;
        float dot = 0.0f;
        for (size_t j = 0; j < k; ++j) {
            uint8_t byte = row[j / 2];
            uint8_t nib = (j % 2 == 0) ? (byte & 0xf) : (byte >> 4);
            int q = (int)(int8_t)nib - 8;
            float scale = oracle_f16_to_f32(rs[j / gs]);
            dot += ((float)q * scale) * b[j];
        }
        out[i] = dot;
    }
}

/* Batched/dtype form of the symmetric i4 GEMV: x widened from f32/f16, M activation rows. */
void oracle_qgemv_i4_sym(const uint8_t* w, const uint16_t* scales_f16, size_t n_scales, size_t gs,
                         const void* x, int x_dtype, size_t M, size_t N, size_t K, float* y)
{
    size_t row_stride = (K + 1) / 2;
    size_t spr = n_scales / N;
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            const uint8_t* row = w + n * row_stride;
            const uint16_t* rs = scales_f16 + n * spr;
            float dot = 0.0f;
            for (size_t j = 0; j < K; ++j) {
                uint8_t byte = row[j / 2];
                uint8_t nib = (j % 2 == 0) ? (byte & 0xf) : (byte >> 4);
                int q = (int)nib - 8;
                float scale = oracle_f16_to_f32(rs[j / gs]);
                dot += ((float)q * scale) * load_as_f32(x, x_dtype, mi * K + j);
            }
            y[mi * N + n] = dot;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Rank-4 dtypes: f16 weights, i2 (2-bit per-row symmetric), q1_0_g128.      */
/* ------------------------------------------------------------------------ */

/* cpu_kernels::matmul_f16_f32, x86 branch (cpu_kernels.rs:135-214, :205-211):
 * acc += f32(w[kk]) * b[kk], sequential, product and sum rounded apart.
 * Batched/dtype form: x [M][K] widened from f32/f16/bf16, y [M][N]. */
void oracle_qgemv_f16(const uint16_t* w, const void* x, int x_dtype, size_t M, size_t N, size_t K, float* y)
{
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            const uint16_t* row = w + n * K;
            float acc = 0.0f;
            for (size_t kk = 0; kk < K; ++kk) {
                const float p = oracle_f16_to_f32(row[kk]) * load_as_f32(x, x_dtype, mi * K + kk);
                acc = acc + p;
            }
            y[mi * N + n] = acc;
        }
    }
}

/* dequant_i2 (qwen.rs:1582-1589, gemma.rs:2220-2227): 2-bit code -> centroid. */
static inline float i2_centroid(unsigned q)
{
    switch (q & 3u) {
    case 0: return -1.5f;
    case 1: return -0.5f;
    case 2: return 0.5f;
    default: return 1.5f;
    }
}

/* i2 row GEMV, row_stride = ceil(K/4) bytes, element j = bits 2(j%4)..+1 of
 * byte j/4 (low bits first), one f16 scale per row (".qscale").
 * scale_mode 0: Qwen dot_i2_scaled_row (qwen.rs:1591-1606, used by the linear
 *   fallback qwen.rs:1092-1101): acc += x * dq; result acc * scale.
 * scale_mode 1: Gemma dot_i2_scaled_row (gemma.rs:1673-1687):
 *   acc += x * (dq * scale). */
void oracle_qgemv_i2(const uint8_t* w, const uint16_t* scales_f16, int scale_mode, const void* x, int x_dtype,
                     size_t M, size_t N, size_t K, float* y)
{
    const size_t row_stride = (K + 3) / 4;
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            const uint8_t* row = w + n * row_stride;
            const float scale = oracle_f16_to_f32(scales_f16[n]);
            float acc = 0.0f;
            for (size_t j = 0; j < K; ++j) {
                const float dq = i2_centroid((unsigned)(row[j / 4] >> (2 * (j % 4))));
                const float xv = load_as_f32(x, x_dtype, mi * K + j);
                if (scale_mode == 0) {
                    const float p = xv * dq;
                    acc = acc + p;
                } else {
                    const float wv = dq * scale;
                    const float p = xv * wv;
                    acc = acc + p;
                }
            }
            y[mi * N + n] = scale_mode == 0 ? acc * scale : acc;
        }
    }
}

/* q1_0_g128 row GEMV (qwen.rs:1004-1022; metal.rs:542-570 mv_q1_0_g128):
 * a row is K/128 blocks of 18 bytes: f16 d (little endian) then 16 bytes of
 * sign bits, element b*8+j of the block = bit j of byte b; value d if the bit
 * is set, else -d; acc += value * x, sequential.  K % 128 == 0. */
void oracle_qgemv_q1_0_g128(const uint8_t* w, const void* x, int x_dtype, size_t M, size_t N, size_t K, float* y)
{
    const size_t nblk = K / 128, row_stride = nblk * 18;
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            const uint8_t* row = w + n * row_stride;
            float acc = 0.0f;
            for (size_t i = 0; i < nblk; ++i) {
                const uint8_t* blk = row + i * 18;
                const float d = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                for (int b = 0; b < 16; ++b)
                    for (int j = 0; j < 8; ++j) {
                        const float v = (blk[2 + b] >> j) & 1 ? d : -d;
                        const float p = v * load_as_f32(x, x_dtype, mi * K + i * 128 + (size_t)b * 8 + j);
                        acc = acc + p;
                    }
            }
            y[mi * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* MLX 4-bit affine (u32 words, 8 nibbles, per-64-group scale+bias).        */
/* ------------------------------------------------------------------------ */

/* Dequant of LfmRunner::linear_i4_out_in (crates/cellm-model/src/lfm.rs:1006-1025):
 * G = 64 in the reference (the parameter generalises it), gpr = ceil(K/G), P = K/8,
 * w[n, 8p+k] = ((Wq[n*P+p] >> 4k) & 0xF) as f32 * S[n*gpr + (8p)/64] + B[...]
 * (separate mul then add).  Elements past 8*P (K not a multiple of 8) stay 0,
 * as the reference's zero-initialised buffer leaves them. */
void oracle_q4_affine_dequant_f32(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                                  size_t N, size_t K, size_t G, float* out)
{
    size_t gpr = (K + G - 1) / G;
    size_t P = K / 8;
#pragma omp parallel for schedule(static)
    for (size_t n = 0; n < N; ++n) {
        float* row = out + n * K;
        for (size_t j = 0; j < K; ++j) row[j] = 0.0f;
        for (size_t p = 0; p < P; ++p) {
            uint32_t packed = wq[n * P + p];
            size_t g = (p * 8) / G;
            float scale = load_as_f32(scales, sb_dtype, n * gpr + g);
            float bias = load_as_f32(biases, sb_dtype, n * gpr + g);
            for (size_t k = 0; k < 8; ++k) {
                float nib = (float)((packed >> (k * 4)) & 0xFu);
                row[p * 8 + k] = nib * scale + bias;
            }
        }
    }
}

/* Full affine GEMV: dequant as above, then the cached-f32 dot
 * (lfm.rs:1056-1063): acc += w[j] * x[j], j ascending.
 * The affine lm_head ( lfm.rs:715-737) evaluates the same per-element
 * formula q*s+b and the same ascending-j sum, so it yields identical bits. */
void oracle_qgemv_q4_affine(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                            const void* x, int x_dtype, size_t M, size_t N, size_t K, size_t G, float* y)
{
    size_t gpr = (K + G - 1) / G;
    size_t P = K / 8;
    for (size_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for schedule(static)
        for (size_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (size_t j = 0; j < K; ++j) {
                float w = 0.0f;
                size_t p = j / 8;
                if (p < P) {
                    uint32_t packed = wq[n * P + p];
                    size_t g = (p * 8) / G;
                    float scale = load_as_f32(scales, sb_dtype, n * gpr + g);
                    float bias = load_as_f32(biases, sb_dtype, n * gpr + g);
                    float nib = (float)((packed >> ((j % 8) * 4)) & 0xFu);
                    w = nib * scale + bias;
                }
                acc += w * load_as_f32(x, x_dtype, mi * K + j);
            }
            y[mi * N + n] = acc;
        }
    }
}

/* The affine lm_head as written in the reference (lfm.rs:700-741): group loop, j loop, the
 * on-the-fly dequant and out-of-range defaults (scale 1.0, bias 0.0).  Kept
 * separate so a test can show it equals oracle_qgemv_q4_affine bit for bit. */
void oracle_lfm_lm_head_q4_affine(const uint32_t* wq, size_t nwords, const float* scales, const float* biases,
                                  size_t nsb, const float* x, size_t vocab, size_t hidden, float* out)
{
    const size_t group_size = 64;
    size_t groups_per_row = (hidden + group_size - 1) / group_size;
    size_t packed_in = hidden / 8;
#pragma omp parallel for schedule(static)
    for (size_t vocab_idx = 0; vocab_idx < vocab; ++vocab_idx) {
        size_t row_offset = vocab_idx * packed_in;
        float acc = 0.0f;
        for (size_t g = 0; g < groups_per_row; ++g) {
            size_t g_start = g * group_size;
            size_t g_end = (g + 1) * group_size < hidden ? (g + 1) * group_size : hidden;
            size_t scale_idx = vocab_idx * groups_per_row + g;
            float scale = scale_idx < nsb ? scales[scale_idx] : 1.0f;
            float bias = scale_idx < nsb ? biases[scale_idx] : 0.0f;
            for (size_t j = g_start; j < g_end; ++j) {
                size_t packed_idx = row_offset + (j / 8);
                size_t nibble_pos = j % 8;
                if (packed_idx < nwords) {
                    uint32_t packed = wq[packed_idx];
                    int nibble = (int)((packed >> (nibble_pos * 4)) & 0xF);
                    float q = (float)nibble;
                    float w = q * scale + bias;
                    acc += w * x[j];
                }
            }
        }
        out[vocab_idx] = acc;
    }
}

/* dequant_u32_affine_to_f16 (tools/convert/src/main.rs:4349-4444):
 * in_dim = packed_in*8, groups = ceil(in_dim/gs), g = min(i/gs, groups-1),
 * fp = (q as f32) * scale + bias (two roundings), h = f16::from_f32(fp) (RNE). */
void oracle_dequant_q4_affine_f16(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                                  size_t N, size_t K, size_t gs, uint16_t* out)
{
    size_t packed_in = K / 8;
    size_t in_dim = packed_in * 8;
    size_t groups = (in_dim + gs - 1) / gs;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < N; ++r) {
        for (size_t i = 0; i < in_dim; ++i) {
            uint32_t word = wq[r * packed_in + i / 8];
            uint32_t q = (word >> ((i % 8) * 4)) & 0xFu;
            size_t g = i / gs;
            if (g > groups - 1) g = groups - 1;
            float scale = load_as_f32(scales, sb_dtype, r * groups + g);
            float bias = load_as_f32(biases, sb_dtype, r * groups + g);
            float fp = (float)q * scale + bias;
            out[r * in_dim + i] = oracle_f32_to_f16(fp);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* dense f32 matmul (cpu_kernels.rs:36-63).                                 */
/* ------------------------------------------------------------------------ */

/* n == 1: row dot; else out[i, j] += a[i,k] * b[k,j] in i-k-j order.  The
 * reference uses `+=`, so the caller zeroes `out` first; this restatement
 * does not zero it either. */
void oracle_matmul_f32(const float* a, size_t m, size_t k, const float* b, size_t n, float* out)
{
    if (n == 1) {
#pragma omp parallel for schedule(static)
        for (size_t i = 0; i < m; ++i) {
            const float* row = a + i * k;
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; ++kk) acc += row[kk] * b[kk];
            out[i] = acc;
        }
    } else {
#pragma omp parallel for schedule(static)
        for (size_t i = 0; i < m; ++i) {
            const float* a_row = a + i * k;
            float* out_row = out + i * n;
            for (size_t kk = 0; kk < k; ++kk) {
                float av = a_row[kk];
                const float* b_row = b + kk * n;
                for (size_t j = 0; j < n; ++j) out_row[j] += av * b_row[j];
            }
        }
    }
}

/* Prefill reference for the qGEMM: Y[M,N] = X[M,K] . dequant(W)^T, each
 * element summed over k ascending from zero (the dense matmul over the affine f32 or f16 dequant).
 * w_f32 is the dequantized weight [N,K] (row-major out x in); x widened from
 * f32/f16.  The per-element order equals the dense matmul's i-k-j loop with a zeroed out. */
void oracle_gemm_xwT_f32(const void* x, int x_dtype, const float* w_f32, size_t M, size_t N, size_t K, float* y)
{
#pragma omp parallel for schedule(static)
    for (size_t mi = 0; mi < M; ++mi) {
        for (size_t n = 0; n < N; ++n) {
            const float* row = w_f32 + n * K;
            float acc = 0.0f;
            for (size_t kk = 0; kk < K; ++kk) acc += load_as_f32(x, x_dtype, mi * K + kk) * row[kk];
            y[mi * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* pieces of LlamaRunner::step_inner used around the projections.           */
/* ------------------------------------------------------------------------ */

/* rms_norm_f32 (cpu_kernels.rs:17-34). */
void oracle_rms_norm_f32(const float* x, const float* weight, size_t n, float eps, float* out)
{
    float mean_sq = 0.0f;
    for (size_t i = 0; i < n; ++i) mean_sq += x[i] * x[i];
    mean_sq /= (float)n;
    float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv_rms * weight[i];
}

/* rope_non_interleaved_inplace_f32 (cpu_kernels.rs:264-277), rotary_dim = head_dim. */
void oracle_rope_half_f32(float* x, size_t n_heads, size_t head_dim, size_t pos, float theta)
{
    size_t half = head_dim / 2;
    for (size_t h = 0; h < n_heads; ++h) {
        float* head = x + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            float inv_freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
            float angle = (float)pos * inv_freq;
            float s = sinf(angle), c = cosf(angle);
            float x0 = head[i];
            float x1 = head[half + i];
            head[i] = x0 * c - x1 * s;
            head[half + i] = x1 * c + x0 * s;
        }
    }
}

/* rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292): the pairs (2i, 2i + 1)
 * of each head, with the angle of pair i as in the rotate-half form above. */
void oracle_rope_interleaved_f32(float* x, size_t n_heads, size_t head_dim, size_t pos, float theta)
{
    size_t half = head_dim / 2;
    for (size_t h = 0; h < n_heads; ++h) {
        float* head = x + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            float inv_freq = powf(theta, -(2.0f * (float)i) / (float)head_dim);
            float angle = (float)pos * inv_freq;
            float s = sinf(angle), c = cosf(angle);
            float x0 = head[2 * i];
            float x1 = head[2 * i + 1];
            head[2 * i] = x0 * c - x1 * s;
            head[2 * i + 1] = x1 * c + x0 * s;
        }
    }
}

/* softmax_f32_inplace_cpu_local (crates/cellm-cache/src/kvcache.rs:1206-1227). */
void oracle_softmax_f32(float* x, size_t n)
{
    if (n == 0) return;
    float max_v = -INFINITY;
    for (size_t i = 0; i < n; ++i) if (x[i] > max_v) max_v = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) { x[i] = expf(x[i] - max_v); sum += x[i]; }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (size_t i = 0; i < n; ++i) x[i] *= inv;
    }
}

/* CpuKvStorage::attention_single_token_gqa_f32 (kvcache.rs:710-789) over f16
 * K/V rows addressed by per-token element bases (KvCacheLayout::token_base_elem,
 * crates/cellm-core/src/kv_cache.rs:62-73).  `scores` is scratch of length seq.
 * attn_scale: Some(s) when > 0, else None = 1/sqrt(head_dim) (:752);
 * soft_cap: Some(c) when > 0, s = tanh(s / c) * c per score (:768-770). */
void oracle_attention_gqa_f16kv(const uint16_t* kcache, const uint16_t* vcache, const size_t* bases, size_t seq,
                                const float* q, size_t n_heads, size_t n_kv_heads, size_t head_dim, float attn_scale,
                                float soft_cap, float* scores, float* out)
{
    for (size_t i = 0; i < n_heads * head_dim; ++i) out[i] = 0.0f;
    if (seq == 0) return;
    float scale = attn_scale > 0.0f ? attn_scale : 1.0f / sqrtf((float)head_dim);
    size_t group_size = n_heads / n_kv_heads;
    if (group_size < 1) group_size = 1;
    for (size_t h = 0; h < n_heads; ++h) {
        size_t kv_h = h / group_size;
        if (kv_h > n_kv_heads - 1) kv_h = n_kv_heads - 1;
        const float* qh = q + h * head_dim;
        for (size_t t = 0; t < seq; ++t) {
            const uint16_t* kt = kcache + bases[t] + kv_h * head_dim;
            float dot = 0.0f;
            for (size_t i = 0; i < head_dim; ++i) dot += qh[i] * oracle_f16_to_f32(kt[i]);
            float sc = dot * scale;
            if (soft_cap > 0.0f) sc = tanhf(sc / soft_cap) * soft_cap;
            scores[t] = sc;
        }
        oracle_softmax_f32(scores, seq);
        float* out_h = out + h * head_dim;
        for (size_t t = 0; t < seq; ++t) {
            const uint16_t* vt = vcache + bases[t] + kv_h * head_dim;
            float w = scores[t];
            for (size_t i = 0; i < head_dim; ++i) out_h[i] += w * oracle_f16_to_f32(vt[i]);
        }
    }
}

/* SiLU(gate) * up in place on gate (llama.rs:477-484). */
void oracle_silu_mul_f32(float* gate, const float* up, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i];
        float s = 1.0f / (1.0f + expf(-g));
        gate[i] = g * s;
    }
    for (size_t i = 0; i < n; ++i) gate[i] *= up[i];
}

/* gelu_tanh_f32 (crates/cellm-model/src/gemma.rs:1689-1693) times up, in place on
 * gate, as the Gemma MLP loop (gemma.rs:844-846): k = 0.797_884_6f32,
 * c = 0.044_715f32, 0.5 * x * (1 + tanh(k * (x + c * x * x * x))) with Rust's
 * left-to-right products, then * up[i]. */
void oracle_gelu_tanh_mul_f32(float* gate, const float* up, size_t n)
{
    const float k = 0.7978846f;
    const float c = 0.044715f;
    for (size_t i = 0; i < n; ++i) {
        float x = gate[i];
        float g = 0.5f * x * (1.0f + tanhf(k * (x + c * x * x * x)));
        gate[i] = g * up[i];
    }
}

/* topk_from_logits(..)[0] for top_k = 1 (llama.rs:1049-1078): first index of
 * the maximum (a later equal value does not replace the kept one). */
int64_t oracle_argmax_first(const float* logits, size_t n)
{
    if (n == 0) return -1;
    size_t best = 0;
    float min_val = logits[0];
    for (size_t v = 1; v < n; ++v) {
        if (logits[v] > min_val) { best = v; min_val = logits[v]; }
    }
    return (int64_t)best;
}
