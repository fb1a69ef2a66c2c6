/*
 * cellm_hip.h -- C ABI of the MI355X (gfx950) quantized-weight matmul library.
 *
 * This is the drop-in boundary for cellm's quantized projection path: a Rust
 * `HipOps` (the sibling of `MetalOps`, crates/cellm-kernels/src/metal.rs:637-661)
 * binds these functions one-to-one and a `BackendKind::Hip` selects it.
 * Each declaration cites the reference interface it replaces.
 *
 * Conventions (mirroring crates/cellm-sdk/include/cellm.h:19-26 and ffi.rs:21-52):
 *   - every function returns int32_t: 0 (CELLM_HIP_OK) on success, < 0 on error;
 *   - on error a message is stored per calling thread and read with
 *     cellm_hip_last_error_message();
 *   - no CPU fallback exists: an entry point either runs on the GPU or fails.
 *
 * Layouts (all row-major, "HF linear weight: [out, in]", llama.rs:770-776):
 *   int8:       W [n, k] int8; scales [n] (per row) or [1] (per tensor)
 *   q4 affine:  Wq [n, k/8] uint32, nibble j of word p = element 8p+j;
 *               scales, biases [n, ceil(k/group)] ; w = q*scale + bias
 *   i4 sym:     W [n, ceil(k/2)] uint8, low nibble = even element;
 *               scales f16 [n * spr], spr = n_scales / n, w = (nib-8)*scale[j/gs]
 *   x [m, k], y [m, n] (f32).
 *
 * Async entry points take device pointers and a stream (a hipStream_t passed
 * as void*; NULL is HIP's default stream, as in the HIP API) and return as
 * soon as the work is queued, like MetalOps::encode_* (metal.rs:813-1176).
 * The context's own stream (cellm_hip_get_stream) serves the sync calls.  Sync entry
 * points take host pointers, cache the weights on the device under a name
 * key, and return after the result is back in host memory, like
 * MetalOps::logits_* (metal.rs:1017-1204).
 */
#ifndef CELLM_HIP_H
#define CELLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CELLM_HIP_OK 0
#define CELLM_HIP_ERR_INVALID_ARG (-1)
#define CELLM_HIP_ERR_DEVICE (-2)
#define CELLM_HIP_ERR_OUT_OF_MEMORY (-3)
#define CELLM_HIP_ERR_NOT_FOUND (-4)
#define CELLM_HIP_ERR_UNSUPPORTED (-5)

/* Element type of scales, biases and activations. */
typedef enum {
    CELLM_HIP_DTYPE_F32 = 0,
    CELLM_HIP_DTYPE_F16 = 1,
    CELLM_HIP_DTYPE_BF16 = 2
} cellm_hip_dtype_t;

typedef struct cellm_hip_ctx cellm_hip_ctx_t;

/* ---- errors, devices, lifetime ------------------------------------------ */

/* Takes the calling thread's last error message: copies it NUL-terminated,
 * truncated to buf_len - 1 bytes, clears it, and returns the number of bytes
 * written (excluding the NUL).  A NULL buffer or buf_len 0 returns 0 and
 * leaves the message.  Replaces cellm_last_error_message
 * (crates/cellm-sdk/include/cellm.h:24-26, crates/cellm-sdk/src/ffi.rs:126-138);
 * the message is per thread, as cellm.h documents.  Every entry point catches
 * C++ exceptions and reports them as error codes (ffi.rs:142 catches panics). */
size_t cellm_hip_last_error_message(char* buf, size_t buf_len);

/* Number of visible HIP devices. */
int32_t cellm_hip_device_count(int32_t* out_count);

/* Launches out = a + b on `device` and checks the result on the host.
 * Replaces MetalKernels::smoke_test_add_f32 (metal.rs:33-93), the probe that
 * select_backend runs (tools/infer/src/main.rs:591-615). */
int32_t cellm_hip_smoke_test(int32_t device);

/* Creates a context bound to `device`: an owned stream, a name-keyed device
 * weight cache and scratch buffers.  Replaces MetalOps::create (metal.rs:705-746). */
int32_t cellm_hip_create(int32_t device, cellm_hip_ctx_t** out_ctx);

/* Frees every cached weight and scratch buffer, then the context. */
void cellm_hip_destroy(cellm_hip_ctx_t* ctx);

/* Waits for all work queued on the context's own stream. */
int32_t cellm_hip_synchronize(cellm_hip_ctx_t* ctx);

/* Returns the context's own stream (a hipStream_t) in *out_stream. */
int32_t cellm_hip_get_stream(cellm_hip_ctx_t* ctx, void** out_stream);

/* ---- device weight cache (MetalOps::tensor_cache, metal.rs:660,1045-1050) - */

/* Uploads `nbytes` from host memory once under `key`; a second upload of the
 * same key returns the existing buffer.  *out_dev receives the device pointer
 * (256-byte aligned), owned by the context. */
int32_t cellm_hip_weight_upload(cellm_hip_ctx_t* ctx, const char* key, const void* host, size_t nbytes,
                                const void** out_dev);

/* Looks up a cached weight; CELLM_HIP_ERR_NOT_FOUND if absent. */
int32_t cellm_hip_weight_lookup(cellm_hip_ctx_t* ctx, const char* key, const void** out_dev, size_t* out_nbytes);

/* Frees one cached weight; CELLM_HIP_ERR_NOT_FOUND if absent. */
int32_t cellm_hip_weight_evict(cellm_hip_ctx_t* ctx, const char* key);

/* Number of cached weights and their total bytes. */
int32_t cellm_hip_weight_cache_stats(cellm_hip_ctx_t* ctx, size_t* out_entries, size_t* out_bytes);

/* ---- async entry points (device pointers) ------------------------------- */

/* int8 per-row-scaled GEMV / GEMM:
 *   y[i, r] = (sum_j W[r, j] * x[i, j]) * scale[per_row ? r : 0]  (+ bias[r] if bias != NULL)
 * scale applied after the sum as in cpu_kernels::matmul_i8_f32
 * (crates/cellm-kernels/src/cpu_kernels.rs:66-133); per-row scales when
 * n_scales >= n, as MetalOps::encode_mv_i8_bias decides (metal.rs:891-904),
 * one per-tensor scale when n_scales == 1; other counts are refused
 * (CELLM_HIP_ERR_INVALID_ARG), where the reference would use scale[0].
 * scale_dtype: F32/F16/BF16; x_dtype: F32/F16/BF16.  m <= 4 runs the decode
 * GEMV; larger m with f16 x and k % 64 == 0 runs the MFMA GEMM.  With few
 * output rows over a long k, 2..64 rows split k over work items whose partial
 * sums go to the context's per-stream workspace (grown on demand, as for the
 * split-K qGEMM) and a second kernel adds them in a fixed order.  f32 x at
 * 3..4 rows over a long output (n >= 32768, n % 16 == 0, k % 64 == 0,
 * 128 <= k <= 1024, 16-byte aligned w and x: a multi-session lm_head) runs on
 * int8 MFMA: each x row becomes x' = rint(x * 2^e) with |x'| <= 2^20 for the
 * row's power of two, split into three signed 8-bit digits; the integer sums
 * over k are exact and the row scale follows them, so x keeps 2^-20 of its
 * row's largest |x| (within 3e-5 normwise of the f32 reference order). */
int32_t cellm_hip_qgemv_i8(cellm_hip_ctx_t* ctx, const int8_t* w, const void* scales, int32_t scale_dtype,
                           int64_t n_scales, const void* x, int32_t x_dtype, const float* bias, float* y, int64_t m,
                           int64_t n, int64_t k, void* stream);

/* MLX 4-bit affine GEMV / GEMM:
 *   y[i, r] = sum_j (q[r, j] * S[r, j/group] + B[r, j/group]) * x[i, j]
 * Replaces LfmRunner::linear_i4_out_in (crates/cellm-model/src/lfm.rs:985-1066)
 * and its dequant -> MetalOps::logits_f32 route (lfm.rs:1049-1054).
 * k % 8 == 0; group a power of two >= 8 (MLX uses 64).  2..64 rows with f16 x
 * run the batched MFMA path, split over k through the per-stream workspace
 * for few output rows over a long k, as cellm_hip_qgemv_i8.
 * f32 x (m <= 4) with f32 scales and biases runs an f32 dot (x kept in f32,
 * the nibbles widened exactly).  With f16/bf16 scales it is multiplied as two
 * f16 parts, hi = RNE_f16(x') and lo = RNE_f16(x' - hi), of each 32-element
 * chunk scaled by a power of two x' = x * 2^e that puts the chunk's largest
 * |x| in [2^13, 2^14): any finite f32 x keeps about 22 bits, and the result is
 * scaled back exactly.  The split holds for the fused gate/up and QKV entry
 * points below too.  Long outputs
 * (n >= 32768, n % 16 == 0, k % 128 == 0, k <= 1024, group 64, 16-byte
 * aligned wq and x: the affine lm_head) run on int8 MFMA instead: each row
 * is rounded to integers x' = rint(x * 2^e) with |x'| <= 2^20 for the row's
 * largest |x|, split into three signed 8-bit digits, and summed exactly per
 * group; x keeps 2^-20 of its row's largest value, scaled back exactly. */
int32_t cellm_hip_qgemv_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                  int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype, float* y,
                                  int64_t m, int64_t n, int64_t k, void* stream);

/* Fused QKV, one launch for m <= 4 (f16/f32 x, cols % 16 == 0, 16-byte
 * aligned W and x; other shapes run three cellm_hip_qgemv_i8 launches):
 *   q = (Wq . x) * sq (+ bq), k and v likewise with rows_kv rows each.
 * Each projection has its own scales (per row when n_s >= rows, per tensor when n_s == 1)
 * and optional bias (NULL = none); all scales share scale_dtype.  Replaces
 * MetalOps::encode_qkv_i8 / encode_qkv_i8_bias (crates/cellm-kernels/src/metal.rs:923-945,
 * 1153-1160; kernel mv_qkv_i8 metal.rs:387-439). */
int32_t cellm_hip_qgemv_i8_qkv(cellm_hip_ctx_t* ctx, const int8_t* wq, const void* sq, int64_t n_sq, const float* bq,
                               const int8_t* wk, const void* sk, int64_t n_sk, const float* bk, const int8_t* wv,
                               const void* sv, int64_t n_sv, const float* bv, int32_t scale_dtype, const void* x,
                               int32_t x_dtype, float* q, float* k_out, float* v, int64_t m, int64_t rows_q,
                               int64_t rows_kv, int64_t cols, void* stream);

/* The q, k and v projections of MLX 4-bit affine weights sharing x, in one
 * launch for m <= 4 (f16 or f32 x, cols % 32 == 0, group >= 32, 16-byte
 * aligned x and W); other shapes run one GEMV per projection.  sq/bq ... are
 * each matrix's scales and group biases in sb_dtype (cellm_hip_qgemv_q4_affine);
 * biasq/biask/biasv (f32 [rows], or NULL) are added after each row sum, as
 * add_projection_bias_if_present does (qwen.rs:1132-1139).  No reference
 * counterpart as one call: the u32 runners call linear_f16_out_in once per
 * projection (lfm.rs:924-981); this is the q4 form of
 * cellm_hip_qgemv_i8_qkv. */
int32_t cellm_hip_qgemv_q4_affine_qkv(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* sq, const void* bq,
                                      const float* biasq, const uint32_t* wk, const void* sk, const void* bk,
                                      const float* biask, const uint32_t* wv, const void* sv, const void* bv,
                                      const float* biasv, int32_t sb_dtype, int64_t group, const void* x,
                                      int32_t x_dtype, float* q, float* k_out, float* v, int64_t m, int64_t rows_q,
                                      int64_t rows_kv, int64_t cols, void* stream);

/* Gate and up projections with the SiLU * up epilogue:
 *   h = silu((Wg . x) * sg (+ bg)) * ((Wu . x) * su (+ bu)),  silu(g) = g / (1 + exp(-g)).
 * One launch for m <= 4 under the conditions of cellm_hip_qgemv_i8_qkv; other
 * shapes run two GEMVs and an elementwise kernel.  Replaces the gate/up
 * encode_mv_i8(_bias) pair plus encode_silu_mul_f32_inplace of the decode
 * graphs (crates/cellm-model/src/llama_graph.rs:318-327,
 * crates/cellm-model/src/qwen.rs:1445-1453; metal.rs:235-245, 956), and the
 * CPU loop of llama.rs:477-484. */
int32_t cellm_hip_qgemv_i8_gate_up_silu(cellm_hip_ctx_t* ctx, const int8_t* wg, const void* sg, int64_t n_sg,
                                        const float* bg, const int8_t* wu, const void* su, int64_t n_su,
                                        const float* bu, int32_t scale_dtype, const void* x, int32_t x_dtype, float* h,
                                        int64_t m, int64_t n, int64_t k, void* stream);

/* The same for MLX 4-bit affine gate/up weights; sg/bg and su/bu are the affine
 * scales/biases of each matrix.  One launch computes both rows and the SiLU *
 * up for m <= 4 with f16 x, k % 32 == 0, group >= 32 and 16-byte aligned x,
 * wg and wu; other shapes run two cellm_hip_qgemv_q4_affine launches and the
 * SiLU * up kernel. */
int32_t cellm_hip_qgemv_q4_affine_gate_up_silu(cellm_hip_ctx_t* ctx, const uint32_t* wg, const void* sg,
                                               const void* bg, const uint32_t* wu, const void* su, const void* bu,
                                               int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype,
                                               float* h, int64_t m, int64_t n, int64_t k, void* stream);

/* Gemma's MLP activation in place of SiLU (crates/cellm-model/src/gemma.rs:844-846,
 * gemma_graph.rs:435-436):
 *   h = gelu_tanh(g) * u,  gelu_tanh(g) = 0.5 g (1 + tanh(0.7978846 (g + 0.044715 g^3)))
 * in the order of gelu_tanh_f32 (gemma.rs:1689-1693), g and u as in the SiLU
 * entry points above, with the same arguments, launch shapes and fallbacks. */
int32_t cellm_hip_qgemv_i8_gate_up_gelu(cellm_hip_ctx_t* ctx, const int8_t* wg, const void* sg, int64_t n_sg,
                                        const float* bg, const int8_t* wu, const void* su, int64_t n_su,
                                        const float* bu, int32_t scale_dtype, const void* x, int32_t x_dtype, float* h,
                                        int64_t m, int64_t n, int64_t k, void* stream);
int32_t cellm_hip_qgemv_q4_affine_gate_up_gelu(cellm_hip_ctx_t* ctx, const uint32_t* wg, const void* sg,
                                               const void* bg, const uint32_t* wu, const void* su, const void* bu,
                                               int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype,
                                               float* h, int64_t m, int64_t n, int64_t k, void* stream);

/* The same over symmetric i4 gate/up weights (gemma.rs:1446-1471 runs the i4
 * branch of linear_f16_out_in for each): two cellm_hip_qgemv_i4_sym launches
 * (arguments as there, one gs for both) and the GELU * up kernel. */
int32_t cellm_hip_qgemv_i4_gate_up_gelu(cellm_hip_ctx_t* ctx, const uint8_t* wg, const uint16_t* sg, int64_t n_sg,
                                        const uint8_t* wu, const uint16_t* su, int64_t n_su, int64_t gs,
                                        const void* x, int32_t x_dtype, float* h, int64_t m, int64_t n, int64_t k,
                                        void* stream);

/* One projection of a batch (cellm_hip_qgemv_batch).  kind
 * CELLM_HIP_OP_QGEMV_I8 takes the arguments of cellm_hip_qgemv_i8 (w int8,
 * scales, sb_dtype = scale dtype, n_scales, bias; biases and group unused);
 * kind CELLM_HIP_OP_QGEMV_Q4_AFFINE those of cellm_hip_qgemv_q4_affine (w =
 * u32 words, scales, biases, sb_dtype, group; n_scales and bias unused);
 * kind CELLM_HIP_OP_QGEMV_F16 those of cellm_hip_qgemv_f16 (w only);
 * kind CELLM_HIP_OP_QGEMV_I2 those of cellm_hip_qgemv_i2 (w, scales = f16 row
 * scales, group = scale_mode); kind CELLM_HIP_OP_QGEMV_Q1_0_G128 those of
 * cellm_hip_qgemv_q1_0_g128 (w only); kind CELLM_HIP_OP_QGEMV_I4_SYM those of
 * cellm_hip_qgemv_i4_sym (w bytes, scales = f16, n_scales, group = gs).
 * Unused fields are ignored. */
#define CELLM_HIP_OP_QGEMV_I8 0
#define CELLM_HIP_OP_QGEMV_Q4_AFFINE 1
#define CELLM_HIP_OP_QGEMV_F16 2
#define CELLM_HIP_OP_QGEMV_I2 3
#define CELLM_HIP_OP_QGEMV_Q1_0_G128 4
#define CELLM_HIP_OP_QGEMV_I4_SYM 5
typedef struct {
    int32_t kind;
    int32_t sb_dtype;
    int32_t x_dtype;
    int32_t group;
    const void* w;
    const void* scales;
    const void* biases;
    int64_t n_scales;
    const void* x;
    const float* bias;
    float* y;
    int64_t m;
    int64_t n;
    int64_t k;
} cellm_hip_qgemv_op_t;

/* Enqueues ops[0..n_ops) in order on one stream with one call, as the
 * reference's fused decode graphs encode consecutive projections on one Metal
 * command encoder (crates/cellm-model/src/llama_graph.rs:245-336: encode_qkv_i8,
 * encode_mv_i8 for o / gate / up / down).  Each op is checked and launched as
 * its single-op entry point does; the first failing op's status is returned
 * and the ops before it stay enqueued. */
int32_t cellm_hip_qgemv_batch(cellm_hip_ctx_t* ctx, const cellm_hip_qgemv_op_t* ops, int64_t n_ops, void* stream);

/* Symmetric i4 GEMV: y[i, r] = sum_j ((nib - 8) * scale[r*spr + j/gs]) * x[i, j],
 * spr = n_scales / n.  Replaces cpu_kernels::matmul_i4_f32 (cpu_kernels.rs:219-243)
 * and MetalOps::encode_mv_i4 (metal.rs:1167-1176). */
int32_t cellm_hip_qgemv_i4_sym(cellm_hip_ctx_t* ctx, const uint8_t* w, const uint16_t* scales_f16, int64_t n_scales,
                               int64_t gs, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k,
                               void* stream);

/* f16-weight GEMV: y[i, r] = sum_j f32(W[r, j]) * x[i, j], W [n][k] f16
 * (2-byte aligned).  Replaces cpu_kernels::matmul_f16_f32
 * (cpu_kernels.rs:135-214) in the runners' "f16" linear arms (qwen.rs:1073,
 * llama.rs:898) and MetalOps::encode_mv_f16 / mv_f16 (metal.rs:347-363,
 * 1089). */
int32_t cellm_hip_qgemv_f16(cellm_hip_ctx_t* ctx, const uint16_t* w_f16, const void* x, int32_t x_dtype, float* y,
                            int64_t m, int64_t n, int64_t k, void* stream);

/* i2 GEMV: W [n][ceil(k/4)] bytes, element j = bits 2(j%4)..2(j%4)+1 of byte
 * j/4, code c -> centroid {-1.5, -0.5, 0.5, 1.5}[c] (dequant_i2,
 * qwen.rs:1582-1589); one f16 scale per row.  scale_mode 0 applies the scale
 * to the row sum (Qwen dot_i2_scaled_row, qwen.rs:1591-1606); scale_mode 1
 * to each element (Gemma dot_i2_scaled_row, gemma.rs:1673-1687). */
int32_t cellm_hip_qgemv_i2(cellm_hip_ctx_t* ctx, const uint8_t* w, const uint16_t* scales_f16, int32_t scale_mode,
                           const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k, void* stream);

/* q1_0_g128 GEMV: each row is k/128 blocks of 18 bytes, a little-endian f16
 * d then 16 bytes of sign bits (element 8b+j = bit j of byte b; value d when
 * set, -d otherwise).  Replaces the "q1_0_g128" arm of Qwen's dot_row
 * (qwen.rs:1004-1022) and MetalOps::encode_mv_q1 / mv_q1_0_g128
 * (metal.rs:542-570).  k % 128 == 0. */
int32_t cellm_hip_qgemv_q1_0_g128(cellm_hip_ctx_t* ctx, const uint8_t* w, const void* x, int32_t x_dtype, float* y,
                                  int64_t m, int64_t n, int64_t k, void* stream);

/* Prefill qGEMM on MFMA: Y[m, n] = X[m, k] . dequant(Wq)^T, X f16, Y f32,
 * weight tiles dequantized to f16 as tools/convert/src/main.rs:4349-4444 does.
 * No reference counterpart (prefill is token-by-token, llama.rs:214-233);
 * its oracle is cpu_kernels::matmul_f32 (cpu_kernels.rs:36-63). k % 64 == 0. */
int32_t cellm_hip_qgemm_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                  int32_t sb_dtype, int64_t group, const uint16_t* x_f16, float* y, int64_t m,
                                  int64_t n, int64_t k, void* stream);

/* int8 qGEMM on MFMA (exact int8 -> f16 tiles, per-row scale in the epilogue). */
int32_t cellm_hip_qgemm_i8(cellm_hip_ctx_t* ctx, const int8_t* w, const void* scales, int32_t scale_dtype,
                           int64_t n_scales, const uint16_t* x_f16, const float* bias, float* y, int64_t m, int64_t n,
                           int64_t k, void* stream);

/* Bit-exact dequant of MLX affine weights to f32 (lfm.rs:1014-1025 rounding)
 * or f16 (RNE of the f32 value, tools/convert/src/main.rs:4430-4436). */
int32_t cellm_hip_dequant_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                    int32_t sb_dtype, int64_t group, void* out, int32_t out_dtype, int64_t n,
                                    int64_t k, void* stream);

/* ---- sync entry points (host pointers, weights cached by key) ----------- */

/* MetalOps::logits_i8 (metal.rs:1044-1066): x f32 [cols], w int8 [rows, cols],
 * scales f16 [rows], out f32 [rows]. */
int32_t cellm_hip_logits_i8(cellm_hip_ctx_t* ctx, const float* x, const int8_t* w, const uint16_t* scales_f16,
                            size_t rows, size_t cols, const char* cache_key, float* out);

/* MetalOps::logits_i4 (metal.rs:1178-1204) with the CPU reference's scale
 * indexing (spr = n_scales / rows, cpu_kernels.rs:228-229). */
int32_t cellm_hip_logits_i4(cellm_hip_ctx_t* ctx, const float* x, const uint8_t* w, const uint16_t* scales_f16,
                            size_t n_scales, size_t rows, size_t cols, size_t gs, const char* cache_key, float* out);

/* The LFM affine linear (lfm.rs:985-1066) without the f32 dequant cache:
 * x f32 [cols], Wq [rows, cols/8], scales/biases [rows, ceil(cols/64)]. */
int32_t cellm_hip_logits_q4_affine(cellm_hip_ctx_t* ctx, const float* x, const uint32_t* wq, const void* scales,
                                   const void* biases, int32_t sb_dtype, size_t rows, size_t cols,
                                   const char* cache_key, float* out);

/* ---- decode-step ops around the projections (async, device pointers) ----
 * The device side of the fused Metal decode graph
 * (crates/cellm-model/src/llama_graph.rs:140-405).  `rows` sessions, one
 * activation row each; `positions` is a device int32[rows]; a paged K/V cache
 * is an f16 array addressed as KvCacheLayout::token_base_elem
 * (crates/cellm-core/src/kv_cache.rs:62-73):
 *   base = block * (n_layers * tokens_per_block * kv_dim)
 *        + layer * (tokens_per_block * kv_dim) + (pos % tokens_per_block) * kv_dim
 * with block = block_tables[row * max_blocks + pos / tokens_per_block]
 * (device uint32).  Pages with block >= total_blocks are skipped. */

/* embed_token, i8 branch (crates/cellm-model/src/llama.rs:676-701):
 * out[r] = f32(embed_i8[t]) * f32(scales_f16[t]), t = tokens[r] % vocab. */
int32_t cellm_hip_embed_i8(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const int8_t* embed_i8,
                           const uint16_t* scales_f16, int64_t vocab, int64_t hidden, float* out, void* stream);

/* embed_token, f16 branch (llama.rs:687-693): out[r] = f32(embed_f16[t]),
 * t = tokens[r] % vocab (f16 bits [vocab, hidden]). */
int32_t cellm_hip_embed_f16(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const uint16_t* embed_f16,
                            int64_t vocab, int64_t hidden, float* out, void* stream);

/* embed_token, i4 branch (llama.rs:703-718): out[r][i] = f32(nibble - 8) *
 * f32(scales_f16[t]), rows of ceil(hidden / 2) bytes with element 2j in the low
 * nibble of byte j, t = tokens[r] % vocab. */
int32_t cellm_hip_embed_i4(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const uint8_t* embed_i4,
                           const uint16_t* scales_f16, int64_t vocab, int64_t hidden, float* out, void* stream);

/* MetalOps::encode_rms_norm_f16w (metal.rs) / rms_norm_f32 (cpu_kernels.rs:17-34)
 * per row: out = x * (1 / sqrt(mean(x^2) + eps)) * weight; weight f32/f16/bf16 [n]. */
int32_t cellm_hip_rms_norm(cellm_hip_ctx_t* ctx, const float* x, const void* weight, int32_t weight_dtype,
                           int64_t rows, int64_t n, float eps, float* out, void* stream);

/* The residual add of a sub-layer (x[i] += y[i], llama.rs:440 and :494)
 * followed by the next RMSNorm (cellm_hip_rms_norm) in one launch:
 * x += y in place, then out = rms_norm(x) * weight.  Same results as
 * cellm_hip_add_f32_inplace followed by cellm_hip_rms_norm. */
int32_t cellm_hip_add_rms_norm(cellm_hip_ctx_t* ctx, float* x, const float* y, const void* weight,
                               int32_t weight_dtype, int64_t rows, int64_t n, float eps, float* out, void* stream);

/* MetalOps::encode_rope_half_f32 with rotary_dim = head_dim
 * (rope_non_interleaved_inplace_f32, cpu_kernels.rs:264-277), in place on
 * x [rows][n_heads][head_dim].  cos_sin [table_positions][head_dim/2][2] holds
 * (cos, sin) of pos * theta^(-2i/head_dim), computed by the caller as the
 * reference does in f32; positions are clamped to the table. */
int32_t cellm_hip_rope_half_f32(cellm_hip_ctx_t* ctx, float* x, int64_t rows, int64_t n_heads, int64_t head_dim,
                                const int32_t* positions, const float* cos_sin, int64_t table_positions, void* stream);

/* rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292): the same rotation of
 * the pairs (2i, 2i + 1) of each head instead of (i, i + head_dim/2), with the
 * same table (the angle of pair i is pos * theta^(-2i/head_dim) in both). */
int32_t cellm_hip_rope_interleaved_f32(cellm_hip_ctx_t* ctx, float* x, int64_t rows, int64_t n_heads, int64_t head_dim,
                                       const int32_t* positions, const float* cos_sin, int64_t table_positions,
                                       void* stream);

/* The RoPE layout of the context's fused decode ops (cellm_hip_rope_kv_write_f16
 * and cellm_hip_decode_qkv_rope_kv): 0 rotate-half (the default), 1 interleaved.
 * The reference's Llama runner picks it once, from CELLM_LLAMA_ROPE_INTERLEAVED
 * (crates/cellm-model/src/llama.rs:80-82, used at :391-396). */
int32_t cellm_hip_set_rope_interleaved(cellm_hip_ctx_t* ctx, int32_t interleaved);

/* MetalKvStorage::encode_write_token_f32 / write_token_f32 (kvcache.rs:589-615):
 * k, v [rows][kv_dim] f32 -> f16 (RNE) at each row's position in `layer`. */
int32_t cellm_hip_kv_write_f16(cellm_hip_ctx_t* ctx, const float* k, const float* v, int64_t rows, int64_t kv_dim,
                               const int32_t* positions, uint16_t* kcache, uint16_t* vcache,
                               const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                               int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream);

/* The step's q/k rotation and K/V write in one launch
 * (llama_graph.rs:273-281 encodes them as three): RoPE in place on q
 * [rows][n_heads][head_dim] and k [rows][n_kv_heads][head_dim], then the
 * rotated k and v written as f16 at each row's position in `layer`.  Same
 * results as cellm_hip_rope_half_f32 on q and on k followed by
 * cellm_hip_kv_write_f16 (cellm_hip_rope_interleaved_f32 when the context's
 * layout is interleaved, cellm_hip_set_rope_interleaved). */
int32_t cellm_hip_rope_kv_write_f16(cellm_hip_ctx_t* ctx, float* q, float* k, const float* v, int64_t rows,
                                    int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const int32_t* positions,
                                    const float* cos_sin, int64_t table_positions, uint16_t* kcache, uint16_t* vcache,
                                    const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                                    int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream);

/* One launch for "residual add + input_layernorm, q/k/v projections, RoPE,
 * K/V write" of a decode layer (llama_graph.rs:245-292 encodes them as
 * separate dispatches): x_out = x_prev + y (y may be NULL: x_prev as is),
 * xn = rms_norm(x_out) * norm_w (f32 weights), q = RoPE(Wq xn) into q_out
 * [rows][n_heads][head_dim], k = RoPE(Wk xn) and v = Wv xn written as f16 at
 * each row's position in `layer` of the paged cache.  int8 weights [out][hidden]
 * with f16 row scales.  x_out must be a different buffer from x_prev and y.
 * rows 1..4, hidden % 16 == 0 and <= 4096; otherwise CELLM_HIP_ERR_UNSUPPORTED
 * (use the separate calls).  RoPE pairs follow cellm_hip_set_rope_interleaved. */
int32_t cellm_hip_decode_qkv_rope_kv(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out,
                                     const float* norm_w, float eps, const int8_t* wq, const uint16_t* sq,
                                     const int8_t* wk, const uint16_t* sk, const int8_t* wv, const uint16_t* sv,
                                     int64_t rows, int64_t hidden, int64_t n_heads, int64_t n_kv_heads,
                                     int64_t head_dim, const int32_t* positions, const float* cos_sin,
                                     int64_t table_positions, float* q_out, uint16_t* kcache, uint16_t* vcache,
                                     const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                                     int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream);

/* The same for "residual add + post_attention_layernorm, gate/up, SiLU * up"
 * (llama_graph.rs:310-327): x_out = x_prev + y, xn = rms_norm(x_out) * norm_w,
 * h [rows][inter] = silu(Wg xn) * (Wu xn).  Same limits as above. */
int32_t cellm_hip_decode_gate_up_silu(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out,
                                      const float* norm_w, float eps, const int8_t* wg, const uint16_t* sg,
                                      const int8_t* wu, const uint16_t* su, int64_t rows, int64_t hidden,
                                      int64_t inter, float* h, void* stream);

/* The two entry points above for MLX 4-bit affine weights (the u32 layers of
 * the Qwen2 decode step, qwen.rs:1355-1453: input_layernorm, the q/k/v
 * projections with their biases, RoPE and the K/V write; then
 * post_attention_layernorm, gate/up and SiLU * up).  Weights as in
 * cellm_hip_qgemv_q4_affine_qkv / _gate_up_silu: u32 words [out][hidden / 8],
 * scales and biases [out][hidden / group]; here f32 (sb_dtype
 * CELLM_HIP_DTYPE_F32) with group a power of two >= 32.  biasq/biask/biasv are
 * the f32 projection biases [out] or NULL; they are added to the row sums
 * before RoPE (add_projection_bias_if_present, qwen.rs:1132-1139).  The dot
 * runs in f32 over the normalised activations (no f16 rounding of x).  x_prev,
 * y, x_out and norm_w 16-byte aligned; rows 1..4, hidden % 32 == 0 and
 * <= 4096; otherwise CELLM_HIP_ERR_UNSUPPORTED (use the separate calls). */
int32_t cellm_hip_decode_q4_affine_qkv_rope_kv(
    cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
    const uint32_t* wq, const void* sq, const void* bq, const float* biasq, const uint32_t* wk, const void* sk,
    const void* bk, const float* biask, const uint32_t* wv, const void* sv, const void* bv, const float* biasv,
    int32_t sb_dtype, int64_t group, int64_t rows, int64_t hidden, int64_t n_heads, int64_t n_kv_heads,
    int64_t head_dim, const int32_t* positions, const float* cos_sin, int64_t table_positions, float* q_out,
    uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
    int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream);
int32_t cellm_hip_decode_q4_affine_gate_up_silu(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y,
                                                float* x_out, const float* norm_w, float eps, const uint32_t* wg,
                                                const void* sg, const void* bg, const uint32_t* wu, const void* su,
                                                const void* bu, int32_t sb_dtype, int64_t group, int64_t rows,
                                                int64_t hidden, int64_t inter, float* h, void* stream);

/* MetalKvStorage::encode_attention / attention_single_token_gqa_f32
 * (kvcache.rs:710-789, 1377-1439): each row attends over positions
 * 0..positions[r] of `layer`; q and out [rows][n_heads][head_dim] f32, query
 * head h reads kv head h / (n_heads / n_kv_heads).  score = (q . k) * scale,
 * scale = attn_scale, or 1/sqrt(head_dim) when attn_scale is 0 (the
 * reference's None); soft_cap > 0 maps each score s to tanh(s / soft_cap) *
 * soft_cap (Gemma), 0 = none.  Needs n_heads % n_kv_heads == 0, at most 8
 * query heads per kv head, head_dim 64 or 128, max_blocks * tokens_per_block
 * <= 32768.  Tables of up to 512 positions (max_blocks * tokens_per_block)
 * run one block per (row, query head) over the whole sequence, with no
 * workspace use.  Longer tables are split over the sequence in chunks of 64
 * positions, one block each; the last chunk block of each (row, kv head) to
 * finish combines the group's softmax partials in the same launch (workspace
 * owned by the context, per stream: 64 KB of group counters, zeroed when the
 * workspace is allocated and left at zero by every call, then the partials).
 * More than 16384 (row, kv head) groups take a second combine launch. */
int32_t cellm_hip_attention_gqa_f16kv(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                      const uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks,
                                      int64_t total_blocks, const int32_t* positions, int64_t rows, int64_t n_heads,
                                      int64_t n_kv_heads, int64_t head_dim, int64_t n_layers, int64_t tokens_per_block,
                                      int64_t layer, float attn_scale, float soft_cap, float* out, void* stream);

/* Sliding-window attention of Gemma-3/4 sliding layers (gemma.rs:747-780:
 * the gather starts at seq.saturating_sub(sliding_window), seq = the row's
 * position + 1; the pattern of gemma.rs:570-585 picks the layers): as
 * cellm_hip_attention_gqa_f16kv, but each row attends only to its last
 * `window` positions, max(0, positions[r] + 1 - window) .. positions[r].
 * window 0 attends to every position (the full-attention layers); window < 0
 * is CELLM_HIP_ERR_INVALID_ARG.  Same limits and workspace. */
int32_t cellm_hip_attention_gqa_f16kv_window(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                             const uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks,
                                             int64_t total_blocks, const int32_t* positions, int64_t rows,
                                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t n_layers,
                                             int64_t tokens_per_block, int64_t layer, float attn_scale, float soft_cap,
                                             int64_t window, float* out, void* stream);

/* cellm_hip_attention_gqa_f16kv without any allocation, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments and results; the group counters and softmax partials of
 * the split form (tables of more than 512 positions) go to a static device
 * array of 8 MiB that each GPU holds until the process ends,
 * so calls that need more -- 65536 + rows * n_heads * ceil(max_blocks *
 * tokens_per_block / 64) * (head_dim + 2) * 4 bytes -- fail with
 * CELLM_HIP_ERR_INVALID_ARG.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other contexts, other threads) race and must be serialised
 * by the caller. */
int32_t cellm_hip_attention_gqa_f16kv_noalloc(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                              const uint16_t* vcache, const uint32_t* block_tables,
                                              int64_t max_blocks, int64_t total_blocks, const int32_t* positions,
                                              int64_t rows, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                              int64_t n_layers, int64_t tokens_per_block, int64_t layer,
                                              float attn_scale, float soft_cap, float* out, void* stream);

/* MetalOps::encode_silu_mul_f32_inplace (metal.rs:232-243, the CPU loop of
 * llama.rs:477-484): gate[i] = silu(gate[i]) * up[i], silu(g) = g / (1 + exp(-g)),
 * in place on gate. */
int32_t cellm_hip_silu_mul_f32(cellm_hip_ctx_t* ctx, float* gate, const float* up, int64_t n, void* stream);

/* MetalOps::encode_gelu_tanh_mul_f32_inplace (metal.rs:245-257, 966-982; the CPU
 * loop of gemma.rs:844-846): gate[i] = gelu_tanh(gate[i]) * up[i], gelu_tanh as
 * cellm_hip_qgemv_i8_gate_up_gelu. */
int32_t cellm_hip_gelu_tanh_mul_f32(cellm_hip_ctx_t* ctx, float* gate, const float* up, int64_t n, void* stream);

/* MetalOps::encode_add_f32_inplace: x[i] += y[i]. */
int32_t cellm_hip_add_f32_inplace(cellm_hip_ctx_t* ctx, float* x, const float* y, int64_t n, void* stream);

/* topk_from_logits(..)[0] (llama.rs:1049-1078) after the non-finite -> -inf
 * sanitize (llama.rs:1081-1092), per row: the first index of the maximum.
 * One launch of 4096-element chunk blocks per row (rows <= 65535); rows of
 * more than one chunk hand their chunk maxima to the row's last block through
 * the context's per-stream scratch (a few bytes per chunk, allocated on the
 * first call that needs more, counters left at zero by every call). */
int32_t cellm_hip_argmax_f32(cellm_hip_ctx_t* ctx, const float* logits, int64_t rows, int64_t n, int32_t* out_index,
                             float* out_value, void* stream);

/* The same first maximum (topk_from_logits(..)[0], llama.rs:1049-1092) as a
 * packed key per row, for callers that read the result on the host anyway
 * (the greedy decode loop, llama.rs:1049-1078): out_keys[r] = max(out_keys[r],
 * key of the row's first maximum), one 64-bit atomic max per 4096-element
 * chunk, so no scratch, counter or combining block.  out_keys must hold zero
 * before the call (a zero key is below every key; e.g. clear it with the
 * step's uploaded inputs) and be 8-byte aligned; a repeated call on the same
 * logits leaves the keys as they are.  Key: high word = the value's bits in
 * unsigned order (non-finite values taken as -inf, -0 as +0), low word =
 * 0xffffffff - index; the two calls below decode a key (host only, no device). */
int32_t cellm_hip_argmax_f32_keys(cellm_hip_ctx_t* ctx, const float* logits, int64_t rows, int64_t n,
                                  uint64_t* out_keys, void* stream);
int32_t cellm_hip_argmax_key_index(uint64_t key);
float cellm_hip_argmax_key_value(uint64_t key);

/* ---- .cellm model files -----------------------------------------------------
 * CellmFile (crates/cellm-model/src/cellm_file.rs:58-146): "CELLM", version 1,
 * u32 little-endian header length, JSON header whose "tensors" list gives
 * each tensor's name, absolute offset_bytes, nbytes, shape and dtype string
 * ("f32", "f16", "bf16", "i8", "u8", "u32", "i4", "i2", "q1_0_g128", ...;
 * int8 / i4 / i2 weights have an f16 "<name>.qscale" companion, MLX affine
 * u32 weights ".scales" / ".biases").  The file is memory-mapped read-only
 * and every tensor range is checked at open.  These calls touch no device. */
typedef struct cellm_file cellm_file_t;

/* The model fields of CellmHeader (cellm_file.rs:20-48) a runner needs;
 * optional counts the header omits are -1, tie_word_embeddings -1 if absent. */
typedef struct {
    char model_type[64];
    int64_t vocab_size;
    int64_t hidden_dim;
    int64_t intermediate_size;
    int64_t num_layers;
    int64_t num_heads;
    int64_t num_kv_heads;
    int64_t head_dim;
    int64_t bos_token_id;
    int64_t eos_token_id;
    int64_t max_position_embeddings;
    float rms_norm_eps;
    float rope_theta;
    int32_t tie_word_embeddings;
} cellm_file_config_t;

/* One entry of the header's tensor list (CellmTensorIndex, cellm_file.rs:11-18);
 * name and dtype stay valid until cellm_file_close. */
typedef struct {
    const char* name;
    const char* dtype;
    int64_t shape[8];
    int32_t ndim;
    uint64_t offset_bytes;
    uint64_t nbytes;
} cellm_file_tensor_t;

/* CellmFile::load: map, validate, parse; pages are touched once (the
 * reference's pre-warm, cellm_file.rs:91-105). */
int32_t cellm_file_open(const char* path, cellm_file_t** out);
void cellm_file_close(cellm_file_t* f);
int32_t cellm_file_config(const cellm_file_t* f, cellm_file_config_t* out);
/* The raw JSON header text (not NUL-terminated), valid until close. */
int32_t cellm_file_header_json(const cellm_file_t* f, const char** out_text, size_t* out_len);
int64_t cellm_file_tensor_count(const cellm_file_t* f);
/* The index-th tensor of the header, in header order. */
int32_t cellm_file_tensor_at(const cellm_file_t* f, int64_t index, cellm_file_tensor_t* out);
/* tensor_index / has_tensor: CELLM_HIP_ERR_NOT_FOUND if the name is absent
 * (out may be NULL to test presence). */
int32_t cellm_file_find(const cellm_file_t* f, const char* name, cellm_file_tensor_t* out);
/* tensor_bytes (cellm_file.rs:138-146): the mapped bytes of a tensor. */
int32_t cellm_file_tensor_bytes(const cellm_file_t* f, const char* name, const void** out_host, size_t* out_nbytes);

/* Device-resident weights from a file: every tensor whose name starts with
 * name_prefix (NULL or "" = all) goes into ctx's weight cache under its own
 * name, one host-to-device copy each, as the Metal graphs preload every
 * tensor of the file once (preload_weight, llama_graph.rs:92-110, gemma_graph.rs:145;
 * called from llama.rs:146).  Returns how many tensors and bytes were
 * uploaded; look them up with cellm_hip_weight_lookup. */
int32_t cellm_hip_upload_cellm_file(cellm_hip_ctx_t* ctx, const cellm_file_t* f, const char* name_prefix,
                                    int64_t* out_count, size_t* out_bytes);

/* One projection y[m, out] = W x[m, in] (x, y: f32 device arrays) by the dtype
 * of the .cellm tensor `weight_name` (an exact name, as the runners'
 * *_by_exact_name lookups take it), with the rules of one runner family's
 * linear_f16_out_in:
 *   LLAMA (llama.rs:743-941): 2-D [out, in] check; "f16"; "i8" + f16 .qscale,
 *         one per row; "i4" + .qscale, gs = in (the row's first scale).
 *   QWEN  (qwen.rs:1033-1105): "f16"; "i8"; "i4" with gs = in / (scales per
 *         row) when .qscale holds more than one scale per row;
 *         "q1_0_g128" (dot_row, :1004-1022); "i2" with the row scale applied
 *         to the sum (:1591-1606).
 *   GEMMA (gemma.rs:1358-1499): [out, in] check; "f16"; "i8"; "i4" with
 *         exactly one scale per row; "i2" with the scale applied per element
 *         (:1673-1687).
 *   LFM   (lfm.rs:924-981): "u32" with "<base>.scales" and "<base>.biases"
 *         (f32, groups of 64) -> MLX affine GEMV; any other tensor is read as
 *         f16.
 * Each arm runs the GEMV entry point of its format (cellm_hip_qgemv_*) on
 * `stream`.  The tensors it reads are uploaded into the context's weight
 * cache under their file names on the first call (blocking), as MetalOps
 * caches weights by name (metal.rs:1045-1050); two files with equal tensor
 * names therefore need two contexts.  Other dtypes and malformed tensors
 * return CELLM_HIP_ERR_UNSUPPORTED / CELLM_HIP_ERR_INVALID_ARG with the
 * reference's messages. */
#define CELLM_HIP_FAMILY_LLAMA 0
#define CELLM_HIP_FAMILY_QWEN 1
#define CELLM_HIP_FAMILY_GEMMA 2
#define CELLM_HIP_FAMILY_LFM 3
int32_t cellm_hip_linear_file(cellm_hip_ctx_t* ctx, const cellm_file_t* f, const char* weight_name, int32_t family,
                              const float* x, float* y, int64_t m, int64_t out_dim, int64_t in_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CELLM_HIP_H */
