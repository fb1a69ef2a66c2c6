/*
 * cellm_llama_step.h -- Llama decode steps over libcellm_hip.so: a host-side
 * step whose projections run on the HIP qGEMV (cellm_llama_*), and a
 * device-resident step (cellm_llama_dev_*, below).
 *
 * This is the runner side of the boundary, above the C ABI of cellm_hip.h.
 * The host-side step mirrors LlamaRunner::step_topk / step_inner
 * (crates/cellm-model/src/llama.rs:189-212, 235-647) with every int8
 * projection (q, k, v, o, gate, up, down, tied lm_head) issued to the HIP
 * qGEMV, while embedding, RMSNorm, RoPE, the paged f16 KV cache and GQA
 * attention stay on the CPU ("the existing path", as a Rust runner with a
 * HipOps would keep them).  Greedy top-1 follows topk_from_logits
 * (llama.rs:1049-1078).
 *
 * Status codes are those of cellm_hip.h; this library's own messages are
 * read with cellm_llama_last_error_message (errors raised inside
 * libcellm_hip.so are copied there too).
 */
#ifndef CELLM_LLAMA_STEP_H
#define CELLM_LLAMA_STEP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape (ModelConfig, crates/cellm-model/src/lib.rs; .cellm header). */
typedef struct {
    int32_t n_layers;
    int32_t hidden;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t intermediate;
    int32_t vocab;
    float rms_norm_eps;
    float rope_theta;
    int32_t tokens_per_block; /* KvCacheLayout::tokens_per_block */
    int32_t total_blocks;     /* KvCacheLayout::total_blocks */
} cellm_llama_config_t;

/* One layer's host tensors: int8 [out, in] weights with f16 per-row scales
 * (".qscale"), f16 RMSNorm weights.  Order: q, k, v, o, gate, up, down. */
typedef struct {
    const int8_t* w[7];
    const uint16_t* scale_f16[7];
    const uint16_t* input_layernorm_f16;
    const uint16_t* post_attention_layernorm_f16;
} cellm_llama_layer_t;

typedef struct cellm_llama cellm_llama_t;

/* Copies the calling thread's last error message; returns its full length. */
size_t cellm_llama_last_error_message(char* buf, size_t buf_len);

/* Builds the runner on `device`, uploading every projection weight once into
 * the HIP weight cache.  embed_i8 [vocab, hidden] with f16 row scales is also
 * the tied lm_head.  Host arrays may be freed after the call. */
int32_t cellm_llama_create(const cellm_llama_config_t* cfg, const cellm_llama_layer_t* layers,
                           const int8_t* embed_i8, const uint16_t* embed_scale_f16,
                           const uint16_t* final_norm_f16, int32_t device, cellm_llama_t** out);

void cellm_llama_destroy(cellm_llama_t* m);

/* The CPU paged KV cache: K and V are f16 arrays of
 * total_blocks * n_layers * tokens_per_block * n_kv_heads * head_dim elements,
 * laid out as KvCacheLayout::token_base_elem (crates/cellm-core/src/kv_cache.rs:62-73).
 * Returned pointers stay valid until destroy; callers may seed them. */
int32_t cellm_llama_kv_cache(cellm_llama_t* m, uint16_t** k_f16, uint16_t** v_f16, size_t* n_elems);

/* One decode step of one session (LlamaRunner::step_topk with top_k = 1):
 * embeds `token`, writes this position's K/V into block
 * block_table[pos / tokens_per_block], attends over positions 0..pos, and
 * returns the greedy id and its logit.  logits_out (vocab floats) is optional. */
int32_t cellm_llama_step(cellm_llama_t* m, uint32_t token, size_t pos, const uint32_t* block_table,
                         size_t n_blocks, uint32_t* out_token, float* out_logit, float* logits_out);

/* ---- device-resident step ------------------------------------------------
 * The HIP counterpart of the fused Metal decode graph
 * LlamaGraphState::step_fused (crates/cellm-model/src/llama_graph.rs:140-405):
 * weights in the HIP weight cache, a paged f16 K/V cache on the device
 * (same layout as cellm_llama_kv_cache), RMSNorm, RoPE, the K/V write, GQA
 * attention and the greedy id on the device (cellm_hip.h decode-step ops).
 * A step decodes up to max_rows (1..4) sessions together: one GEMV per
 * projection over all their rows, instead of the reference's one session at
 * a time (crates/cellm-sdk/src/lib.rs:581-599). */
typedef struct cellm_llama_dev cellm_llama_dev_t;

/* Weights as for cellm_llama_create.  max_blocks: entries per block table
 * (positions up to max_blocks * tokens_per_block - 1).  The K/V cache starts
 * zeroed.  The step's launches are captured as one HIP graph per row count
 * (1..max_rows) here, and steps replay them. */
int32_t cellm_llama_dev_create(const cellm_llama_config_t* cfg, const cellm_llama_layer_t* layers,
                               const int8_t* embed_i8, const uint16_t* embed_scale_f16,
                               const uint16_t* final_norm_f16, int32_t device, int32_t max_rows, int32_t max_blocks,
                               cellm_llama_dev_t** out);

/* The same runner from a .cellm file (LlamaRunner::load, llama.rs:39-75): the
 * model shape from the header (head_dim defaults to hidden / heads), f16
 * norms, and each projection dispatched on the dtype of its weight tensor as
 * the runners' linear_f16_out_in does (llama.rs:781-941, lfm.rs:924-981,
 * gemma.rs:1358-1499):
 *   "i8"  [out, in] + f16 "<w>.qscale" [out]            -> cellm_hip_qgemv_i8;
 *   "u32" [out, in/8] MLX affine words + f32 "<base>.scales" / "<base>.biases"
 *         [out, ceil(in/64)] (tools/convert_lfm.py:123-136)
 *                                                        -> cellm_hip_qgemv_q4_affine;
 *   "i4"  [out, in] (ceil(in/2) bytes per row) + f16 "<w>.qscale", one or more
 *         scales per row; Llama reads each row's first (gs = in, llama.rs:932)
 *                                                        -> cellm_hip_qgemv_i4_sym;
 *   "f16" [out, in] (llama.rs:898)                       -> cellm_hip_qgemv_f16.
 * The header's model_type picks the layer (crates/cellm-sdk/src/lib.rs:125-135):
 *   "qwen*": the Qwen2 layer of QwenRunner and its fused Metal step
 *     (qwen.rs:309-630, 1255-1470): tensor prefix "model.language_model.",
 *     "language_model.model.", "model." or "" (qwen.rs:339-342); an optional
 *     f16 "<stem>.bias" [out] on any projection, added after it
 *     (qwen.rs:1132-1139); i4 with s scales per row in groups of in / s
 *     (qwen.rs:1076-1077); also "i2" [out, in] + f16 .qscale [out], the scale
 *     on the row sum (qwen.rs:1087-1096) -> cellm_hip_qgemv_i2, and
 *     "q1_0_g128" (qwen.rs:1004-1022) -> cellm_hip_qgemv_q1_0_g128.  q/k norms
 *     (Qwen3) and model_type qwen3_5 are CELLM_HIP_ERR_UNSUPPORTED.
 *   anything else: the Llama layer, prefix "" or "language_model." before
 *     "model." (detect_llama_prefix, llama.rs:1094-1113).
 * The embedding is "i8" or "i4" (+ f16 .qscale, one per row) or "f16"
 * (embed_token, llama.rs:676-726, qwen.rs:850-918) -> cellm_hip_embed_i8 /
 * _i4 / _f16, and is the lm_head, read through the GEMV of its format, unless
 * the file has an lm_head.weight (llama.rs:522-646, qwen.rs:575-630).  Other
 * dtypes are CELLM_HIP_ERR_UNSUPPORTED.  A model whose projections are all
 * "i8" without biases runs the fused decode launches; any other mix runs one
 * launch per projection (the int8 QKV and gate/up pairs as one launch each,
 * biases in their epilogue).  tokens_per_block / total_blocks size the paged
 * K/V cache; the file is closed before this returns. */
int32_t cellm_llama_dev_create_from_file(const char* path, int32_t device, int32_t max_rows, int32_t max_blocks,
                                         int32_t tokens_per_block, int32_t total_blocks, cellm_llama_dev_t** out);

void cellm_llama_dev_destroy(cellm_llama_dev_t* m);

/* enable = 0: steps enqueue their launches one by one instead of replaying
 * the captured graph (same kernels, same arguments); 1: replay (default). */
int32_t cellm_llama_dev_set_graphs(cellm_llama_dev_t* m, int32_t enable);

/* Copy the whole K and V caches (n_elems f16 each, cellm_llama_kv_cache layout)
 * to / from the device. */
int32_t cellm_llama_dev_kv_upload(cellm_llama_dev_t* m, const uint16_t* k_f16, const uint16_t* v_f16,
                                  size_t n_elems);
int32_t cellm_llama_dev_kv_download(cellm_llama_dev_t* m, uint16_t* k_f16, uint16_t* v_f16, size_t n_elems);

/* One decode step for `rows` sessions: tokens[rows], positions[rows],
 * block_tables[rows * max_blocks].  Each session writes its K/V at its
 * position and attends over 0..position.  Returns each greedy id (and its
 * logit in out_logits, optional); logits_out [rows * vocab] is optional. */
int32_t cellm_llama_dev_step(cellm_llama_dev_t* m, int32_t rows, const uint32_t* tokens, const int32_t* positions,
                             const uint32_t* block_tables, uint32_t* out_tokens, float* out_logits, float* logits_out);

/* The RoPE table of the device step: out[p][i] = (cos, sin) of
 * p * theta^(-2i/head_dim) for p < positions, i < head_dim / 2, in f32 as
 * rope_non_interleaved_inplace_f32 computes them (cpu_kernels.rs:264-277). */
int32_t cellm_llama_rope_table(float theta, int32_t head_dim, int32_t positions, float* out);

#ifdef __cplusplus
}
#endif

#endif /* CELLM_LLAMA_STEP_H */
