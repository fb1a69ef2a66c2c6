// Host-side launchers for the cellm HIP kernels.  All pointers are device
// pointers; all launches are asynchronous on `st`.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cellm {

// Decode GEMV, int8 weights with one scale per output row (per_channel=1) or
// one scale for the tensor (per_channel=0).  M <= 4 and K % 16 == 0 take the
// fast kernels; anything else runs the generic one-wave-per-row kernel.
hipError_t launch_qgemv_i8(const int8_t* w, const void* S, int sdt, int per_channel, const void* x, int xdt,
                           const float* bias, float* y, int M, int N, int K, hipStream_t st, int force_generic);

// Decode GEMV, MLX 4-bit affine weights (u32 words, 8 nibbles; scale+bias per group).
hipError_t launch_qgemv_q4_affine(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                  const void* x, int xdt, float* y, int M, int N, int K, hipStream_t st,
                                  int force_generic);
int qgemv_q4_lds_bytes(int M, int K);

// Symmetric i4 (u8 bytes, low nibble = even element, (nib-8)*scale); team kernel for K % 32 == 0,
// per-row or 32-multiple groups, M <= 4; one wave per row otherwise.
hipError_t launch_qgemv_i4_sym(const uint8_t* w, const uint16_t* S, int spr, int gs, const void* x, int xdt, float* y,
                               int M, int N, int K, hipStream_t st);

// Bit-exact dequant of MLX affine weights: out_dt f32 (lfm.rs order) or f16
// (converter RNE).
hipError_t launch_dequant_q4_affine(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                    void* out, int out_dt, int N, int K, hipStream_t st);

// Fused multi-output int8 GEMV (qgemv.hip): nseg (1..3) matrices sharing x
// in one launch, or (silu) seg 0 = gate, seg 1 = up with h = silu(g) * u
// written to seg 0's y.  Requires M <= 4, f16/f32 x, K % 16 == 0 and 16-byte
// aligned W and x (qgemv_i8_fused_supported).
struct I8FusedSeg {
    const int8_t* w;
    const void* s;
    const float* bias;
    float* y;
    int n;
    int per_channel;
};
bool qgemv_i8_fused_supported(int xdt, int M, int K, const void* x, const I8FusedSeg* segs, int nseg);
hipError_t launch_qgemv_i8_fused(const I8FusedSeg* segs, int nseg, bool silu, int act, int sdt, const void* x, int xdt,
                                 int M, int K, hipStream_t st);

// MLX q4 gate/up + SiLU in one launch: h[m,n] = silu(gate[m,n]) * up[m,n] (f16 x, M <= 4,
// K % 32 == 0, group >= 32, 16-byte aligned x and weights, x in 64 KB of LDS).
bool qgemv_q4_gate_up_supported(int xdt, int M, int K, int group_size, const void* x, const void* wg, const void* wu);
hipError_t launch_qgemv_q4_gate_up_silu(const uint32_t* wg, const void* Sg, const void* Bg, const uint32_t* wu,
                                        const void* Su, const void* Bu, int sbt, int group_size, const void* x,
                                        int xdt, float* h, int M, int N, int K, int act, hipStream_t st);

// h[i] = silu(g[i]) * u[i] in place on g (dequant.hip), silu(g) = g / (1 + exp(-g)).
// gate[i] = act(gate[i]) * up[i] for act ACT_SILU / ACT_GELU_TANH (common.hpp act_mul)
hipError_t launch_act_mul(int act, float* g, const float* u, size_t count, hipStream_t st);
hipError_t launch_silu_mul(float* g, const float* u, size_t count, hipStream_t st);
// y[m, n] += bias[n] over M rows of N (the projection-bias fallback of the multi-segment q4 GEMV)
hipError_t launch_add_bias_rows(float* y, const float* bias, int M, int N, hipStream_t st);

// Up to three MLX q4 matrices sharing x in one launch (f16 or f32 x, M <= 4, K % 32 == 0,
// group >= 32, 16-byte aligned x and W), each with its own scales S, group biases B,
// optional f32 projection bias [n] and output y [M][n].
struct Q4FusedSeg {
    const uint32_t* w;
    const void* S;
    const void* B;
    const float* bias;
    float* y;
    int n;
};
bool qgemv_q4_segs_supported(int xdt, int M, int K, int group_size, const void* x, const Q4FusedSeg* segs, int nseg);
hipError_t launch_qgemv_q4_segs(const Q4FusedSeg* segs, int nseg, int sbt, int group_size, const void* x, int xdt,
                                int M, int K, hipStream_t st);

// Prefill / batched qGEMM on MFMA: Y[M,N] = X[M,K] . dequant(W)[N,K]^T with
// W tiles dequantized to f16 in LDS and f32 accumulation.  Requires K % 64 == 0
// and 16-byte aligned W and X.  `workspace` (qgemm_workspace_bytes: wt 0 = q4
// affine, 1 = int8) enables split-K; nullptr runs without it.
int qgemm_splits(int M, int N, int K);
size_t qgemm_workspace_bytes(int wt, int M, int N, int K, int group_size, int sbt);
hipError_t launch_qgemm_q4_affine_ws(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                     const _Float16* x, float* y, int M, int N, int K, float* workspace,
                                     hipStream_t st);
hipError_t launch_qgemm_i8_ws(const int8_t* w, const void* S, int sdt, int per_channel, const _Float16* x,
                              const float* bias, float* y, int M, int N, int K, float* workspace, hipStream_t st);

// Batched decode on MFMA (2 <= M <= 64, f16 x): int8 needs K % 64 == 0 and
// K >= 128, q4 K % 128 == 0, K >= 256 and group >= 32; 16-byte aligned W and x;
// ceil16(M) * N * 4 < 2^31.
// Small N over a long K splits K over work items (partial sums in `ws`, then a
// reduction kernel); qgemv_mfma_workspace_bytes is the size that needs, 0 when
// the shape runs unsplit.  Without enough workspace the shape runs unsplit.
bool qgemv_mfma_supported(int wt, int M, int N, int K, int group_size);
size_t qgemv_mfma_workspace_bytes(int wt, int M, int N, int K);

// q4 affine with f32 x on MFMA (1 <= M <= 4, N % 16 == 0, K % 128 == 0, K <= 1024,
// group 64; 16-byte aligned W and x): nibbles as exact f16 integers, x as hi + lo f16
// parts scaled per (row, group) by a power of two, scale and bias folded per group.
bool qgemv_q4_f32x_mfma_supported(int M, int N, int K, int group_size);
// int8 rows over f32 x on int8 MFMA (x as three 8-bit digits per row, one power of two per row; the
// row scale after the exact integer sums): M <= 4, N % 16 == 0, K % 64 == 0, 128 <= K <= 1024.
bool qgemv_i8_f32x_mfma_supported(int M, int N, int K);
hipError_t launch_qgemv_i8_f32x_mfma(const int8_t* w, const void* S, int sdt, int per_channel, const float* bias,
                                     const float* x, float* y, int M, int N, int K, hipStream_t st);
hipError_t launch_qgemv_q4_f32x_mfma(const uint32_t* wq, const void* S, const void* B, int sbt, const float* x,
                                     float* y, int M, int N, int K, hipStream_t st);
hipError_t launch_qgemv_mfma_i8(const int8_t* w, const void* S, int sdt, int per_channel, const _Float16* x,
                                const float* bias, float* y, int M, int N, int K, float* ws, size_t ws_bytes,
                                hipStream_t st);
hipError_t launch_qgemv_mfma_q4(const uint32_t* wq, const void* S, const void* B, int sbt, int group_size,
                                const _Float16* x, float* y, int M, int N, int K, float* ws, size_t ws_bytes,
                                hipStream_t st);

// Decode-step kernels (decode.hip).  `rows` sessions, one activation row each;
// positions and block tables are device arrays ([rows] int32, [rows][max_blocks]
// uint32); K/V caches are f16 pages laid out as KvCacheLayout::token_base_elem.
hipError_t launch_embed_i8(const uint32_t* tokens, int rows, const int8_t* emb, const uint16_t* scale, int vocab,
                           int hidden, float* x, hipStream_t st);
hipError_t launch_embed_f16(const uint32_t* tokens, int rows, const uint16_t* emb, int vocab, int hidden, float* x,
                            hipStream_t st);
hipError_t launch_embed_i4(const uint32_t* tokens, int rows, const uint8_t* emb, const uint16_t* scale, int vocab,
                           int hidden, float* x, hipStream_t st);
hipError_t launch_rms_norm(const float* x, const void* w, int wdt, int rows, int n, float eps, float* out,
                           hipStream_t st);
hipError_t launch_add_rms_norm(float* x, const float* y, const void* w, int wdt, int rows, int n, float eps,
                               float* out, hipStream_t st);
hipError_t launch_rope_kv_write_f16(float* q, float* k, const float* v, int rows, int n_heads, int n_kv_heads,
                                    int head_dim, const int32_t* pos, const float* cos_sin, int table_positions,
                                    uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int max_blocks,
                                    int total_blocks, int n_layers, int tokens_per_block, int layer, int interleaved, hipStream_t st);
hipError_t launch_rope_half(float* x, int rows, int n_heads, int head_dim, const int32_t* pos, const float* cos_sin,
                            int table_positions, int interleaved, hipStream_t st);
hipError_t launch_kv_write_f16(const float* k, const float* v, int rows, int kv_dim, const int32_t* pos,
                               uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int max_blocks,
                               int total_blocks, int n_layers, int tokens_per_block, int layer, hipStream_t st);
bool attention_supported(int n_heads, int n_kv_heads, int head_dim, int max_seq);
size_t attention_workspace_bytes(int rows, int n_heads, int n_kv_heads, int head_dim, int max_seq);
// Bytes at the start of an attention workspace that hold its group counters:
// zero when the workspace is first used, and zero again after every call.
size_t attention_counter_bytes();
hipError_t launch_attention_gqa_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                                      const uint32_t* block_tables, int max_blocks, int total_blocks,
                                      const int32_t* pos, int rows, int n_heads, int n_kv_heads, int head_dim,
                                      int n_layers, int tokens_per_block, int layer, float attn_scale,
                                      float soft_cap, float* out, float* workspace, hipStream_t st,
                                      int window = 0);  // window > 0: each row attends to its last `window` positions
// First maximum per row (non-finite -> -inf): chunk blocks of 4096 elements in one launch; rows past
// one chunk need scratch of argmax_scratch_bytes whose first argmax_counter_bytes (the per-row
// counters) are zero before the first call and are left at zero by every call.
size_t argmax_scratch_bytes(int rows, int n);
size_t argmax_counter_bytes(int rows);
hipError_t launch_argmax(const float* logits, int rows, int n, int32_t* idx, float* val, void* scratch, hipStream_t st);
// The same first maximum per row as a packed key (value order in the high word, 0xffffffff - index
// in the low word) merged into keys[r] by one 64-bit atomic max per chunk block: keys start at zero;
// no scratch.
hipError_t launch_argmax_keys(const float* logits, int rows, int n, uint64_t* keys, hipStream_t st);
// Size of the static attention scratch (decode.hip) and the current device's
// address of it (hipGetSymbolAddress once per device, cached).
constexpr size_t kAttnStaticScratchBytes = (size_t)8 << 20;
hipError_t attention_static_scratch(float** out);
// Fused decode-step GEMVs (decode.hip): residual add + RMSNorm prologue, int8
// GEMV of two rows per team, RoPE + K/V write or SiLU * up epilogue.
bool decode_fused_supported(int rows, int H);
size_t decode_fused_lds_bytes(int rows, int H);
hipError_t launch_decode_qkv(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                             const int8_t* const w[3], const uint16_t* const s[3], int rows, int H, int n_heads,
                             int n_kv_heads, int head_dim, const int32_t* pos, const float* cos_sin,
                             int table_positions, float* q_out, uint16_t* kcache, uint16_t* vcache,
                             const uint32_t* block_tables, int max_blocks, int total_blocks, int n_layers,
                             int tokens_per_block, int layer, int interleaved, hipStream_t st);
hipError_t launch_decode_gate_up(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                 const int8_t* wg, const uint16_t* sg, const int8_t* wu, const uint16_t* su, int rows,
                                 int H, int N, float* h, hipStream_t st);
// The same two launches over MLX q4 affine weights (u32 words, f32 scales and
// biases, group a power of two >= 32) with an f32 dot: rows 1..4, H % 32 == 0,
// H <= 4096; q/k/v projection biases optional (null entries).
bool decode_q4_fused_supported(int rows, int H, int group);
// Plain MLX q4 affine GEMV over f32 x at M <= 4 with f32 scales/biases (decode.hip): x in LDS as f32,
// f32 dot; K % 32 == 0 and K <= 2048, group a power of two >= 32.
bool qgemv_q4_x32_supported(int M, int N, int K, int group);
// The same over longer rows (2048 < K, four rows of x within 160 KB of LDS: K <= 7936): each row
// split over the waves of one block.
bool qgemv_q4_x32s_supported(int M, int N, int K, int group);
hipError_t launch_qgemv_q4_x32s(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                                int N, int K, int group, hipStream_t st);
hipError_t launch_qgemv_q4_x32(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                               int N, int K, int group, hipStream_t st);
hipError_t launch_decode_q4_qkv(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                const uint32_t* const w[3], const float* const s[3], const float* const b[3],
                                const float* const bias[3], int group, int rows, int H, int n_heads, int n_kv_heads,
                                int head_dim, const int32_t* pos, const float* cos_sin, int table_positions,
                                float* q_out, uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables,
                                int max_blocks, int total_blocks, int n_layers, int tokens_per_block, int layer,
                                int interleaved, hipStream_t st);
hipError_t launch_decode_q4_gate_up(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                    const uint32_t* wg, const float* sg, const float* bg, const uint32_t* wu,
                                    const float* su, const float* bu, int group, int rows, int H, int N, int act,
                                    float* h, hipStream_t st);

// Remaining .cellm weight formats (lowbit.hip): f16 rows, i2 (2-bit per-row
// symmetric, scale_mode 0 = scale at the end, 1 = per element), q1_0_g128.
enum { LB_F16 = 0, LB_I2 = 1, LB_Q1 = 2 };
size_t lowbit_row_bytes(int fmt, int K);
hipError_t launch_qgemv_lowbit(int fmt, const void* w, const uint16_t* S, int scale_mode, const void* x, int xdt,
                               float* y, int M, int N, int K, hipStream_t st);

// Device smoke test kernel: out[i] = a[i] + b[i].
// y[0..count) = v (used where a result is all zeros, e.g. K == 0)
hipError_t launch_fill_f32(float* y, float v, size_t count, hipStream_t st);
hipError_t launch_add_f32(const float* a, const float* b, float* out, int n, hipStream_t st);

}  // namespace cellm
