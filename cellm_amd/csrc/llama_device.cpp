// Device-resident Llama decode step over libcellm_hip.so (declared in
// include/cellm_llama_step.h): the HIP counterpart of the fused Metal decode
// graph LlamaGraphState::step_fused (crates/cellm-model/src/llama_graph.rs:140-405).
// Weights are uploaded once into the context's name-keyed weight cache
// (preload_weight, llama_graph.rs:92-99); the paged f16 K/V cache, the RoPE
// table and the activations live on the device; a step is one stream of
// launches through the C ABI and one small copy back.
//
// Unlike the reference, which decodes sessions one at a time
// (crates/cellm-sdk/src/lib.rs:581-599), a step takes up to max_rows sessions
// at once: every projection runs as one GEMV over all their activation rows,
// so each weight byte is read once per step, not once per session.
//
// The host parts (validation, the RoPE cos/sin table) are compiled without FP
// contraction so the table holds exactly the f32 values the CPU reference
// computes (cpu_kernels.rs:264-277).
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdlib>
#include <cctype>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/cellm_hip.h"
#include "../../include/cellm_llama_step.h"
#include "api_guard.hpp"

namespace cellm_step {
extern thread_local cellm::ErrorSlot g_err;  // llama_step.cpp: read by cellm_llama_last_error_message
int32_t report_exception(int32_t code, const char* what);
bool llama_rope_interleaved_from_env();      // llama_step.cpp
}

namespace {

using cellm_step::g_err;

int32_t fail(int32_t code, const char* fmt, ...)
{
    char buf[sizeof(g_err.msg)];
    va_list ap;
    va_start(ap, fmt);
    const int n = vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err.store(buf, n < 0 ? 0 : ((size_t)n < sizeof(buf) ? (size_t)n : sizeof(buf) - 1));
    return code;
}

int32_t from_hip_lib(int32_t rc, const char* what)
{
    char buf[512];
    cellm_hip_last_error_message(buf, sizeof(buf));
    return fail(rc, "%s: %s", what, buf);
}

int32_t from_runtime(hipError_t e, const char* what)
{
    return fail(e == hipErrorOutOfMemory ? CELLM_HIP_ERR_OUT_OF_MEMORY : CELLM_HIP_ERR_DEVICE, "%s: %s", what,
                hipGetErrorString(e));
}

#define RT_TRY(expr, what)                                 \
    do {                                                   \
        hipError_t e_ = (expr);                            \
        if (e_ != hipSuccess) return from_runtime(e_, what); \
    } while (0)
#define LIB_TRY(expr, what)                          \
    do {                                             \
        int32_t rc_ = (expr);                        \
        if (rc_ != CELLM_HIP_OK) return from_hip_lib(rc_, what); \
    } while (0)

const char* kNames[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                         "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj"};

// f16::from_bits(h).to_f32() (exact)
float h2f(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {
            const float v = (float)m * 5.9604644775390625e-08f;
            return sign ? -v : v;
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

struct DevBuf {
    void* p = nullptr;
    ~DevBuf()
    {
        if (p) (void)hipFree(p);
    }
    int32_t alloc(size_t bytes, const char* what)
    {
        RT_TRY(hipMalloc(&p, bytes ? bytes : 1), what);
        return CELLM_HIP_OK;
    }
    template <typename T>
    T* as() const
    {
        return reinterpret_cast<T*>(p);
    }
};

// One projection on the device, by the weight format of its .cellm tensor
// (the dtype dispatch of linear_f16_out_in: llama.rs:743-941, gemma.rs:1358-1499,
// lfm.rs:924-981):
//   I8: "i8" [out, in] + f16 "<w>.qscale" [out], scale applied to the row sum;
//   Q4: "u32" [out, in/8] MLX affine words + f32 "<base>.scales" / "<base>.biases"
//       [out, ceil(in/64)] (tools/convert_lfm.py:123-136), group 64;
//   I4: "i4" [out, in], ceil(in/2) bytes per row, low nibble even, + f16
//       "<w>.qscale" [out]: one scale per row (gs = in, gemma.rs:1466-1471);
//   F16: "f16" [out, in], no scale (llama.rs:898 matmul_f16_f32);
//   I2, Q1 (Qwen files only): "i2" [out, in] in ceil(in/4) bytes per row + f16
//       "<w>.qscale" [out], the scale on the row sum (qwen.rs:1087-1096,
//       1591-1606); "q1_0_g128" [out, in] in in/128 blocks of 18 bytes
//       (qwen.rs:1004-1022).
// The embedding takes one of I8, I4 or F16 (embed_token, llama.rs:676-726), and
// the tied lm_head is the embedding in the same format (llama.rs:576-646).
enum ProjKind : int32_t { PK_I8 = 0, PK_Q4 = 1, PK_I4 = 2, PK_F16 = 3, PK_I2 = 4, PK_Q1 = 5 };

// Runner family: LLAMA follows LlamaRunner (llama.rs); QWEN the Qwen2 layers
// of QwenRunner and its fused Metal step (qwen.rs:309-630, 1255-1470): the same
// layer with optional f16 biases on every projection, added after it, and
// Qwen's weight formats.
enum Family : int32_t { FAM_LLAMA = 0, FAM_QWEN = 1 };

struct Proj {
    int32_t kind = PK_I8;
    const void* w = nullptr;
    const void* s = nullptr;  // I8/I4/I2: f16 row scales; Q4: f32 group scales; F16/Q1: none
    const void* b = nullptr;  // Q4: f32 group biases
    int64_t ns = 0, gs = 0;   // I4: scales in .qscale and the group size they cover
    const float* bias = nullptr;  // projection bias as f32, repeated for max_rows rows; nullptr: none
};

// Host-side source of one projection (mapped file bytes or caller memory).
struct HostProj {
    int32_t kind = PK_I8;
    const void* w = nullptr;
    size_t w_bytes = 0;
    const void* s = nullptr;
    size_t s_bytes = 0;
    const void* b = nullptr;
    size_t b_bytes = 0;
    int64_t ns = 0, gs = 0;              // I4: 0 = one scale per row, gs = in
    const uint16_t* bias_f16 = nullptr;  // [bias_n = out] f16, or nullptr
    size_t bias_n = 0;
};

struct HostModel {
    std::vector<HostProj> p;  // n_layers * 7, in kNames order
    std::vector<const uint16_t*> n1, n2;
    HostProj embed;  // kind I8, I4 or F16; s: f16 row scales (none for F16)
    HostProj lm;     // w == nullptr: tied to the embedding
    const uint16_t* final_norm = nullptr;
    bool rope_interleaved = false;  // RoPE pairs (2i, 2i + 1) instead of (i, i + head_dim/2)
};

}  // namespace

struct cellm_llama_dev {
    cellm_llama_config_t cfg{};
    int32_t max_rows = 0, max_blocks = 0, table_positions = 0;
    int device = 0;
    cellm_hip_ctx_t* hip = nullptr;
    void* stream = nullptr;
    size_t kvd = 0, kv_elems = 0;
    // device views of the cached weights: 7 projections per layer, then the lm_head
    std::vector<Proj> p;
    Proj lm;     // the tied embedding unless the model has its own lm_head
    Proj embed;  // kind I8, I4 or F16
    std::vector<const float*> attn_norm, mlp_norm;
    const float* final_norm = nullptr;
    DevBuf kcache, vcache, rope, x, x2, xn, q, k, v, attn, proj, h, up, logits, io;
    // fused add+norm+GEMV launches: every projection int8, rows <= 4, hidden % 16 == 0, hidden <= 4096
    bool fused = false;
    // the same over MLX q4 affine q/k/v (projection biases allowed) and gate/up (no biases), hidden % 32 == 0
    bool fused_q4 = false;
    // io: [tokens u32 | positions i32 | block tables u32 | greedy keys u64 (zero when uploaded)]
    void* host_io = nullptr;  // pinned mirror of io
    size_t io_tokens = 0, io_pos = 0, io_bt = 0, io_keys = 0, io_bytes = 0;
    // one captured graph per row count (index rows - 1): the step's launches
    // from the embedding to the argmax, replayed with one hipGraphLaunch
    hipGraph_t graph[4] = {};
    hipGraphExec_t graph_exec[4] = {};
    bool use_graphs = false;
};

namespace {

int32_t upload(cellm_llama_dev* m, const std::string& key, const void* host, size_t bytes, const void** dev)
{
    LIB_TRY(cellm_hip_weight_upload(m->hip, key.c_str(), host, bytes, dev), key.c_str());
    return CELLM_HIP_OK;
}

int32_t upload_norm(cellm_llama_dev* m, const std::string& key, const uint16_t* f16, size_t n, const float** dev)
{
    std::vector<float> f(n);
    for (size_t i = 0; i < n; ++i) f[i] = h2f(f16[i]);  // rmsnorm_weight (llama.rs:728-741)
    const void* d = nullptr;
    if (int32_t rc = upload(m, key, f.data(), n * sizeof(float), &d)) return rc;
    *dev = reinterpret_cast<const float*>(d);
    return CELLM_HIP_OK;
}

void out_in(const cellm_llama_config_t& c, int j, size_t* out, size_t* in)
{
    const size_t hid = (size_t)c.hidden, kv = (size_t)c.n_kv_heads * c.head_dim, inter = (size_t)c.intermediate;
    const size_t o[7] = {hid, kv, kv, hid, inter, inter, hid};
    const size_t i[7] = {hid, hid, hid, hid, hid, hid, inter};
    *out = o[j];
    *in = i[j];
}


// One projection y[R][out] = W x[R][in] by its weight format.
int32_t run_proj(cellm_llama_dev* m, const Proj& pr, const float* x, float* y, int64_t R, int64_t out, int64_t in,
                 const char* what)
{
    cellm_hip_ctx_t* H = m->hip;
    void* S = m->stream;
    if (pr.kind == PK_I8) {  // the bias rides in the GEMV's epilogue
        LIB_TRY(cellm_hip_qgemv_i8(H, static_cast<const int8_t*>(pr.w), pr.s, CELLM_HIP_DTYPE_F16, out, x,
                                   CELLM_HIP_DTYPE_F32, pr.bias, y, R, out, in, S),
                what);
        return CELLM_HIP_OK;
    }
    if (pr.kind == PK_Q4) {
        LIB_TRY(cellm_hip_qgemv_q4_affine(H, static_cast<const uint32_t*>(pr.w), pr.s, pr.b, CELLM_HIP_DTYPE_F32, 64,
                                          x, CELLM_HIP_DTYPE_F32, y, R, out, in, S),
                what);
    } else if (pr.kind == PK_I4) {
        LIB_TRY(cellm_hip_qgemv_i4_sym(H, static_cast<const uint8_t*>(pr.w), static_cast<const uint16_t*>(pr.s),
                                       pr.ns ? pr.ns : out, pr.gs ? pr.gs : in, x, CELLM_HIP_DTYPE_F32, y, R, out, in,
                                       S),
                what);
    } else if (pr.kind == PK_I2) {
        LIB_TRY(cellm_hip_qgemv_i2(H, static_cast<const uint8_t*>(pr.w), static_cast<const uint16_t*>(pr.s), 0, x,
                                   CELLM_HIP_DTYPE_F32, y, R, out, in, S),
                what);
    } else if (pr.kind == PK_Q1) {
        LIB_TRY(cellm_hip_qgemv_q1_0_g128(H, static_cast<const uint8_t*>(pr.w), x, CELLM_HIP_DTYPE_F32, y, R, out, in,
                                          S),
                what);
    } else {
        LIB_TRY(cellm_hip_qgemv_f16(H, static_cast<const uint16_t*>(pr.w), x, CELLM_HIP_DTYPE_F32, y, R, out, in, S),
                what);
    }
    // add_projection_bias_if_present (qwen.rs:1132-1139); the bias holds max_rows copies
    if (pr.bias) LIB_TRY(cellm_hip_add_f32_inplace(H, y, pr.bias, R * out, S), what);
    return CELLM_HIP_OK;
}

// The step's device work for `rows` sessions, enqueued on the runner's stream:
// inputs are read from io (tokens, positions, block tables), the greedy ids
// and logits are left in io and m->logits.  Only kernel launches: no
// allocation, copy or synchronisation, so the sequence can be captured.
int32_t enqueue_step(cellm_llama_dev* m, int32_t rows)
{
    const cellm_llama_config_t& c = m->cfg;
    const int64_t tpb = c.tokens_per_block, MB = m->max_blocks;
    unsigned char* dio = m->io.as<unsigned char>();
    const uint32_t* d_tok = reinterpret_cast<const uint32_t*>(dio + m->io_tokens);
    const int32_t* d_pos = reinterpret_cast<const int32_t*>(dio + m->io_pos);
    const uint32_t* d_bt = reinterpret_cast<const uint32_t*>(dio + m->io_bt);
    uint64_t* d_keys = reinterpret_cast<uint64_t*>(dio + m->io_keys);

    const int64_t R = rows, hid = c.hidden, kvd = (int64_t)m->kvd, inter = c.intermediate, vocab = c.vocab;
    const int64_t L = c.n_layers;
    float *x = m->x.as<float>(), *xn = m->xn.as<float>(), *q = m->q.as<float>(), *k = m->k.as<float>();
    float *v = m->v.as<float>(), *attn = m->attn.as<float>(), *proj = m->proj.as<float>(), *h = m->h.as<float>();
    uint16_t *kc = m->kcache.as<uint16_t>(), *vc = m->vcache.as<uint16_t>();
    cellm_hip_ctx_t* H = m->hip;
    void* S = m->stream;
    const float eps = c.rms_norm_eps;
    auto i8w = [](const Proj& pr) { return static_cast<const int8_t*>(pr.w); };
    auto i8s = [](const Proj& pr) { return static_cast<const uint16_t*>(pr.s); };

    const Proj& E = m->embed;
    if (E.kind == PK_I8)
        LIB_TRY(cellm_hip_embed_i8(H, d_tok, R, static_cast<const int8_t*>(E.w), static_cast<const uint16_t*>(E.s),
                                   vocab, hid, x, S),
                "embed");
    else if (E.kind == PK_I4)
        LIB_TRY(cellm_hip_embed_i4(H, d_tok, R, static_cast<const uint8_t*>(E.w), static_cast<const uint16_t*>(E.s),
                                   vocab, hid, x, S),
                "embed");
    else
        LIB_TRY(cellm_hip_embed_f16(H, d_tok, R, static_cast<const uint16_t*>(E.w), vocab, hid, x, S), "embed");
    if (m->fused || m->fused_q4) {
        // 5 launches per layer; the residual stream alternates between x and x2
        float* x2 = m->x2.as<float>();
        auto u32w = [](const Proj& pr) { return static_cast<const uint32_t*>(pr.w); };
        for (int64_t l = 0; l < L; ++l) {
            const Proj* P = &m->p[l * 7];
            const float* yl = l == 0 ? nullptr : proj;
            if (m->fused)
                LIB_TRY(cellm_hip_decode_qkv_rope_kv(H, x, yl, x2, m->attn_norm[l], eps, i8w(P[0]), i8s(P[0]),
                                                     i8w(P[1]), i8s(P[1]), i8w(P[2]), i8s(P[2]), R, hid, c.n_heads,
                                                     c.n_kv_heads, c.head_dim, d_pos, m->rope.as<float>(),
                                                     m->table_positions, q, kc, vc, d_bt, MB, c.total_blocks, L, tpb,
                                                     l, S),
                        "residual + input_layernorm + qkv + rope + kv write");
            else
                LIB_TRY(cellm_hip_decode_q4_affine_qkv_rope_kv(
                            H, x, yl, x2, m->attn_norm[l], eps, u32w(P[0]), P[0].s, P[0].b, P[0].bias, u32w(P[1]),
                            P[1].s, P[1].b, P[1].bias, u32w(P[2]), P[2].s, P[2].b, P[2].bias, CELLM_HIP_DTYPE_F32, 64,
                            R, hid, c.n_heads, c.n_kv_heads, c.head_dim, d_pos, m->rope.as<float>(),
                            m->table_positions, q, kc, vc, d_bt, MB, c.total_blocks, L, tpb, l, S),
                        "residual + input_layernorm + q4 qkv + bias + rope + kv write");
            LIB_TRY(cellm_hip_attention_gqa_f16kv(H, q, kc, vc, d_bt, MB, c.total_blocks, d_pos, R, c.n_heads,
                                                  c.n_kv_heads, c.head_dim, L, tpb, l, 0.0f, 0.0f, attn, S),
                    "attention");
            if (int32_t rc = run_proj(m, P[3], attn, proj, R, hid, hid, "o_proj")) return rc;
            if (m->fused)
                LIB_TRY(cellm_hip_decode_gate_up_silu(H, x2, proj, x, m->mlp_norm[l], eps, i8w(P[4]), i8s(P[4]),
                                                      i8w(P[5]), i8s(P[5]), R, hid, inter, h, S),
                        "residual + post_attention_layernorm + gate/up");
            else
                LIB_TRY(cellm_hip_decode_q4_affine_gate_up_silu(H, x2, proj, x, m->mlp_norm[l], eps, u32w(P[4]),
                                                                P[4].s, P[4].b, u32w(P[5]), P[5].s, P[5].b,
                                                                CELLM_HIP_DTYPE_F32, 64, R, hid, inter, h, S),
                        "residual + post_attention_layernorm + q4 gate/up");
            if (int32_t rc = run_proj(m, P[6], h, proj, R, hid, inter, "down_proj")) return rc;
        }
        LIB_TRY(cellm_hip_add_rms_norm(H, x, proj, m->final_norm, CELLM_HIP_DTYPE_F32, R, hid, eps, xn, S),
                "residual + norm");
    } else {
        LIB_TRY(cellm_hip_rms_norm(H, x, m->attn_norm[0], CELLM_HIP_DTYPE_F32, R, hid, eps, xn, S), "input_layernorm");
        for (int64_t l = 0; l < L; ++l) {
            const Proj* P = &m->p[l * 7];
            // xn = input_layernorm(x), from the previous layer's residual add (or the embedding)
            if (P[0].kind == PK_I8 && P[1].kind == PK_I8 && P[2].kind == PK_I8) {
                LIB_TRY(cellm_hip_qgemv_i8_qkv(H, i8w(P[0]), i8s(P[0]), hid, P[0].bias, i8w(P[1]), i8s(P[1]), kvd,
                                               P[1].bias, i8w(P[2]), i8s(P[2]), kvd, P[2].bias, CELLM_HIP_DTYPE_F16,
                                               xn, CELLM_HIP_DTYPE_F32, q, k, v, R, hid, kvd, hid, S),
                        "qkv");
            } else if (P[0].kind == PK_Q4 && P[1].kind == PK_Q4 && P[2].kind == PK_Q4) {
                // the three MLX affine projections in one launch, biases in its epilogue
                LIB_TRY(cellm_hip_qgemv_q4_affine_qkv(H, static_cast<const uint32_t*>(P[0].w), P[0].s, P[0].b,
                                                      P[0].bias, static_cast<const uint32_t*>(P[1].w), P[1].s, P[1].b,
                                                      P[1].bias, static_cast<const uint32_t*>(P[2].w), P[2].s, P[2].b,
                                                      P[2].bias, CELLM_HIP_DTYPE_F32, 64, xn, CELLM_HIP_DTYPE_F32, q,
                                                      k, v, R, hid, kvd, hid, S),
                        "qkv");
            } else {
                if (int32_t rc = run_proj(m, P[0], xn, q, R, hid, hid, "q_proj")) return rc;
                if (int32_t rc = run_proj(m, P[1], xn, k, R, kvd, hid, "k_proj")) return rc;
                if (int32_t rc = run_proj(m, P[2], xn, v, R, kvd, hid, "v_proj")) return rc;
            }
            LIB_TRY(cellm_hip_rope_kv_write_f16(H, q, k, v, R, c.n_heads, c.n_kv_heads, c.head_dim, d_pos,
                                                m->rope.as<float>(), m->table_positions, kc, vc, d_bt, MB,
                                                c.total_blocks, L, tpb, l, S),
                    "rope + kv write");
            LIB_TRY(cellm_hip_attention_gqa_f16kv(H, q, kc, vc, d_bt, MB, c.total_blocks, d_pos, R, c.n_heads,
                                                  c.n_kv_heads, c.head_dim, L, tpb, l, 0.0f, 0.0f, attn, S),
                    "attention");
            if (int32_t rc = run_proj(m, P[3], attn, proj, R, hid, hid, "o_proj")) return rc;
            LIB_TRY(cellm_hip_add_rms_norm(H, x, proj, m->mlp_norm[l], CELLM_HIP_DTYPE_F32, R, hid, eps, xn, S),
                    "residual + post_attention_layernorm");
            if (P[4].kind == PK_I8 && P[5].kind == PK_I8) {
                LIB_TRY(cellm_hip_qgemv_i8_gate_up_silu(H, i8w(P[4]), i8s(P[4]), inter, P[4].bias, i8w(P[5]),
                                                        i8s(P[5]), inter, P[5].bias, CELLM_HIP_DTYPE_F16, xn,
                                                        CELLM_HIP_DTYPE_F32, h, R, inter, hid, S),
                        "gate/up");
            } else if (P[4].kind == PK_Q4 && P[5].kind == PK_Q4 && !P[4].bias && !P[5].bias) {
                LIB_TRY(cellm_hip_qgemv_q4_affine_gate_up_silu(
                            H, static_cast<const uint32_t*>(P[4].w), P[4].s, P[4].b,
                            static_cast<const uint32_t*>(P[5].w), P[5].s, P[5].b, CELLM_HIP_DTYPE_F32, 64, xn,
                            CELLM_HIP_DTYPE_F32, h, R, inter, hid, S),
                        "gate/up");
            } else {
                float* upb = m->up.as<float>();
                if (int32_t rc = run_proj(m, P[4], xn, h, R, inter, hid, "gate_proj")) return rc;
                if (int32_t rc = run_proj(m, P[5], xn, upb, R, inter, hid, "up_proj")) return rc;
                LIB_TRY(cellm_hip_silu_mul_f32(H, h, upb, R * inter, S), "silu * up");
            }
            if (int32_t rc = run_proj(m, P[6], h, proj, R, hid, inter, "down_proj")) return rc;
            // residual, then the next layer's input_layernorm (the final norm after the last layer)
            const float* next_norm = l + 1 < L ? m->attn_norm[l + 1] : m->final_norm;
            LIB_TRY(cellm_hip_add_rms_norm(H, x, proj, next_norm, CELLM_HIP_DTYPE_F32, R, hid, eps, xn, S),
                    "residual + norm");
        }
    }
    // lm_head (tied embedding or lm_head.weight, llama.rs:522-567), greedy id on the device
    float* lg = m->logits.as<float>();
    if (int32_t rc = run_proj(m, m->lm, xn, lg, R, vocab, hid, "lm_head")) return rc;
    // greedy id as a packed key per row (the upload of the step inputs zeroes the keys)
    LIB_TRY(cellm_hip_argmax_f32_keys(H, lg, R, vocab, d_keys, S), "argmax");
    return CELLM_HIP_OK;
}

// Size every scratch buffer of the HIP context for all row counts, then
// capture one graph per row count.  The context grows a per-stream scratch
// buffer (split-K partials, attention partials) on the first call that needs
// more and never shrinks it, so after one eager step at each row count no
// later step reallocates, and the captured kernel arguments stay valid.  The
// eager steps run at position 0 on block 0 and the K/V cache is cleared
// afterwards.
// A captured step must hold kernel launches only (no copy, memset or host
// node: those would tie the graph to host buffers or record a clear), each
// with a function and a non-empty grid.  Checked once per captured graph.
int32_t check_step_graph(hipGraph_t g, int32_t rows)
{
    size_t n = 0;
    RT_TRY(hipGraphGetNodes(g, nullptr, &n), "hipGraphGetNodes(count)");
    if (n == 0) return fail(CELLM_HIP_ERR_DEVICE, "captured step for %d rows is empty", rows);
    std::vector<hipGraphNode_t> nodes(n);
    RT_TRY(hipGraphGetNodes(g, nodes.data(), &n), "hipGraphGetNodes");
    for (size_t i = 0; i < n; ++i) {
        hipGraphNodeType type;
        RT_TRY(hipGraphNodeGetType(nodes[i], &type), "hipGraphNodeGetType");
        if (type != hipGraphNodeTypeKernel)
            return fail(CELLM_HIP_ERR_DEVICE, "captured step for %d rows: node %zu has type %d, not a kernel", rows, i,
                        (int)type);
        hipKernelNodeParams kp{};
        RT_TRY(hipGraphKernelNodeGetParams(nodes[i], &kp), "hipGraphKernelNodeGetParams");
        if (!kp.func || kp.gridDim.x == 0 || kp.gridDim.y == 0 || kp.gridDim.z == 0 || kp.blockDim.x == 0)
            return fail(CELLM_HIP_ERR_DEVICE, "captured step for %d rows: kernel node %zu has no function or grid", rows,
                        i);
    }
    return CELLM_HIP_OK;
}

int32_t prepare_graphs(cellm_llama_dev* m)
{
    const hipStream_t st = reinterpret_cast<hipStream_t>(m->stream);
    memset(m->host_io, 0, m->io_bytes);
    RT_TRY(hipMemcpyAsync(m->io.p, m->host_io, m->io_bytes, hipMemcpyHostToDevice, st), "clear step io");
    for (int32_t r = 1; r <= m->max_rows; ++r)
        if (int32_t rc = enqueue_step(m, r)) return rc;
    RT_TRY(hipStreamSynchronize(st), "warm-up steps");
    RT_TRY(hipMemsetAsync(m->kcache.p, 0, m->kv_elems * 2, st), "clear K cache");
    RT_TRY(hipMemsetAsync(m->vcache.p, 0, m->kv_elems * 2, st), "clear V cache");
    RT_TRY(hipStreamSynchronize(st), "clear K/V cache");
    for (int32_t r = 1; r <= m->max_rows; ++r) {
        RT_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        const int32_t rc = enqueue_step(m, r);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return from_runtime(e, "hipStreamEndCapture");
        m->graph[r - 1] = g;
        if (int32_t rc2 = check_step_graph(g, r)) return rc2;
        RT_TRY(hipGraphInstantiate(&m->graph_exec[r - 1], g, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    m->use_graphs = true;
    return CELLM_HIP_OK;
}

int32_t dev_create_impl(const cellm_llama_config_t* cfg, const HostModel& hm, int32_t device, int32_t max_rows,
                        int32_t max_blocks, cellm_llama_dev_t** out);

}  // namespace

extern "C" {

int32_t cellm_llama_rope_table(float theta, int32_t head_dim, int32_t positions, float* out)
{
    CELLM_API_BEGIN
    if (!out || head_dim <= 0 || head_dim % 2 || positions <= 0)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "bad rope table arguments");
    const int32_t half = head_dim / 2;
    for (int32_t p = 0; p < positions; ++p)
        for (int32_t i = 0; i < half; ++i) {
            // rope_non_interleaved_inplace_f32 (cpu_kernels.rs:264-277), f32 throughout
            const float inv_freq = std::pow(theta, -(2.0f * (float)i) / (float)head_dim);
            const float angle = (float)p * inv_freq;
            out[((size_t)p * half + i) * 2] = std::cos(angle);
            out[((size_t)p * half + i) * 2 + 1] = std::sin(angle);
        }
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_dev_create(const cellm_llama_config_t* cfg, const cellm_llama_layer_t* layers,
                               const int8_t* embed_i8, const uint16_t* embed_scale_f16,
                               const uint16_t* final_norm_f16, int32_t device, int32_t max_rows, int32_t max_blocks,
                               cellm_llama_dev_t** out)
{
    CELLM_API_BEGIN
    if (!cfg || !layers || !embed_i8 || !embed_scale_f16 || !final_norm_f16 || !out)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (cfg->n_layers <= 0 || cfg->n_layers > 4096) return fail(CELLM_HIP_ERR_INVALID_ARG, "bad n_layers");
    HostModel hm;
    for (int32_t l = 0; l < cfg->n_layers; ++l) {
        for (int j = 0; j < 7; ++j) {
            size_t o, i;
            out_in(*cfg, j, &o, &i);
            HostProj hp;
            hp.kind = PK_I8;
            hp.w = layers[l].w[j];
            hp.w_bytes = o * i;
            hp.s = layers[l].scale_f16[j];
            hp.s_bytes = o * 2;
            hm.p.push_back(hp);
        }
        hm.n1.push_back(layers[l].input_layernorm_f16);
        hm.n2.push_back(layers[l].post_attention_layernorm_f16);
    }
    hm.embed.kind = PK_I8;
    hm.embed.w = embed_i8;
    hm.embed.w_bytes = (size_t)cfg->vocab * (size_t)cfg->hidden;
    hm.embed.s = embed_scale_f16;
    hm.embed.s_bytes = (size_t)cfg->vocab * 2;
    hm.final_norm = final_norm_f16;
    hm.rope_interleaved = cellm_step::llama_rope_interleaved_from_env();
    return dev_create_impl(cfg, hm, device, max_rows, max_blocks, out);
    CELLM_API_END(cellm_step::report_exception)
}

}  // extern "C"

namespace {

int32_t dev_create_impl(const cellm_llama_config_t* cfg, const HostModel& hm, int32_t device, int32_t max_rows,
                        int32_t max_blocks, cellm_llama_dev_t** out)
{
    if (!cfg || !hm.embed.w || (hm.embed.kind != PK_F16 && !hm.embed.s) || !hm.final_norm || !out)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (hm.embed.kind != PK_I8 && hm.embed.kind != PK_I4 && hm.embed.kind != PK_F16)
        return fail(CELLM_HIP_ERR_UNSUPPORTED, "embedding format %d is not i8, i4 or f16", hm.embed.kind);
    *out = nullptr;
    const cellm_llama_config_t& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate <= 0 || c.vocab <= 0 || c.tokens_per_block <= 0 || c.total_blocks <= 0)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "non-positive dimension in config");
    if (c.head_dim * c.n_heads != c.hidden)  // llama.rs:285-289
        return fail(CELLM_HIP_ERR_INVALID_ARG, "hidden_size must equal num_heads * head_dim");
    if (c.n_heads % c.n_kv_heads != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "n_heads %% n_kv_heads != 0");
    if (max_rows < 1 || max_rows > 4) return fail(CELLM_HIP_ERR_INVALID_ARG, "max_rows must be 1..4");
    if (max_blocks < 1 || max_blocks > c.total_blocks)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "max_blocks must be 1..total_blocks");
    if (hm.p.size() != (size_t)c.n_layers * 7 || hm.n1.size() != (size_t)c.n_layers ||
        hm.n2.size() != (size_t)c.n_layers)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "projection list does not match n_layers");
    auto* m = new cellm_llama_dev();
    m->cfg = c;
    m->max_rows = max_rows;
    m->max_blocks = max_blocks;
    m->device = device;
    m->kvd = (size_t)c.n_kv_heads * c.head_dim;
    m->table_positions = max_blocks * c.tokens_per_block;
    auto bail = [&](int32_t rc) {
        cellm_llama_dev_destroy(m);
        return rc;
    };
    int32_t rc = cellm_hip_create(device, &m->hip);
    if (rc) {
        m->hip = nullptr;
        return bail(from_hip_lib(rc, "cellm_hip_create"));
    }
    if ((rc = cellm_hip_get_stream(m->hip, &m->stream))) return bail(from_hip_lib(rc, "cellm_hip_get_stream"));
    if ((rc = cellm_hip_set_rope_interleaved(m->hip, hm.rope_interleaved ? 1 : 0)))
        return bail(from_hip_lib(rc, "cellm_hip_set_rope_interleaved"));
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(device) != hipSuccess)
        return bail(fail(CELLM_HIP_ERR_DEVICE, "hipSetDevice(%d) failed", device));
    const size_t hid = (size_t)c.hidden, L = (size_t)c.n_layers;
    // the cache keys follow the .cellm tensor names of each format
    auto upload_proj = [&](const std::string& base, const HostProj& hp, Proj* pr) -> int32_t {
        const bool scaled = hp.kind != PK_F16 && hp.kind != PK_Q1;
        if (!hp.w || (scaled && !hp.s) || (hp.kind == PK_Q4 && !hp.b))
            return fail(CELLM_HIP_ERR_INVALID_ARG, "%s: weight or scale data missing", base.c_str());
        const void *dw = nullptr, *ds = nullptr, *db = nullptr;
        if (int32_t r = upload(m, base + ".weight", hp.w, hp.w_bytes, &dw)) return r;
        if (hp.kind == PK_Q4) {
            if (int32_t r = upload(m, base + ".scales", hp.s, hp.s_bytes, &ds)) return r;
            if (int32_t r = upload(m, base + ".biases", hp.b, hp.b_bytes, &db)) return r;
        } else if (scaled) {
            if (int32_t r = upload(m, base + ".weight.qscale", hp.s, hp.s_bytes, &ds)) return r;
        }
        pr->kind = hp.kind;
        pr->w = dw;
        pr->s = ds;
        pr->b = db;
        pr->ns = hp.ns;
        pr->gs = hp.gs;
        pr->bias = nullptr;
        if (hp.bias_f16) {
            // widened to f32 once at upload (qwen.rs:232-239) and repeated for each of the max_rows rows, so one
            // elementwise add covers a whole batch
            std::vector<float> rep((size_t)max_rows * hp.bias_n);
            for (int32_t r = 0; r < max_rows; ++r)
                for (size_t j = 0; j < hp.bias_n; ++j) rep[(size_t)r * hp.bias_n + j] = h2f(hp.bias_f16[j]);
            const void* d = nullptr;
            if (int32_t r = upload(m, base + ".bias", rep.data(), rep.size() * sizeof(float), &d)) return r;
            pr->bias = static_cast<const float*>(d);
        }
        return CELLM_HIP_OK;
    };
    m->p.resize(L * 7);
    bool all_i8 = true, q4_fusable = true;
    for (size_t l = 0; l < L; ++l) {
        const std::string pre = "model.layers." + std::to_string(l) + ".";
        for (int j = 0; j < 7; ++j) {
            if ((rc = upload_proj(pre + kNames[j], hm.p[l * 7 + j], &m->p[l * 7 + j]))) return bail(rc);
            all_i8 = all_i8 && hm.p[l * 7 + j].kind == PK_I8 && !hm.p[l * 7 + j].bias_f16;
            // q/k/v (j < 3) and gate/up (j = 4, 5) in the fused q4 launches; gate/up without biases
            if (j != 3 && j != 6)
                q4_fusable = q4_fusable && hm.p[l * 7 + j].kind == PK_Q4 && (j < 3 || !hm.p[l * 7 + j].bias_f16);
        }
        const float *a = nullptr, *b = nullptr;
        if (!hm.n1[l] || !hm.n2[l]) return bail(fail(CELLM_HIP_ERR_INVALID_ARG, "layer %zu norm missing", l));
        if ((rc = upload_norm(m, pre + "input_layernorm.weight", hm.n1[l], hid, &a)) ||
            (rc = upload_norm(m, pre + "post_attention_layernorm.weight", hm.n2[l], hid, &b)))
            return bail(rc);
        m->attn_norm.push_back(a);
        m->mlp_norm.push_back(b);
    }
    if ((rc = upload_proj("model.embed_tokens", hm.embed, &m->embed)) ||
        (rc = upload_norm(m, "model.norm.weight", hm.final_norm, hid, &m->final_norm)))
        return bail(rc);
    m->lm = m->embed;  // tied: the lm_head reads the embedding in its own format
    if (hm.lm.w && (rc = upload_proj("lm_head", hm.lm, &m->lm))) return bail(rc);

    // paged K/V (KvCacheLayout: total_blocks x layers x tokens_per_block x kv_dim), zeroed
    m->kv_elems = (size_t)c.total_blocks * L * c.tokens_per_block * m->kvd;
    const size_t R = (size_t)max_rows, inter = (size_t)c.intermediate;
    if ((rc = m->kcache.alloc(m->kv_elems * 2, "hipMalloc(K cache)")) ||
        (rc = m->vcache.alloc(m->kv_elems * 2, "hipMalloc(V cache)")) ||
        (rc = m->rope.alloc((size_t)m->table_positions * c.head_dim * sizeof(float), "hipMalloc(rope table)")) ||
        (rc = m->x.alloc(R * hid * 4, "hipMalloc(x)")) || (rc = m->x2.alloc(R * hid * 4, "hipMalloc(x2)")) ||
        (rc = m->xn.alloc(R * hid * 4, "hipMalloc(xn)")) ||
        (rc = m->q.alloc(R * hid * 4, "hipMalloc(q)")) || (rc = m->k.alloc(R * m->kvd * 4, "hipMalloc(k)")) ||
        (rc = m->v.alloc(R * m->kvd * 4, "hipMalloc(v)")) || (rc = m->attn.alloc(R * hid * 4, "hipMalloc(attn)")) ||
        (rc = m->proj.alloc(R * hid * 4, "hipMalloc(proj)")) || (rc = m->h.alloc(R * inter * 4, "hipMalloc(h)")) ||
        (rc = m->up.alloc(R * inter * 4, "hipMalloc(up)")) ||
        (rc = m->logits.alloc(R * (size_t)c.vocab * 4, "hipMalloc(logits)")))
        return bail(rc);
    hipError_t e = hipMemset(m->kcache.p, 0, m->kv_elems * 2);
    if (e == hipSuccess) e = hipMemset(m->vcache.p, 0, m->kv_elems * 2);
    if (e != hipSuccess) return bail(from_runtime(e, "hipMemset(K/V cache)"));
    {
        std::vector<float> table((size_t)m->table_positions * c.head_dim);
        if ((rc = cellm_llama_rope_table(c.rope_theta, c.head_dim, m->table_positions, table.data()))) return bail(rc);
        e = hipMemcpy(m->rope.p, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) return bail(from_runtime(e, "upload rope table"));
    }
    m->fused = all_i8 && (c.hidden % 16) == 0 && c.hidden <= 4096 && c.head_dim % 2 == 0;
    m->fused_q4 = !m->fused && q4_fusable && (c.hidden % 32) == 0 && c.hidden >= 64 && c.hidden <= 4096 &&
                  c.head_dim % 2 == 0;
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    m->io_tokens = 0;
    m->io_pos = align(R * 4);
    m->io_bt = m->io_pos + align(R * 4);
    m->io_keys = m->io_bt + align(R * (size_t)max_blocks * 4);
    m->io_bytes = m->io_keys + align(R * 8);
    if ((rc = m->io.alloc(m->io_bytes, "hipMalloc(step io)"))) return bail(rc);
    e = hipHostMalloc(&m->host_io, m->io_bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        m->host_io = nullptr;
        return bail(from_runtime(e, "hipHostMalloc(step io)"));
    }
    if ((rc = prepare_graphs(m))) return bail(rc);
    (void)hipSetDevice(prev);
    *out = m;
    return CELLM_HIP_OK;
}

}  // namespace

extern "C" {

void cellm_llama_dev_destroy(cellm_llama_dev_t* m)
{
    CELLM_API_BEGIN
    if (!m) return;
    if (m->hip) (void)cellm_hip_synchronize(m->hip);
    for (int r = 0; r < 4; ++r) {
        if (m->graph_exec[r]) (void)hipGraphExecDestroy(m->graph_exec[r]);
        if (m->graph[r]) (void)hipGraphDestroy(m->graph[r]);
    }
    if (m->host_io) (void)hipHostFree(m->host_io);
    m->host_io = nullptr;
    // device buffers free themselves; the weight cache goes with the context
    cellm_hip_ctx_t* hip = m->hip;
    delete m;
    if (hip) cellm_hip_destroy(hip);
    CELLM_API_END_VOID
}

int32_t cellm_llama_dev_create_from_file(const char* path, int32_t device, int32_t max_rows, int32_t max_blocks,
                                         int32_t tokens_per_block, int32_t total_blocks, cellm_llama_dev_t** out)
{
    CELLM_API_BEGIN
    if (!path || !out) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    cellm_file_t* f = nullptr;
    if (int32_t rc = cellm_file_open(path, &f)) return from_hip_lib(rc, "cellm_file_open");
    struct Closer {
        cellm_file_t* f;
        ~Closer() { cellm_file_close(f); }
    } closer{f};
    cellm_file_config_t fc;
    if (int32_t rc = cellm_file_config(f, &fc)) return from_hip_lib(rc, "cellm_file_config");
    // LlamaRunner::load (llama.rs:39-53): head_dim defaults to hidden / heads
    const int64_t head_dim = fc.head_dim > 0 ? fc.head_dim : (fc.num_heads > 0 ? fc.hidden_dim / fc.num_heads : 0);
    const int64_t dims[] = {fc.num_layers, fc.hidden_dim, fc.num_heads, fc.num_kv_heads, head_dim,
                            fc.intermediate_size, fc.vocab_size};
    for (int64_t d : dims)
        if (d <= 0 || d > INT32_MAX) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: bad model dimension");
    cellm_llama_config_t c{};
    c.n_layers = (int32_t)fc.num_layers;
    c.hidden = (int32_t)fc.hidden_dim;
    c.n_heads = (int32_t)fc.num_heads;
    c.n_kv_heads = (int32_t)fc.num_kv_heads;
    c.head_dim = (int32_t)head_dim;
    c.intermediate = (int32_t)fc.intermediate_size;
    c.vocab = (int32_t)fc.vocab_size;
    c.rms_norm_eps = fc.rms_norm_eps;
    c.rope_theta = fc.rope_theta;
    c.tokens_per_block = tokens_per_block;
    c.total_blocks = total_blocks;

    // The runner family from the header's model_type, as the SDK picks a runner
    // (crates/cellm-sdk/src/lib.rs:125-135): "qwen*" runs the Qwen2 layer, anything else the Llama one.
    const std::string model_type = fc.model_type;
    const int32_t family = model_type.compare(0, 4, "qwen") == 0 ? FAM_QWEN : FAM_LLAMA;
    if (family == FAM_QWEN && model_type.find("qwen3_5") != std::string::npos)
        return fail(CELLM_HIP_ERR_UNSUPPORTED,
                    "model_type %s (linear-attention layers, offset norms) is not supported by the device step",
                    model_type.c_str());
    auto has = [&](const std::string& n) { return cellm_file_find(f, n.c_str(), nullptr) == CELLM_HIP_OK; };
    // Tensor names are base + "layers.N.…", base + "norm.weight", base + "embed_tokens.weight".
    std::string base;
    if (family == FAM_LLAMA) {
        // detect_llama_prefix (llama.rs:1094-1113)
        bool found = false;
        for (const char* p : {"", "language_model."}) {
            const std::string b = std::string(p) + "model.";
            if (has(b + "embed_tokens.weight") && has(b + "norm.weight")) {
                base = b;
                found = true;
                break;
            }
        }
        if (!found)
            return fail(CELLM_HIP_ERR_NOT_FOUND,
                        "missing required llama tensors: model.embed_tokens.weight/model.norm.weight");
    } else {
        // the prefix order of QwenRunner::step_inner (qwen.rs:339-342)
        bool found = false;
        for (const char* p : {"model.language_model.", "language_model.model.", "model."}) {
            if (has(std::string(p) + "embed_tokens.weight")) {
                base = p;
                found = true;
                break;
            }
        }
        if (!found) base = "";
        // per-head q/k RMSNorms (qwen.rs:433-468) sit between the projections and RoPE: not in this step
        for (int32_t l = 0; l < c.n_layers; ++l)
            for (const char* nm : {"self_attn.q_norm.weight", "self_attn.k_norm.weight"})
                if (has(base + "layers." + std::to_string(l) + "." + nm))
                    return fail(CELLM_HIP_ERR_UNSUPPORTED, "%slayers.%d.%s: q/k norms are not supported by the "
                                "device step", base.c_str(), l, nm);
    }
    // a tensor of the given dtype and shape ([d0] when d1 < 0) holding `nbytes`, as mapped bytes
    auto tensor = [&](const std::string& name, const char* dtype, int64_t d0, int64_t d1, uint64_t nbytes,
                      const void** p) -> int32_t {
        cellm_file_tensor_t t;
        if (cellm_file_find(f, name.c_str(), &t) != CELLM_HIP_OK)
            return fail(CELLM_HIP_ERR_NOT_FOUND, "tensor %s missing", name.c_str());
        if (strcmp(t.dtype, dtype) != 0)
            return fail(CELLM_HIP_ERR_UNSUPPORTED, "tensor %s is %s; the device step takes %s", name.c_str(), t.dtype,
                        dtype);
        const bool shape_ok = d1 < 0 ? (t.ndim == 1 && t.shape[0] == d0)
                                     : (t.ndim == 2 && t.shape[0] == d0 && t.shape[1] == d1);
        if (!shape_ok || t.nbytes != nbytes)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s has shape/bytes that do not match the config",
                        name.c_str());
        return cellm_file_tensor_bytes(f, name.c_str(), p, nullptr) == CELLM_HIP_OK
                   ? CELLM_HIP_OK
                   : fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s unreadable", name.c_str());
    };
    // One projection [o, i] by the dtype of its weight tensor, as the runners'
    // linear_f16_out_in dispatch on it (llama.rs:781-941, lfm.rs:924-981,
    // gemma.rs:1358-1499).
    auto load_proj = [&](const std::string& w, int64_t o, int64_t i, HostProj* hp, bool rows_only) -> int32_t {
        cellm_file_tensor_t t;
        if (cellm_file_find(f, w.c_str(), &t) != CELLM_HIP_OK)
            return fail(CELLM_HIP_ERR_NOT_FOUND, "tensor %s missing", w.c_str());
        if (strcmp(t.dtype, "i8") == 0) {
            hp->kind = PK_I8;
            hp->w_bytes = (size_t)(o * i);
            hp->s_bytes = (size_t)o * 2;
            if (int32_t rc = tensor(w, "i8", o, i, hp->w_bytes, &hp->w)) return rc;
            return tensor(w + ".qscale", "f16", o, -1, hp->s_bytes, &hp->s);
        }
        if (strcmp(t.dtype, "u32") == 0) {
            // MLX affine: [o, i/8] words; f32 scales/biases [o, ceil(i/64)] named by the weight's base
            // ("<base>.scales" for "<base>.weight", lfm.rs:932-941; tools/convert_lfm.py:123-136)
            if (i % 8 != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "%s: in_dim %lld not a multiple of 8", w.c_str(),
                                        (long long)i);
            const std::string base = w.size() > 7 && w.compare(w.size() - 7, 7, ".weight") == 0
                                         ? w.substr(0, w.size() - 7)
                                         : w;
            const int64_t groups = (i + 63) / 64;
            hp->kind = PK_Q4;
            hp->w_bytes = (size_t)(o * i / 2);
            hp->s_bytes = hp->b_bytes = (size_t)(o * groups * 4);
            if (int32_t rc = tensor(w, "u32", o, i / 8, hp->w_bytes, &hp->w)) return rc;
            if (int32_t rc = tensor(base + ".scales", "f32", o, groups, hp->s_bytes, &hp->s)) return rc;
            return tensor(base + ".biases", "f32", o, groups, hp->b_bytes, &hp->b);
        }
        if (strcmp(t.dtype, "i4") == 0) {
            // [o, i] with ceil(i/2) bytes per row (i4_packed_nbytes_for_shape) and f16 .qscale.  Per row
            // (rows_only, the embedding and lm_head loops read scales[row]) or as matmul_i4_f32 reads
            // them for a projection: spr = count / o scales per row, gs = i for Llama (llama.rs:932, the
            // row's first scale) and i / spr for Qwen when spr > 1 (qwen.rs:1076-1077).
            hp->kind = PK_I4;
            hp->w_bytes = (size_t)(o * ((i + 1) / 2));
            if (int32_t rc = tensor(w, "i4", o, i, hp->w_bytes, &hp->w)) return rc;
            cellm_file_tensor_t st;
            const std::string sn = w + ".qscale";
            if (cellm_file_find(f, sn.c_str(), &st) != CELLM_HIP_OK)
                return fail(CELLM_HIP_ERR_NOT_FOUND, "tensor %s missing", sn.c_str());
            const int64_t count = (int64_t)(st.nbytes / 2);
            if (strcmp(st.dtype, "f16") != 0 || count < o || count % o != 0 || (rows_only && count != o))
                return fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s: %lld f16 scales for %lld rows", sn.c_str(),
                            (long long)count, (long long)o);
            const int64_t spr = count / o;
            hp->ns = count;
            hp->gs = (family == FAM_QWEN && spr > 1) ? i / spr : i;
            if (hp->gs < 1 || (i - 1) / hp->gs >= spr)
                return fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s: %lld scales per row do not cover %lld columns",
                            sn.c_str(), (long long)spr, (long long)i);
            hp->s_bytes = (size_t)count * 2;
            return cellm_file_tensor_bytes(f, sn.c_str(), &hp->s, nullptr) == CELLM_HIP_OK
                       ? CELLM_HIP_OK
                       : fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s unreadable", sn.c_str());
        }
        if (strcmp(t.dtype, "f16") == 0) {
            hp->kind = PK_F16;
            hp->w_bytes = (size_t)(o * i) * 2;
            return tensor(w, "f16", o, i, hp->w_bytes, &hp->w);
        }
        if (family == FAM_QWEN && strcmp(t.dtype, "i2") == 0) {
            // ceil(i/4) bytes per row, one f16 scale per row on the row sum (qwen.rs:1087-1096)
            hp->kind = PK_I2;
            hp->w_bytes = (size_t)(o * ((i + 3) / 4));
            hp->s_bytes = (size_t)o * 2;
            if (int32_t rc = tensor(w, "i2", o, i, hp->w_bytes, &hp->w)) return rc;
            return tensor(w + ".qscale", "f16", o, -1, hp->s_bytes, &hp->s);
        }
        if (family == FAM_QWEN && strcmp(t.dtype, "q1_0_g128") == 0) {
            // i / 128 blocks of 18 bytes per row (qwen.rs:1004-1022)
            if (i % 128 != 0)
                return fail(CELLM_HIP_ERR_INVALID_ARG, "%s: q1_0_g128 needs in %% 128 == 0", w.c_str());
            hp->kind = PK_Q1;
            hp->w_bytes = (size_t)(o * (i / 128) * 18);
            return tensor(w, "q1_0_g128", o, i, hp->w_bytes, &hp->w);
        }
        return fail(CELLM_HIP_ERR_UNSUPPORTED, "tensor %s is %s; the device step takes i8, u32 (MLX affine), i4%s",
                    w.c_str(), t.dtype, family == FAM_QWEN ? ", f16, i2 or q1_0_g128" : " or f16");
    };
    HostModel hm;
    hm.rope_interleaved = family == FAM_LLAMA && cellm_step::llama_rope_interleaved_from_env();
    hm.p.resize((size_t)c.n_layers * 7);
    for (int32_t l = 0; l < c.n_layers; ++l) {
        const std::string pre = base + "layers." + std::to_string(l) + ".";
        for (int j = 0; j < 7; ++j) {
            size_t o, i;
            out_in(c, j, &o, &i);
            HostProj& hp = hm.p[(size_t)l * 7 + j];
            if (int32_t rc = load_proj(pre + kNames[j] + ".weight", (int64_t)o, (int64_t)i, &hp, false)) return rc;
            // Qwen: "<stem>.bias" [out] f16 when present, added after the projection (qwen.rs:1132-1139,
            // 1361-1363, 1420, 1436-1437, 1457)
            const std::string bn = pre + kNames[j] + ".bias";
            if (family == FAM_QWEN && has(bn)) {
                const void* bp = nullptr;
                if (int32_t rc = tensor(bn, "f16", (int64_t)o, -1, (uint64_t)o * 2, &bp)) return rc;
                hp.bias_f16 = static_cast<const uint16_t*>(bp);
                hp.bias_n = o;
            }
        }
        const void *n1 = nullptr, *n2 = nullptr;
        if (int32_t rc = tensor(pre + "input_layernorm.weight", "f16", c.hidden, -1, (uint64_t)c.hidden * 2, &n1))
            return rc;
        if (int32_t rc =
                tensor(pre + "post_attention_layernorm.weight", "f16", c.hidden, -1, (uint64_t)c.hidden * 2, &n2))
            return rc;
        hm.n1.push_back(static_cast<const uint16_t*>(n1));
        hm.n2.push_back(static_cast<const uint16_t*>(n2));
    }
    // the embedding as embed_token takes it: i8 or i4 with a per-row f16 .qscale, or f16 (llama.rs:676-726,
    // qwen.rs:850-918 without its q1_0_g128 and i2 rows)
    {
        const std::string e = base + "embed_tokens.weight";
        cellm_file_tensor_t t;
        if (cellm_file_find(f, e.c_str(), &t) != CELLM_HIP_OK)
            return fail(CELLM_HIP_ERR_NOT_FOUND, "tensor %s missing", e.c_str());
        if (strcmp(t.dtype, "f16") == 0) {
            hm.embed.kind = PK_F16;
            hm.embed.w_bytes = (size_t)c.vocab * c.hidden * 2;
            if (int32_t rc = tensor(e, "f16", c.vocab, c.hidden, hm.embed.w_bytes, &hm.embed.w)) return rc;
        } else if (strcmp(t.dtype, "i8") == 0 || strcmp(t.dtype, "i4") == 0) {
            if (int32_t rc = load_proj(e, c.vocab, c.hidden, &hm.embed, true)) return rc;
        } else {
            return fail(CELLM_HIP_ERR_UNSUPPORTED, "unsupported embed dtype for model.embed_tokens.weight: %s",
                        t.dtype);
        }
    }
    const void* fn = nullptr;
    if (int32_t rc = tensor(base + "norm.weight", "f16", c.hidden, -1, (uint64_t)c.hidden * 2, &fn)) return rc;
    // lm_head.weight when the file has one, else the tied embedding (llama.rs:522-532; Qwen resolves the name
    // through its prefixes, qwen.rs:577 and :1560-1570)
    const std::string llama_prefix = family == FAM_LLAMA ? base.substr(0, base.size() - 6) : std::string();
    const std::vector<std::string> lm_names =
        family == FAM_LLAMA ? std::vector<std::string>{llama_prefix + "lm_head.weight", "lm_head.weight"}
                            : std::vector<std::string>{"lm_head.weight", "model.lm_head.weight",
                                                       "language_model.model.lm_head.weight",
                                                       "model.language_model.lm_head.weight"};
    for (const std::string& name : lm_names) {
        if (!has(name)) continue;
        if (int32_t rc = load_proj(name, c.vocab, c.hidden, &hm.lm, true)) return rc;
        break;
    }
    hm.final_norm = static_cast<const uint16_t*>(fn);
    return dev_create_impl(&c, hm, device, max_rows, max_blocks, out);
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_dev_set_graphs(cellm_llama_dev_t* m, int32_t enable)
{
    CELLM_API_BEGIN
    if (!m) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    for (int32_t r = 0; enable && r < m->max_rows; ++r)
        if (!m->graph_exec[r]) return fail(CELLM_HIP_ERR_UNSUPPORTED, "no captured graph for %d rows", r + 1);
    m->use_graphs = enable != 0;
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_dev_kv_upload(cellm_llama_dev_t* m, const uint16_t* k_f16, const uint16_t* v_f16, size_t n_elems)
{
    CELLM_API_BEGIN
    if (!m || !k_f16 || !v_f16) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (n_elems != m->kv_elems) return fail(CELLM_HIP_ERR_INVALID_ARG, "K/V have %zu elements, not %zu", n_elems,
                                            m->kv_elems);
    RT_TRY(hipSetDevice(m->device), "hipSetDevice");
    RT_TRY(hipMemcpy(m->kcache.p, k_f16, n_elems * 2, hipMemcpyHostToDevice), "upload K");
    RT_TRY(hipMemcpy(m->vcache.p, v_f16, n_elems * 2, hipMemcpyHostToDevice), "upload V");
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_dev_kv_download(cellm_llama_dev_t* m, uint16_t* k_f16, uint16_t* v_f16, size_t n_elems)
{
    CELLM_API_BEGIN
    if (!m || !k_f16 || !v_f16) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (n_elems != m->kv_elems) return fail(CELLM_HIP_ERR_INVALID_ARG, "K/V have %zu elements, not %zu", n_elems,
                                            m->kv_elems);
    RT_TRY(hipSetDevice(m->device), "hipSetDevice");
    LIB_TRY(cellm_hip_synchronize(m->hip), "synchronize");
    RT_TRY(hipMemcpy(k_f16, m->kcache.p, n_elems * 2, hipMemcpyDeviceToHost), "download K");
    RT_TRY(hipMemcpy(v_f16, m->vcache.p, n_elems * 2, hipMemcpyDeviceToHost), "download V");
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_dev_step(cellm_llama_dev_t* m, int32_t rows, const uint32_t* tokens, const int32_t* positions,
                             const uint32_t* block_tables, uint32_t* out_tokens, float* out_logits, float* logits_out)
{
    CELLM_API_BEGIN
    if (!m || !tokens || !positions || !block_tables || !out_tokens)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    const cellm_llama_config_t& c = m->cfg;
    if (rows < 1 || rows > m->max_rows) return fail(CELLM_HIP_ERR_INVALID_ARG, "rows must be 1..%d", m->max_rows);
    const int64_t tpb = c.tokens_per_block, MB = m->max_blocks;
    for (int32_t r = 0; r < rows; ++r) {
        const int32_t p = positions[r];
        if (p < 0 || p >= m->table_positions)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "row %d: position %d outside 0..%d", r, p, m->table_positions - 1);
        for (int64_t b = 0; b <= p / tpb; ++b)
            if (block_tables[r * MB + b] >= (uint32_t)c.total_blocks)
                return fail(CELLM_HIP_ERR_INVALID_ARG, "row %d: block %u out of range", r, block_tables[r * MB + b]);
    }
    RT_TRY(hipSetDevice(m->device), "hipSetDevice");
    const hipStream_t st = reinterpret_cast<hipStream_t>(m->stream);
    // inputs: one pinned staging copy
    unsigned char* hio = reinterpret_cast<unsigned char*>(m->host_io);
    memcpy(hio + m->io_tokens, tokens, (size_t)rows * 4);
    memcpy(hio + m->io_pos, positions, (size_t)rows * 4);
    memcpy(hio + m->io_bt, block_tables, (size_t)rows * MB * 4);
    memset(hio + m->io_keys, 0, m->io_bytes - m->io_keys);  // the argmax merges into zero keys
    RT_TRY(hipMemcpyAsync(m->io.p, m->host_io, m->io_bytes, hipMemcpyHostToDevice, st), "upload step inputs");
    if (m->use_graphs) {
        RT_TRY(hipGraphLaunch(m->graph_exec[rows - 1], st), "hipGraphLaunch(step)");
    } else if (int32_t rc = enqueue_step(m, rows)) {
        return rc;
    }
    unsigned char* dio = m->io.as<unsigned char>();
    const float* lg = m->logits.as<float>();
    RT_TRY(hipMemcpyAsync(hio + m->io_keys, dio + m->io_keys, m->io_bytes - m->io_keys, hipMemcpyDeviceToHost, st),
           "download ids");
    if (logits_out)
        RT_TRY(hipMemcpyAsync(logits_out, lg, (size_t)rows * c.vocab * 4, hipMemcpyDeviceToHost, st), "download logits");
    RT_TRY(hipStreamSynchronize(st), "step");
    for (int32_t r = 0; r < rows; ++r) {
        uint64_t key;
        memcpy(&key, hio + m->io_keys + (size_t)r * 8, 8);
        out_tokens[r] = (uint32_t)cellm_hip_argmax_key_index(key);
        if (out_logits) out_logits[r] = cellm_hip_argmax_key_value(key);
    }
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

}  // extern "C"
