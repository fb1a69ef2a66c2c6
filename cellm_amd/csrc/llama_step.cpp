// Host-side Llama decode step over libcellm_hip.so (declared in
// include/cellm_llama_step.h): a C++ mirror of LlamaRunner::step_inner
// (crates/cellm-model/src/llama.rs:235-647) with every projection issued to
// the HIP qGEMV through the sync MetalOps-style entry point
// cellm_hip_logits_i8, exactly as the reference runner routes "i8" weights to
// MetalOps::logits_i8 (llama.rs:781-811).  Embedding, RMSNorm, RoPE, the paged
// f16 KV cache and attention are CPU code restated from the reference; this
// file is compiled with -ffp-contract=off so every f32 operation rounds as
// Rust's does.
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/cellm_hip.h"
#include "../../include/cellm_llama_step.h"
#include "api_guard.hpp"

namespace cellm_step {
thread_local cellm::ErrorSlot g_err = {};  // shared with llama_device.cpp

// LlamaRunner's RoPE layout switch (llama.rs:80-82): CELLM_LLAMA_ROPE_INTERLEAVED set to "1" or
// "true" in any case selects rope_interleaved_inplace_f32 for q and k (llama.rs:391-396); unset or
// anything else keeps rotate-half.  Read once when a runner is created, as the reference does.
bool llama_rope_interleaved_from_env()
{
    const char* v = std::getenv("CELLM_LLAMA_ROPE_INTERLEAVED");
    if (!v) return false;
    if (std::strcmp(v, "1") == 0) return true;
    const char* t = "true";
    for (size_t i = 0;; ++i) {
        const char a = (char)std::tolower((unsigned char)v[i]);
        if (a != t[i]) return false;
        if (a == '\0') return true;
    }
}

// The CELLM_API_END report of this library (no allocation).
int32_t report_exception(int32_t code, const char* what)
{
    char buf[sizeof(g_err.msg)];
    const int n = snprintf(buf, sizeof(buf), "internal error: %s", what ? what : "");
    g_err.store(buf, n < 0 ? 0 : ((size_t)n < sizeof(buf) ? (size_t)n : sizeof(buf) - 1));
    return code;
}
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

int32_t from_hip(int32_t rc, const char* what)
{
    char buf[512];
    cellm_hip_last_error_message(buf, sizeof(buf));
    return fail(rc, "%s: %s", what, buf);
}

// f16::from_bits(h).to_f32() (exact) and f16::from_f32 (RNE).
float h2f(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {
            float v = (float)m * 5.9604644775390625e-08f;
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

uint16_t f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    const int32_t e = (int32_t)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t mm = man | 0x800000u, sh = (uint32_t)(14 - e);
        const uint32_t half = 1u << (sh - 1), rest = mm & ((1u << sh) - 1u);
        uint32_t r = mm >> sh;
        if (rest > half || (rest == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

// rms_norm_f32 (crates/cellm-kernels/src/cpu_kernels.rs:17-34)
void rms_norm(const float* x, const float* w, size_t n, float eps, float* out)
{
    float mean_sq = 0.0f;
    for (size_t i = 0; i < n; ++i) mean_sq += x[i] * x[i];
    mean_sq /= (float)n;
    const float inv_rms = 1.0f / std::sqrt(mean_sq + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv_rms * w[i];
}

// rope_non_interleaved_inplace_f32 with rotary_dim = head_dim (cpu_kernels.rs:264-277),
// the default layout (llama.rs:394-396), or with `interleaved`
// rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292, llama.rs:391-393): the same
// angle for pair i, applied to elements (2i, 2i + 1) instead of (i, i + half)
void rope(float* x, size_t n_heads, size_t head_dim, size_t pos, float theta, bool interleaved)
{
    const size_t half = head_dim / 2;
    for (size_t h = 0; h < n_heads; ++h) {
        float* head = x + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            const float inv_freq = std::pow(theta, -(2.0f * (float)i) / (float)head_dim);
            const float angle = (float)pos * inv_freq;
            const float s = std::sin(angle), c = std::cos(angle);
            const size_t i0 = interleaved ? 2 * i : i, i1 = interleaved ? 2 * i + 1 : half + i;
            const float x0 = head[i0], x1 = head[i1];
            head[i0] = x0 * c - x1 * s;
            head[i1] = x1 * c + x0 * s;
        }
    }
}

}  // namespace

struct cellm_llama {
    cellm_llama_config_t cfg{};
    bool rope_interleaved = false;  // CELLM_LLAMA_ROPE_INTERLEAVED at creation
    cellm_hip_ctx_t* hip = nullptr;
    std::vector<std::vector<int8_t>> w;       // kept host-side: logits_i8 takes host slices
    std::vector<std::vector<uint16_t>> s;
    std::vector<std::vector<float>> attn_norm, mlp_norm;
    std::vector<int8_t> embed;
    std::vector<uint16_t> embed_scale;
    std::vector<float> final_norm;
    std::vector<uint16_t> kcache, vcache;
    size_t kv_dim = 0;
};

namespace {

const char* kNames[7] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};

void out_in(const cellm_llama_config_t& c, int j, size_t* out, size_t* in)
{
    const size_t hid = (size_t)c.hidden, kv = (size_t)c.n_kv_heads * c.head_dim, inter = (size_t)c.intermediate;
    const size_t o[7] = {hid, kv, kv, hid, inter, inter, hid};
    const size_t i[7] = {hid, hid, hid, hid, hid, hid, inter};
    *out = o[j];
    *in = i[j];
}

// One projection through MetalOps::logits_i8's HIP sibling; key = tensor name.
int32_t linear(cellm_llama* m, int layer, int j, const float* x, float* y)
{
    size_t o, i;
    out_in(m->cfg, j, &o, &i);
    char key[96];
    snprintf(key, sizeof(key), "model.layers.%d.%s.weight", layer, kNames[j]);
    const size_t idx = (size_t)layer * 7 + j;
    const int32_t rc = cellm_hip_logits_i8(m->hip, x, m->w[idx].data(), m->s[idx].data(), o, i, key, y);
    return rc ? from_hip(rc, key) : 0;
}

}  // namespace

extern "C" {

size_t cellm_llama_last_error_message(char* buf, size_t buf_len) { return g_err.take(buf, buf_len); }

int32_t cellm_llama_create(const cellm_llama_config_t* cfg, const cellm_llama_layer_t* layers,
                           const int8_t* embed_i8, const uint16_t* embed_scale_f16, const uint16_t* final_norm_f16,
                           int32_t device, cellm_llama_t** out)
{
    CELLM_API_BEGIN
    if (!cfg || !layers || !embed_i8 || !embed_scale_f16 || !final_norm_f16 || !out)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    const cellm_llama_config_t& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate <= 0 || c.vocab <= 0 || c.tokens_per_block <= 0 || c.total_blocks <= 0)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "non-positive dimension in config");
    if (c.head_dim * c.n_heads != c.hidden)  // llama.rs:285-289
        return fail(CELLM_HIP_ERR_INVALID_ARG, "hidden_size must equal num_heads * head_dim");
    if (c.n_heads % c.n_kv_heads != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "n_heads % n_kv_heads != 0");
    auto* m = new cellm_llama();
    m->cfg = c;
    m->rope_interleaved = cellm_step::llama_rope_interleaved_from_env();
    m->kv_dim = (size_t)c.n_kv_heads * c.head_dim;
    int32_t rc = cellm_hip_create(device, &m->hip);
    if (rc) {
        delete m;
        return from_hip(rc, "cellm_hip_create");
    }
    const size_t hid = (size_t)c.hidden;
    m->w.resize((size_t)c.n_layers * 7);
    m->s.resize((size_t)c.n_layers * 7);
    for (int l = 0; l < c.n_layers; ++l) {
        for (int j = 0; j < 7; ++j) {
            size_t o, i;
            out_in(c, j, &o, &i);
            if (!layers[l].w[j] || !layers[l].scale_f16[j]) {
                cellm_llama_destroy(m);
                return fail(CELLM_HIP_ERR_INVALID_ARG, "layer %d tensor %s missing", l, kNames[j]);
            }
            m->w[(size_t)l * 7 + j].assign(layers[l].w[j], layers[l].w[j] + o * i);
            m->s[(size_t)l * 7 + j].assign(layers[l].scale_f16[j], layers[l].scale_f16[j] + o);
        }
        std::vector<float> a(hid), b(hid);
        for (size_t i = 0; i < hid; ++i) {  // rmsnorm_weight: f16 -> f32 (llama.rs:728-741)
            a[i] = h2f(layers[l].input_layernorm_f16[i]);
            b[i] = h2f(layers[l].post_attention_layernorm_f16[i]);
        }
        m->attn_norm.push_back(std::move(a));
        m->mlp_norm.push_back(std::move(b));
    }
    m->embed.assign(embed_i8, embed_i8 + (size_t)c.vocab * hid);
    m->embed_scale.assign(embed_scale_f16, embed_scale_f16 + c.vocab);
    m->final_norm.resize(hid);
    for (size_t i = 0; i < hid; ++i) m->final_norm[i] = h2f(final_norm_f16[i]);
    const size_t kv_elems = (size_t)c.total_blocks * c.n_layers * c.tokens_per_block * m->kv_dim;
    m->kcache.assign(kv_elems, 0);
    m->vcache.assign(kv_elems, 0);
    // upload every projection once (the weight cache is keyed by tensor name)
    std::vector<float> zx((size_t)std::max(c.hidden, c.intermediate), 0.0f), zy(std::max<size_t>(c.vocab, c.intermediate));
    for (int l = 0; l < c.n_layers; ++l)
        for (int j = 0; j < 7; ++j)
            if ((rc = linear(m, l, j, zx.data(), zy.data()))) {
                cellm_llama_destroy(m);
                return rc;
            }
    rc = cellm_hip_logits_i8(m->hip, zx.data(), m->embed.data(), m->embed_scale.data(), (size_t)c.vocab, hid,
                             "model.embed_tokens.weight", zy.data());
    if (rc) {
        cellm_llama_destroy(m);
        return from_hip(rc, "lm_head upload");
    }
    *out = m;
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

void cellm_llama_destroy(cellm_llama_t* m)
{
    CELLM_API_BEGIN
    if (!m) return;
    if (m->hip) cellm_hip_destroy(m->hip);
    delete m;
    CELLM_API_END_VOID
}

int32_t cellm_llama_kv_cache(cellm_llama_t* m, uint16_t** k_f16, uint16_t** v_f16, size_t* n_elems)
{
    CELLM_API_BEGIN
    if (!m || !k_f16 || !v_f16 || !n_elems) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *k_f16 = m->kcache.data();
    *v_f16 = m->vcache.data();
    *n_elems = m->kcache.size();
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

int32_t cellm_llama_step(cellm_llama_t* m, uint32_t token, size_t pos, const uint32_t* block_table,
                         size_t n_blocks, uint32_t* out_token, float* out_logit, float* logits_out)
{
    CELLM_API_BEGIN
    if (!m || !block_table || !out_token) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    const cellm_llama_config_t& c = m->cfg;
    const size_t hid = (size_t)c.hidden, kvd = m->kv_dim, tpb = (size_t)c.tokens_per_block;
    const size_t nh = (size_t)c.n_heads, nkv = (size_t)c.n_kv_heads, hd = (size_t)c.head_dim;
    const size_t inter = (size_t)c.intermediate, vocab = (size_t)c.vocab, L = (size_t)c.n_layers;
    if (pos / tpb >= n_blocks) return fail(CELLM_HIP_ERR_INVALID_ARG, "pos %zu beyond the block table", pos);
    for (size_t b = 0; b <= pos / tpb; ++b)
        if (block_table[b] >= (uint32_t)c.total_blocks)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "block %u out of range", block_table[b]);
    // KvCacheLayout::token_base_elem (crates/cellm-core/src/kv_cache.rs:62-73)
    auto base_of = [&](size_t tpos, size_t layer) {
        const size_t blk = block_table[tpos / tpb], off = tpos % tpb;
        return blk * (L * tpb * kvd) + layer * (tpb * kvd) + off * kvd;
    };

    // embed_token, i8 branch (llama.rs:676-701): row * f16 scale, token % vocab
    std::vector<float> x(hid), xn(hid), q(hid), k(kvd), v(kvd), attn(hid), proj(hid);
    std::vector<float> gate(inter), up(inter), down(hid), scores(pos + 1);
    const size_t t = token % vocab;
    const float es = h2f(m->embed_scale[t]);
    for (size_t i = 0; i < hid; ++i) x[i] = (float)m->embed[t * hid + i] * es;

    int32_t rc;
    for (size_t l = 0; l < L; ++l) {
        rms_norm(x.data(), m->attn_norm[l].data(), hid, c.rms_norm_eps, xn.data());
        if ((rc = linear(m, (int)l, 0, xn.data(), q.data())) || (rc = linear(m, (int)l, 1, xn.data(), k.data())) ||
            (rc = linear(m, (int)l, 2, xn.data(), v.data())))
            return rc;
        rope(q.data(), nh, hd, pos, c.rope_theta, m->rope_interleaved);
        rope(k.data(), nkv, hd, pos, c.rope_theta, m->rope_interleaved);
        // write_token_f32: f32 -> f16 RNE (crates/cellm-cache/src/kvcache.rs:589-615)
        const size_t wb = base_of(pos, l);
        for (size_t i = 0; i < kvd; ++i) {
            m->kcache[wb + i] = f2h(k[i]);
            m->vcache[wb + i] = f2h(v[i]);
        }
        // CpuKvStorage::attention_single_token_gqa_f32 (kvcache.rs:710-789)
        std::fill(attn.begin(), attn.end(), 0.0f);
        const size_t seq = pos + 1;
        const float scale = 1.0f / std::sqrt((float)hd);
        const size_t group = std::max<size_t>(nh / nkv, 1);
        for (size_t h = 0; h < nh; ++h) {
            const size_t kvh = std::min(h / group, nkv - 1);
            const float* qh = q.data() + h * hd;
            for (size_t tp = 0; tp < seq; ++tp) {
                const uint16_t* kt = m->kcache.data() + base_of(tp, l) + kvh * hd;
                float dot = 0.0f;
                for (size_t i = 0; i < hd; ++i) dot += qh[i] * h2f(kt[i]);
                scores[tp] = dot * scale;
            }
            // softmax_f32_inplace_cpu_local (kvcache.rs:1206-1227)
            float mx = -INFINITY;
            for (size_t tp = 0; tp < seq; ++tp)
                if (scores[tp] > mx) mx = scores[tp];
            float sum = 0.0f;
            for (size_t tp = 0; tp < seq; ++tp) {
                scores[tp] = std::exp(scores[tp] - mx);
                sum += scores[tp];
            }
            if (sum > 0.0f) {
                const float inv = 1.0f / sum;
                for (size_t tp = 0; tp < seq; ++tp) scores[tp] *= inv;
            }
            float* oh = attn.data() + h * hd;
            for (size_t tp = 0; tp < seq; ++tp) {
                const uint16_t* vt = m->vcache.data() + base_of(tp, l) + kvh * hd;
                const float wgt = scores[tp];
                for (size_t i = 0; i < hd; ++i) oh[i] += wgt * h2f(vt[i]);
            }
        }
        if ((rc = linear(m, (int)l, 3, attn.data(), proj.data()))) return rc;
        for (size_t i = 0; i < hid; ++i) x[i] += proj[i];
        rms_norm(x.data(), m->mlp_norm[l].data(), hid, c.rms_norm_eps, xn.data());
        if ((rc = linear(m, (int)l, 4, xn.data(), gate.data())) || (rc = linear(m, (int)l, 5, xn.data(), up.data())))
            return rc;
        for (size_t i = 0; i < inter; ++i) {  // SiLU(gate) * up (llama.rs:477-484)
            const float g = gate[i];
            const float sg = 1.0f / (1.0f + std::exp(-g));
            gate[i] = g * sg;
        }
        for (size_t i = 0; i < inter; ++i) gate[i] *= up[i];
        if ((rc = linear(m, (int)l, 6, gate.data(), down.data()))) return rc;
        for (size_t i = 0; i < hid; ++i) x[i] += down[i];
    }
    rms_norm(x.data(), m->final_norm.data(), hid, c.rms_norm_eps, xn.data());
    // tied lm_head through logits_i8 (llama.rs:549-567), then sanitize (llama.rs:1081-1092)
    std::vector<float> logits(vocab);
    rc = cellm_hip_logits_i8(m->hip, xn.data(), m->embed.data(), m->embed_scale.data(), vocab, hid,
                             "model.embed_tokens.weight", logits.data());
    if (rc) return from_hip(rc, "lm_head");
    for (auto& z : logits)
        if (!std::isfinite(z)) z = -INFINITY;
    // topk_from_logits with k = 1 (llama.rs:1049-1078): the first maximum
    size_t best = 0;
    for (size_t i = 1; i < vocab; ++i)
        if (logits[i] > logits[best]) best = i;
    *out_token = (uint32_t)best;
    if (out_logit) *out_logit = logits[best];
    if (logits_out) memcpy(logits_out, logits.data(), vocab * sizeof(float));
    return CELLM_HIP_OK;
    CELLM_API_END(cellm_step::report_exception)
}

}  // extern "C"
