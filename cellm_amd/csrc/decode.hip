// Decode-step kernels around the projections (gfx950): the device side of a
// Llama decode step, as the reference's fused Metal graph encodes it
// (crates/cellm-model/src/llama_graph.rs:140-405).  Every kernel takes `rows`
// independent sessions (one activation row each) so that a step for several
// sessions reads every projection weight once.
//
//   embed_i8       x = f32(E[tok % vocab]) * f32(scale)        llama.rs:676-701
//   rms_norm       out = x * (1/sqrt(mean(x^2)+eps)) * w        cpu_kernels.rs:17-34
//   add_rms_norm   x += y (residual, llama.rs:440,494), then rms_norm
//   rope_half      rotate-half RoPE from a cos/sin table        cpu_kernels.rs:264-277
//   kv_write_f16   f32 -> f16 (RNE) into the paged cache        kvcache.rs:589-615
//   rope_kv_write  rope_half on q and k, then kv_write_f16, in one launch
//   attention      single-token GQA over f16 K/V pages, with the
//                  optional attn_scale and soft cap              kvcache.rs:710-789
//   argmax         first maximum, non-finite -> -inf            llama.rs:1049-1092
//
// Where the reference rounds a product and a sum separately, so do these
// kernels: FP contraction is off for this file (hipcc contracts a*b+c into
// an FMA by default; HIP's __fmul_rn is an inline a*b from a header outside
// this pragma, so it would still be fused: plain operators are used here).
// Sums over a vector are tree-shaped here and sequential there; softmax uses
// the device expf.
// Paged addressing is KvCacheLayout::token_base_elem
// (crates/cellm-core/src/kv_cache.rs:62-73):
//   base(t, layer) = block[t / tpb] * (L * tpb * kvd) + layer * (tpb * kvd) + (t % tpb) * kvd
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace cellm {

namespace {

constexpr int kNormThreads = 256;
constexpr int kAttnChunk = 64;        // positions per partial-attention block
constexpr int kAttnThreads = 256;
constexpr int kAttnGMax = 8;          // query heads per kv head
constexpr int kAttnMaxChunks = 512;   // positions per sequence <= 32768
// One-launch attention: a counter per (row, kv head) group at the start of the
// workspace, zero between calls (the group's last block resets it).
constexpr int kAttnCounters = 16384;
constexpr size_t kAttnCounterBytes = (size_t)kAttnCounters * sizeof(uint32_t);

// Agent-coherent (sc1) store and load: the one-launch attention hands a group's
// partials to its last block through these, with a wait for the stores before
// the arrival count, instead of an agent-scope fence (an L2 write-back per
// block on this part).
template <bool COH>
__device__ __forceinline__ void st_part(float* p, float v)
{
    if constexpr (COH)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}
template <bool COH>
__device__ __forceinline__ float ld_part(const float* p)
{
    if constexpr (COH)
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *p;
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

__global__ void embed_i8_kernel(const uint32_t* __restrict__ tokens, const int8_t* __restrict__ emb,
                                const uint16_t* __restrict__ scale, int vocab, int hidden, float* __restrict__ x)
{
    const int r = blockIdx.y;
    const size_t t = tokens[r] % (uint32_t)vocab;
    const float s = h2f(scale[t]);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        x[(size_t)r * hidden + i] = (float)emb[t * hidden + i] * s;
}

// embed_token's f16 and i4 branches (llama.rs:687-693, 703-718): one row per token.
__global__ void embed_f16_kernel(const uint32_t* __restrict__ tokens, const uint16_t* __restrict__ emb, int vocab,
                                 int hidden, float* __restrict__ x)
{
    const int r = blockIdx.y;
    const size_t t = tokens[r] % (uint32_t)vocab;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        x[(size_t)r * hidden + i] = h2f(emb[t * hidden + i]);
}

// (nibble - 8) * scale, low nibble = even element, ceil(hidden / 2) bytes per row
__global__ void embed_i4_kernel(const uint32_t* __restrict__ tokens, const uint8_t* __restrict__ emb,
                                const uint16_t* __restrict__ scale, int vocab, int hidden, float* __restrict__ x)
{
    const int r = blockIdx.y;
    const size_t t = tokens[r] % (uint32_t)vocab;
    const float s = h2f(scale[t]);
    const uint8_t* row = emb + t * (size_t)((hidden + 1) / 2);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
        const uint32_t b = row[i >> 1];
        const int q = (int)((i & 1) ? (b >> 4) : (b & 0xFu)) - 8;
        x[(size_t)r * hidden + i] = (float)q * s;
    }
}

template <int WDT>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float* __restrict__ x, const void* __restrict__ w,
                                                               float* __restrict__ out, int n, float eps)
{
    __shared__ float part[kNormThreads / 64];
    const int r = blockIdx.x;
    const float* xr = x + (size_t)r * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kNormThreads) s = s + xr[i] * xr[i];
    s = group_sum<64>(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot = tot + part[i];
    const float mean = tot / (float)n;
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int i = threadIdx.x; i < n; i += kNormThreads)
        out[(size_t)r * n + i] = xr[i] * inv * load_f32<WDT>(w, i);
}

// x += y, then out = rms_norm(x) * w: the residual add of the previous
// sub-layer and the next RMSNorm in one pass; per element the same
// arithmetic, and the same reduction tree, as add_f32 followed by rms_norm.
template <int WDT>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                                   const void* __restrict__ w, float* __restrict__ out,
                                                                   int n, float eps)
{
    constexpr int kRegs = 8;  // rows up to kRegs * kNormThreads stay in registers: one memory latency
    __shared__ float part[kNormThreads / 64];
    const int r = blockIdx.x, t = threadIdx.x;
    float* xr = x + (size_t)r * n;
    const float* yr = y + (size_t)r * n;
    float* orow = out + (size_t)r * n;
    float s = 0.0f;
    const bool in_regs = n <= kRegs * kNormThreads;
    float xv[kRegs], wv[kRegs];
    if (in_regs) {
        float yv[kRegs];
#pragma unroll
        for (int u = 0; u < kRegs; ++u) {
            const int i = min(t + u * kNormThreads, n - 1);
            xv[u] = xr[i];
            yv[u] = yr[i];
            wv[u] = load_f32<WDT>(w, i);
        }
#pragma unroll
        for (int u = 0; u < kRegs; ++u) {
            const int i = t + u * kNormThreads;
            if (i < n) {
                const float v = xv[u] + yv[u];
                xv[u] = v;
                xr[i] = v;
                s = s + v * v;
            }
        }
    } else {
        for (int i = t; i < n; i += kNormThreads) {
            const float v = xr[i] + yr[i];
            xr[i] = v;
            s = s + v * v;
        }
    }
    s = group_sum<64>(s);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot = tot + part[i];
    const float mean = tot / (float)n;
    const float inv = 1.0f / sqrtf(mean + eps);
    if (in_regs) {
#pragma unroll
        for (int u = 0; u < kRegs; ++u) {
            const int i = t + u * kNormThreads;
            if (i < n) orow[i] = xv[u] * inv * wv[u];
        }
    } else {
        for (int i = t; i < n; i += kNormThreads) orow[i] = xr[i] * inv * load_f32<WDT>(w, i);
    }
}

// One thread per (row, head, i < half).  cs[p][i] = (cos, sin) of position p.
// The two elements pair i of a head rotates: i and i + half (rotate-half,
// rope_non_interleaved_inplace_f32, cpu_kernels.rs:264-277) or 2i and 2i + 1
// (rope_interleaved_inplace_f32, cpu_kernels.rs:279-292).  Both use the angle
// pos * theta^(-2i / head_dim) of pair i.
__device__ __forceinline__ int rope_lo(int i, int half, int il) { return il ? 2 * i : i; }
__device__ __forceinline__ int rope_hi(int i, int half, int il) { return il ? 2 * i + 1 : half + i; }

__global__ void rope_half_kernel(float* __restrict__ x, int rows, int n_heads, int head_dim,
                                 const int32_t* __restrict__ pos, const float2* __restrict__ cs, int table_positions,
                                 int il)
{
    const int half = head_dim >> 1;
    const int total = rows * n_heads * half;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int i = idx % half, rh = idx / half;
        const int r = rh / n_heads;
        const int p = min(max(pos[r], 0), table_positions - 1);
        const float2 c = cs[(size_t)p * half + i];
        float* head = x + (size_t)rh * head_dim;
        const int i0 = rope_lo(i, half, il), i1 = rope_hi(i, half, il);
        const float x0 = head[i0], x1 = head[i1];
        head[i0] = x0 * c.x - x1 * c.y;
        head[i1] = x1 * c.x + x0 * c.y;
    }
}

struct PagedKv {
    const uint32_t* bt;  // [rows][max_blocks]
    int max_blocks, total_blocks, n_layers, tpb, kvd;

    // element base of (row, token t) in `layer`, or -1 when the page is out of range
    __device__ __forceinline__ long long base(int r, int t, int layer) const
    {
        const int b = t / tpb;
        if (b >= max_blocks) return -1;
        const uint32_t blk = bt[(size_t)r * max_blocks + b];
        if (blk >= (uint32_t)total_blocks) return -1;
        return ((long long)blk * n_layers + layer) * (long long)tpb * kvd + (long long)(t % tpb) * kvd;
    }
};

__global__ void kv_write_kernel(const float* __restrict__ k, const float* __restrict__ v, int rows,
                                const int32_t* __restrict__ pos, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                PagedKv kv, int layer)
{
    const int total = rows * kv.kvd;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int r = idx / kv.kvd, j = idx - r * kv.kvd;
        const long long b = pos[r] >= 0 ? kv.base(r, pos[r], layer) : -1;
        if (b < 0) continue;
        kc[b + j] = __builtin_bit_cast(uint16_t, (_Float16)k[idx]);
        vc[b + j] = __builtin_bit_cast(uint16_t, (_Float16)v[idx]);
    }
}

// RoPE on q and k, then k and v into the paged cache as f16: the same
// arithmetic as rope_half on q and on k followed by kv_write_f16, in one
// launch.  Work item (row, j): j < n_heads * half rotates the q pair
// (i, i + half) of head j / half; the rest rotate the k pair of one kv head,
// write it back to k, and store that pair of k and of v in the cache.
__global__ void rope_kv_write_kernel(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
                                     int rows, int n_heads, int n_kv_heads, int head_dim,
                                     const int32_t* __restrict__ pos, const float2* __restrict__ cs,
                                     int table_positions, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                     PagedKv kv, int layer, int il)
{
    const int half = head_dim >> 1;
    const int nq = n_heads * half, per_row = nq + n_kv_heads * half;
    const int total = rows * per_row;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int r = idx / per_row, j = idx - r * per_row;
        const int p = min(max(pos[r], 0), table_positions - 1);
        if (j < nq) {
            const int i = j % half;
            const int i0 = rope_lo(i, half, il), i1 = rope_hi(i, half, il);
            const float2 c = cs[(size_t)p * half + i];
            float* head = q + ((size_t)r * n_heads + j / half) * head_dim;
            const float x0 = head[i0], x1 = head[i1];
            head[i0] = x0 * c.x - x1 * c.y;
            head[i1] = x1 * c.x + x0 * c.y;
        } else {
            const int jk = j - nq, kh = jk / half, i = jk % half;
            const int i0 = rope_lo(i, half, il), i1 = rope_hi(i, half, il);
            const float2 c = cs[(size_t)p * half + i];
            const size_t off = ((size_t)r * n_kv_heads + kh) * head_dim;
            const float x0 = k[off + i0], x1 = k[off + i1];
            const float k0 = x0 * c.x - x1 * c.y;
            const float k1 = x1 * c.x + x0 * c.y;
            k[off + i0] = k0;
            k[off + i1] = k1;
            const long long b = pos[r] >= 0 ? kv.base(r, pos[r], layer) : -1;
            if (b < 0) continue;
            const size_t e = (size_t)b + (size_t)kh * head_dim;
            kc[e + i0] = __builtin_bit_cast(uint16_t, (_Float16)k0);
            kc[e + i1] = __builtin_bit_cast(uint16_t, (_Float16)k1);
            vc[e + i0] = __builtin_bit_cast(uint16_t, (_Float16)v[off + i0]);
            vc[e + i1] = __builtin_bit_cast(uint16_t, (_Float16)v[off + i1]);
        }
    }
}

// Combine of one (row, kv head) group's nch chunk partials p (layout of
// attn_partial_kernel) into its G heads' outputs o[g][HD]:
//   o[g][i] = (sum_c acc_c[i] e^(m_c - M)) / (sum_c l_c e^(m_c - M)),  M = max_c m_c
// The chunk maxima and sums go to LDS, together with each thread's first
// kCombinePre partials of its first output (one memory latency for up to
// kCombinePre chunks); wave w then weighs the chunks of heads w and w + 4.
// Chunks are added in chunk order whichever block runs it.
template <int HD, int G, bool COH>
__device__ __forceinline__ void attn_combine_group(const float* __restrict__ p, int nch, float* __restrict__ o,
                                                   float (&cm)[G][kAttnMaxChunks], float (&cl)[G][kAttnMaxChunks],
                                                   float (&invl)[G])
{
    constexpr int kCombinePre = 16;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const size_t cstride = (size_t)G * (HD + 2);
    // this thread's first output and its first partials
    const int i0 = min(t, G * HD - 1);
    const float* pc0 = p + (size_t)(i0 / HD) * (HD + 2) + i0 % HD;
    float pre[kCombinePre];
#pragma unroll
    for (int c = 0; c < kCombinePre; ++c) pre[c] = ld_part<COH>(pc0 + (size_t)min(c, nch - 1) * cstride);
    for (int j = t; j < G * nch; j += kAttnThreads) {
        const int g = j % G, c = j / G;
        cm[g][c] = ld_part<COH>(p + c * cstride + (size_t)g * (HD + 2) + HD);
        cl[g][c] = ld_part<COH>(p + c * cstride + (size_t)g * (HD + 2) + HD + 1);
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {
        float m = -INFINITY;
        for (int c = lane; c < nch; c += 64) m = fmaxf(m, cm[g][c]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.0f;
        for (int c = lane; c < nch; c += 64) {
            const float w = expf(cm[g][c] - m);
            cm[g][c] = w;
            l = l + cl[g][c] * w;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l = l + __shfl_xor(l, off);
        if (lane == 0) invl[g] = l > 0.0f ? 1.0f / l : 0.0f;
    }
    __syncthreads();
    for (int i = t; i < G * HD; i += kAttnThreads) {
        const int g = i / HD, d = i % HD;
        const float* pc = p + (size_t)g * (HD + 2) + d;
        float acc = 0.0f;
        int c = 0;
        if (i == t) {
#pragma unroll
            for (; c < kCombinePre; ++c)
                if (c < nch) acc = acc + pre[c] * cm[g][c];
        }
#pragma unroll 8
        for (; c < nch; ++c) acc = acc + ld_part<COH>(pc + c * cstride) * cm[g][c];
        o[(size_t)g * HD + d] = acc * invl[g];
    }
}

// Partial attention over positions [64c, 64c+64) for one (row, kv head) and
// its G query heads; part layout [row][kvh][chunk][G][HD + 2]: HD weighted-V
// sums, the chunk max and the chunk sum of exp(score - max).  Every K and V
// load of the chunk is issued before any arithmetic (one memory latency):
//   Q.K: thread t -> position t / 4, dims (t % 4) * HD/4 .. + HD/4 (16-B loads)
//   P.V: thread t -> dims (t % 64) * HD/64 .. + HD/64, positions 16 (t / 64) .. + 16
// so wave w owns positions 16w .. 16w + 15 in both phases.
//
// FUSED: one launch.  The partials go out with agent-coherent stores; after
// waiting for them the block counts its arrival in its group's counter, and the
// group's last block to arrive (whichever chunk) combines the group with
// agent-coherent loads into `out` and resets the counter to zero.
// First position a row attends to: with a sliding window of `window`
// positions (window > 0) the last `window` of its `seq`, else all of them
// (gemma.rs:747-751: start = seq.saturating_sub(sliding_window) on sliding
// layers, 0 on full-attention layers).
__device__ __forceinline__ int window_start(int seq, int window) { return window > 0 ? max(seq - window, 0) : 0; }

template <int HD, int G, bool FUSED = false>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, PagedKv kv, int layer, int n_kv_heads, float scale, float soft_cap, int window,
    float* __restrict__ part, int nch_max, uint32_t* __restrict__ counters = nullptr, float* __restrict__ out = nullptr)
{
    constexpr int KD = HD / 4;                             // Q.K dims per thread
    constexpr int KL = KD / 8;                             // 16-byte K loads per thread
    constexpr int VD = HD / 64;                            // P.V dims per thread (1 or 2)
    constexpr int VP = kAttnChunk / 4;                     // P.V positions per thread
    constexpr int QL = (G * HD + kAttnThreads - 1) / kAttnThreads;  // q elements per thread
    using vword_t = typename std::conditional<VD == 1, uint16_t, uint32_t>::type;
    const int n_heads = G * n_kv_heads;
    __shared__ float qs[G * HD];
    __shared__ float ps[G][kAttnChunk];
    __shared__ long long bases[kAttnChunk];
    __shared__ float wmax[4][G], wsum[4][G];
    __shared__ float accs[4][G * HD];
    const int r = blockIdx.x / n_kv_heads, kvh = blockIdx.x % n_kv_heads, ch = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int t0 = ch * kAttnChunk;
    // position, q and this chunk's page entries: independent loads, issued together
    // (addresses clamped in range so that no load sits behind a branch)
    const int p_r = pos[r];
    const float* qr = q + ((size_t)r * n_heads + (size_t)kvh * G) * HD;
    float qv[QL];
#pragma unroll
    for (int j = 0; j < QL; ++j) qv[j] = qr[min(t + j * kAttnThreads, G * HD - 1)];
    const int tt = t0 + lane, blk_i = tt / kv.tpb;
    const uint32_t blk = kv.bt[(size_t)r * kv.max_blocks + min(blk_i, kv.max_blocks - 1)];
    const int seq = min(p_r + 1, kv.max_blocks * kv.tpb);
    const int s0 = window_start(seq, window), c0 = s0 / kAttnChunk;
    if (t0 >= seq || ch < c0) return;  // the same for the whole block
    const int nt = min(kAttnChunk, seq - t0);
#pragma unroll
    for (int j = 0; j < QL; ++j)
        if (t + j * kAttnThreads < G * HD) qs[t + j * kAttnThreads] = qv[j];
    if (t < kAttnChunk)
        bases[t] = (t < nt && tt >= s0 && blk_i < kv.max_blocks && blk < (uint32_t)kv.total_blocks)
                       ? ((long long)blk * kv.n_layers + layer) * (long long)kv.tpb * kv.kvd +
                             (long long)(tt % kv.tpb) * kv.kvd
                       : -1;
    __syncthreads();

    // every K and V load of the chunk (a missing page reads element 0 and is zeroed)
    const int kp = t >> 2, kq = t & 3;
    const long long kb = bases[kp];
    const u4_t* ksrc = reinterpret_cast<const u4_t*>(kc + (kb >= 0 ? kb + (long long)kvh * HD + kq * KD : 0));
    u4_t kraw[KL];
#pragma unroll
    for (int j = 0; j < KL; ++j) kraw[j] = ksrc[j];
    vword_t vraw[VP];
    bool vok[VP];
#pragma unroll
    for (int i = 0; i < VP; ++i) {
        const long long vb = bases[wave * VP + i];
        vok[i] = vb >= 0;
        vraw[i] = *reinterpret_cast<const vword_t*>(vc + (vb >= 0 ? vb + (long long)kvh * HD + lane * VD : 0));
    }
    if (kb < 0) {
#pragma unroll
        for (int j = 0; j < KL; ++j) kraw[j] = u4_t{0, 0, 0, 0};
    }

    // scores: a partial dot over this thread's dims, summed over the 4 threads of the position
    float dot[G];
#pragma unroll
    for (int g = 0; g < G; ++g) dot[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < KL; ++j) {
        const h8_t kh = __builtin_bit_cast(h8_t, kraw[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float kf = (float)kh[e];
            const int d = kq * KD + j * 8 + e;
#pragma unroll
            for (int g = 0; g < G; ++g) dot[g] = dot[g] + qs[g * HD + d] * kf;
        }
    }
    const bool valid = kp < nt && t0 + kp >= s0;
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float d = dot[g];
        d = d + lane_xor<1>(d, 64);
        d = d + lane_xor<2>(d, 64);
        float sg = d * scale;
        if (soft_cap > 0.0f) sg = tanhf(sg / soft_cap) * soft_cap;  // kvcache.rs:768-770
        sc[g] = valid ? sg : -INFINITY;
        float m = sc[g];
        m = fmaxf(m, lane_xor<4>(m, 64));
        m = fmaxf(m, lane_xor<8>(m, 64));
        m = fmaxf(m, lane_xor<16>(m, 64));
        m = fmaxf(m, lane_xor<32>(m, 64));
        if (lane == 0) wmax[wave][g] = m;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float m = fmaxf(fmaxf(wmax[0][g], wmax[1][g]), fmaxf(wmax[2][g], wmax[3][g]));
        const float e = valid ? expf(sc[g] - m) : 0.0f;
        if (kq == 0) ps[g][kp] = e;
        float l = e;
        l = l + lane_xor<4>(l, 64);
        l = l + lane_xor<8>(l, 64);
        l = l + lane_xor<16>(l, 64);
        l = l + lane_xor<32>(l, 64);
        if (lane == 0) wsum[wave][g] = l;
    }
    __syncthreads();

    // weighted V over this wave's 16 positions, then over the 4 waves
    float acc[G][VD];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int d = 0; d < VD; ++d) acc[g][d] = 0.0f;
#pragma unroll
    for (int i = 0; i < VP; ++i) {
        const vword_t w = vok[i] ? vraw[i] : vword_t(0);
        float vf[VD];
        if constexpr (VD == 1) {
            vf[0] = h2f(w);
        } else {
            vf[0] = h2f((uint16_t)(w & 0xffffu));
            vf[1] = h2f((uint16_t)(w >> 16));
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
                const float pg = ps[g][wave * VP + i];
#pragma unroll
            for (int d = 0; d < VD; ++d) acc[g][d] = acc[g][d] + pg * vf[d];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int d = 0; d < VD; ++d) accs[wave][g * HD + lane * VD + d] = acc[g][d];
    }
    __syncthreads();
    float* const grp = part + (((size_t)r * n_kv_heads + kvh) * nch_max) * G * (HD + 2);
    float* const pout = grp + (size_t)ch * G * (HD + 2);
    for (int i = t; i < G * HD; i += kAttnThreads)
        st_part<FUSED>(pout + (size_t)(i / HD) * (HD + 2) + i % HD,
                       (accs[0][i] + accs[1][i]) + (accs[2][i] + accs[3][i]));
    if (t < G) {
        st_part<FUSED>(pout + (size_t)t * (HD + 2) + HD,
                       fmaxf(fmaxf(wmax[0][t], wmax[1][t]), fmaxf(wmax[2][t], wmax[3][t])));
        st_part<FUSED>(pout + (size_t)t * (HD + 2) + HD + 1, (wsum[0][t] + wsum[1][t]) + (wsum[2][t] + wsum[3][t]));
    }
    if constexpr (FUSED) {
        __shared__ float cm[G][kAttnMaxChunks];
        __shared__ float cl[G][kAttnMaxChunks];
        __shared__ float invl[G];
        __shared__ int last;
        // this block's partials are performed at the coherence point before it counts itself
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int nch = (seq + kAttnChunk - 1) / kAttnChunk - c0;  // blocks of the group that reach here
        if (t == 0)
            last = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(nch - 1);
        __syncthreads();
        if (!last) return;
        attn_combine_group<HD, G, true>(grp + (size_t)c0 * G * (HD + 2), nch,
                                        out + ((size_t)r * n_heads + (size_t)kvh * G) * HD, cm, cl, invl);
        if (t == 0) __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// One block per (row, kv head): its G query heads (the two-launch form).
template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                   const int32_t* __restrict__ pos, PagedKv kv,
                                                                   int n_kv_heads, int nch_max, int window,
                                                                   float* __restrict__ out)
{
    __shared__ float cm[G][kAttnMaxChunks];  // chunk maxima, then the weights e^(m_c - M)
    __shared__ float cl[G][kAttnMaxChunks];  // chunk exp-sums
    __shared__ float invl[G];
    const int n_heads = G * n_kv_heads;
    const int r = blockIdx.x / n_kv_heads, kvh = blockIdx.x % n_kv_heads;
    const int seq = min(pos[r] + 1, kv.max_blocks * kv.tpb);
    if (seq <= 0) return;
    const int c0 = window_start(seq, window) / kAttnChunk;  // the first chunk the window reaches
    const int nch = (seq + kAttnChunk - 1) / kAttnChunk - c0;
    const float* p = part + (((size_t)r * n_kv_heads + kvh) * nch_max + c0) * (size_t)G * (HD + 2);
    attn_combine_group<HD, G, false>(p, nch, out + ((size_t)r * n_heads + (size_t)kvh * G) * HD, cm, cl, invl);
}

// Whole-sequence attention in one block per (row, query head), for caches of
// at most S * 256 positions.  16 waves; wave w owns positions
// 256 s + 16 w .. + 15 of each sub-chunk s: Q.K with 4 lanes per position
// (attn_partial_kernel's mapping), P.V with 32 lanes per position and HD/32
// dims per lane, the two half-waves on alternate positions (one 4- or 8-byte
// V load per lane covers two positions), added across halves at the end.
// Every K and V load of the sequence is issued before any arithmetic and the
// softmax max and sum are reduced across the block in LDS, so the head's
// output is the block's only global write:
//   o = (sum_p e^(s_p - M) v_p) / (sum_p e^(s_p - M)),  M = max_p s_p
// (kvcache.rs:710-789, with the one maximum over the sequence the reference
// takes).  The G heads of a kv head read its K and V once each, through L2.
// The waves' P.V sums are added in a fixed order (waves 8..15 onto 0..7, then
// the eight in index order), so a call is deterministic.  A row with no
// position (pos < 0) writes nothing, as in the chunked kernels.
constexpr int kAttnBlockWaves = 16;
constexpr int kAttnBlockThreads = kAttnBlockWaves * 64;
constexpr int kAttnBlockSub = kAttnBlockWaves * 16;  // positions per sub-chunk

template <int HD, int S>
__global__ __launch_bounds__(kAttnBlockThreads) void attn_head_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, PagedKv kv, int layer, int n_heads, int group, float scale, float soft_cap,
    int window, float* __restrict__ out)
{
    constexpr int NW = kAttnBlockWaves, CAP = S * kAttnBlockSub;
    constexpr int KD = HD / 4;  // Q.K dims per lane
    constexpr int KL = KD / 8;  // 16-byte K loads per lane and sub-chunk
    constexpr int VD = HD / 32; // P.V dims per lane: 32 lanes per position, two positions per load
    using vword_t = typename std::conditional<VD == 2, uint32_t, u2_t>::type;
    __shared__ float qs[HD];
    __shared__ float ps[CAP];
    __shared__ long long bases[CAP];
    __shared__ float wmax[NW], wsum[NW];
    __shared__ float accs[NW / 2][HD];
    const int r = blockIdx.x / n_heads, h = blockIdx.x % n_heads, kvh = h / group;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // position, q and the page entries: independent loads, issued together
    const int p_r = pos[r];
    const float qv = q[((size_t)r * n_heads + h) * HD + min(t, HD - 1)];
    const int tp = min(t, CAP - 1), blk_i = tp / kv.tpb;
    const uint32_t blk = kv.bt[(size_t)r * kv.max_blocks + min(blk_i, kv.max_blocks - 1)];
    const int seq = min(p_r + 1, kv.max_blocks * kv.tpb);  // the launcher keeps max_blocks * tpb <= CAP
    if (seq <= 0) return;  // the same for the whole block
    const int s0 = window_start(seq, window);
    if (t < HD) qs[t] = qv;
    if (t < CAP)
        bases[t] = (t >= s0 && t < seq && blk_i < kv.max_blocks && blk < (uint32_t)kv.total_blocks)
                       ? ((long long)blk * kv.n_layers + layer) * (long long)kv.tpb * kv.kvd +
                             (long long)(t % kv.tpb) * kv.kvd
                       : -1;
    __syncthreads();

    // every K and V load (a missing page or a position past the sequence reads
    // element 0 and is zeroed)
    const int kq = lane & 3;
    u4_t kraw[S][KL];
    bool kok[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const long long kb = bases[s * kAttnBlockSub + wave * 16 + (lane >> 2)];
        kok[s] = kb >= 0;
        const u4_t* ksrc = reinterpret_cast<const u4_t*>(kc + (kb >= 0 ? kb + (long long)kvh * HD + kq * KD : 0));
#pragma unroll
        for (int j = 0; j < KL; ++j) kraw[s][j] = ksrc[j];
    }
    // V: lane l reads dims VD (l % 32) .. + VD - 1 of position 2i + l / 32 of the wave's 16
    const int vh = lane >> 5, vl = lane & 31;
    vword_t vraw[S][8];
    uint32_t vok[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        vok[s] = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const long long vb = bases[s * kAttnBlockSub + wave * 16 + 2 * i + vh];
            vok[s] |= (vb >= 0 ? 1u : 0u) << i;
            vraw[s][i] =
                *reinterpret_cast<const vword_t*>(vc + (vb >= 0 ? vb + (long long)kvh * HD + vl * VD : 0));
        }
    }

    // scores of this lane's positions, the wave maximum, then the block maximum
    float sc[S], mloc = -INFINITY;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < KL; ++j) {
            const h8_t kh = __builtin_bit_cast(h8_t, kok[s] ? kraw[s][j] : u4_t{0, 0, 0, 0});
#pragma unroll
            for (int e = 0; e < 8; ++e) dot = dot + qs[kq * KD + j * 8 + e] * (float)kh[e];
        }
        const int pp = s * kAttnBlockSub + wave * 16 + (lane >> 2);
        const bool valid = pp >= s0 && pp < seq;
        dot = dot + lane_xor<1>(dot, 64);
        dot = dot + lane_xor<2>(dot, 64);
        float sg = dot * scale;
        if (soft_cap > 0.0f) sg = tanhf(sg / soft_cap) * soft_cap;  // kvcache.rs:768-770
        sc[s] = valid ? sg : -INFINITY;
        mloc = fmaxf(mloc, sc[s]);
    }
    mloc = fmaxf(mloc, lane_xor<4>(mloc, 64));
    mloc = fmaxf(mloc, lane_xor<8>(mloc, 64));
    mloc = fmaxf(mloc, lane_xor<16>(mloc, 64));
    mloc = fmaxf(mloc, lane_xor<32>(mloc, 64));
    if (lane == 0) wmax[wave] = mloc;
    __syncthreads();
    // weights e^(s - M) into LDS (one lane of each position), and the wave sums
    float m = wmax[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, wmax[w]);
    float l = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int pp = s * kAttnBlockSub + wave * 16 + (lane >> 2);
        const bool valid = pp >= s0 && pp < seq;
        const float e = valid ? expf(sc[s] - m) : 0.0f;
        if (kq == 0) ps[s * kAttnBlockSub + wave * 16 + (lane >> 2)] = e;
        l = l + e;
    }
    l = l + lane_xor<4>(l, 64);
    l = l + lane_xor<8>(l, 64);
    l = l + lane_xor<16>(l, 64);
    l = l + lane_xor<32>(l, 64);
    if (lane == 0) wsum[wave] = l;
    __syncthreads();

    // weighted V over this wave's positions
    float acc[VD];
#pragma unroll
    for (int d = 0; d < VD; ++d) acc[d] = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float pg = ps[s * kAttnBlockSub + wave * 16 + 2 * i + vh];
            const bool ok = (vok[s] >> i) & 1u;
            if constexpr (VD == 2) {
                const uint32_t w = ok ? vraw[s][i] : 0u;
                acc[0] = acc[0] + pg * h2f((uint16_t)(w & 0xffffu));
                acc[1] = acc[1] + pg * h2f((uint16_t)(w >> 16));
            } else {
                const u2_t w = ok ? vraw[s][i] : u2_t{0u, 0u};
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    acc[2 * e] = acc[2 * e] + pg * h2f((uint16_t)(w[e] & 0xffffu));
                    acc[2 * e + 1] = acc[2 * e + 1] + pg * h2f((uint16_t)(w[e] >> 16));
                }
            }
        }
    // the two half-waves hold the even and odd positions: add across them
#pragma unroll
    for (int d = 0; d < VD; ++d) acc[d] = acc[d] + lane_xor<32>(acc[d], 64);
    // across the waves: 8..15 onto 0..7, then the eight in order
    if (wave >= NW / 2 && vh == 0) {
#pragma unroll
        for (int d = 0; d < VD; ++d) accs[wave - NW / 2][vl * VD + d] = acc[d];
    }
    __syncthreads();
    if (wave < NW / 2 && vh == 0) {
#pragma unroll
        for (int d = 0; d < VD; ++d) accs[wave][vl * VD + d] = acc[d] + accs[wave][vl * VD + d];
    }
    __syncthreads();
    if (t < HD) {
        float lt = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) lt = lt + wsum[w];
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < NW / 2; ++j) a = a + accs[j][t];
        out[((size_t)r * n_heads + h) * HD + t] = a * (lt > 0.0f ? 1.0f / lt : 0.0f);
    }
}

// ---- fused decode-step GEMVs: the shared prologue --------------------------------
// decode_i8_kernel and decode_q4_kernel (below) replace "residual add +
// RMSNorm, GEMV(s), epilogue op" with one launch.  Every block stages the whole
// normalised row(s) in LDS (each needs all of xn); block 0 also writes
// x_prev + y to x_out, the next residual stream, a different buffer from
// x_prev so that no block reads a row another has already overwritten.  The
// add and the scaling are those of add_rms_norm_kernel; the sum of squares is
// a tree of another shape (each thread sums 4 neighbouring elements first).
// xn is stored with 4 floats of padding after every 16 (lanes read it at a
// stride of 16 or 32 floats, which would put several lanes on each bank group).

__host__ __device__ __forceinline__ int xpad(int k) { return k + (k >> 4) * 4; }

// The prologue's inputs: thread t's float4 groups t, t + 256, ... (KR of them:
// KR * 1024 >= H) of every row of x_prev (and y) and of the norm weights.
// Loaded first (addresses clamped in range, no branch between them), before
// the weights of the kernel's dot: loads retire in issue order, so the
// prologue then waits for these alone and runs while the weights are in flight.
template <int MT, int KR>
struct NormIn {
    f4_t v[MT][KR], yv[MT][KR], wv[KR];
};

template <int MT, int KR, bool HASY>
__device__ __forceinline__ void load_add_norm(const float* __restrict__ x_prev, const float* __restrict__ y,
                                              const float* __restrict__ w, int rows, int H, NormIn<MT, KR>& in)
{
    const int t = threadIdx.x, H4 = H >> 2;
#pragma unroll
    for (int u = 0; u < KR; ++u) {
        const int g = min(t + u * kNormThreads, H4 - 1);
        in.wv[u] = reinterpret_cast<const f4_t*>(w)[g];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int mm = min(m, rows - 1);
            in.v[m][u] = reinterpret_cast<const f4_t*>(x_prev + (size_t)mm * H)[g];
            if constexpr (HASY) in.yv[m][u] = reinterpret_cast<const f4_t*>(y + (size_t)mm * H)[g];
        }
    }
}

// x rows [rows][H] -> LDS xs[MT][xpad(H)] = rms_norm(x_prev + y) * w from the
// loads of load_add_norm; block 0 writes x_prev + y to x_out (HASY false:
// x_prev as is).  Each thread's sum of squares runs over its groups in order,
// then the same wave and block tree as add_rms_norm_kernel.  CSUM
// (H % 32 == 0): also the sums of the normalised values over each 32-element
// chunk, xsum[m][H / 32] (the eight groups of a chunk sit in eight adjacent lanes).
template <int MT, int KR, bool HASY, bool CSUM = false>
__device__ __forceinline__ void stage_add_norm(NormIn<MT, KR>& in, float* __restrict__ x_out, int rows, int H,
                                               float eps, float* xs, float (*red)[MT], float* xsum = nullptr)
{
    const int t = threadIdx.x;
    const int xst = xpad(H), H4 = H >> 2;
    auto& v = in.v;
    if constexpr (HASY) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int u = 0; u < KR; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[m][u][e] = v[m][u][e] + in.yv[m][u][e];
    }
    // the rows' sums of squares (padding rows m >= rows sum nothing), reduced over the
    // wave transposed (lane l ends with row team_sum_t_index<64, MT>(l)), then over the waves
    float s[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        s[m] = 0.0f;
#pragma unroll
        for (int u = 0; u < KR; ++u) {
            const int g = t + u * kNormThreads;
            if (g < H4 && m < rows) {
#pragma unroll
                for (int e = 0; e < 4; ++e) s[m] = s[m] + v[m][u][e] * v[m][u][e];
            }
        }
    }
    {
        const float sw = team_sum_t<64, MT>(s);
        if ((t & (64 / MT - 1)) == 0) red[t >> 6][team_sum_t_index<64, MT>(t & 63)] = sw;
    }
    if (blockIdx.x == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int u = 0; u < KR; ++u) {
                const int g = t + u * kNormThreads;
                if (g < H4 && m < rows) reinterpret_cast<f4_t*>(x_out + (size_t)m * H)[g] = v[m][u];
            }
    }
    __syncthreads();
    // lane m of every wave computes row m's 1 / rms; every lane reads the MT values back
    float inv[MT];
    {
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < kNormThreads / 64; ++i) tot = tot + red[i][t & (MT - 1)];
        const float mean = tot / (float)H;
        const float il = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int m = 0; m < MT; ++m)
            inv[m] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, il), m));
    }
#pragma unroll
    for (int u = 0; u < KR; ++u) {
        const int g = t + u * kNormThreads;
        float cs[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            f4_t o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = v[m][u][e] * inv[m] * in.wv[u][e];
            if (g < H4) *reinterpret_cast<f4_t*>(xs + m * xst + xpad(4 * g)) = o;  // a group never straddles padding
            cs[m] = (o[0] + o[1]) + (o[2] + o[3]);
        }
        if constexpr (CSUM) {
            // H4 % 8 == 0: the eight groups of a chunk are all in range or all out; the MT chunk
            // sums reduced over the eight lanes transposed (MT <= 8)
            const float c = team_sum_t<8, MT>(cs);
            if (g < H4 && (t & (8 / MT - 1)) == 0) xsum[team_sum_t_index<8, MT>(t & 7) * (H >> 5) + (g >> 3)] = c;
        }
    }
    __syncthreads();
}

struct DecodeQkvArgs {
    const float* x_prev;
    const float* y;
    float* x_out;
    const float* norm_w;
    float eps;
    const int8_t* w[3];    // q, k, v [rows_out][H]
    const uint16_t* s[3];  // f16 row scales
    int rows, H, n_heads, n_kv_heads, head_dim;
    const int32_t* pos;
    const float2* cs;
    int table_positions;
    float* q_out;
    uint16_t* kc;
    uint16_t* vc;
    PagedKv kv;
    int layer;
    int il;  // RoPE pairs: 0 rotate-half (i, i + half), 1 interleaved (2i, 2i + 1)
};

struct DecodeGateUpArgs {
    const float* x_prev;
    const float* y;
    float* x_out;
    const float* norm_w;
    float eps;
    const int8_t* wg;
    const uint16_t* sg;
    const int8_t* wu;
    const uint16_t* su;
    int rows, H, N;
    float* h;  // [rows][N]
};

// ---- fused decode-step GEMVs over MLX q4 affine weights ---------------------
// The q4 counterparts of the two kernels above, for the u32 runners (the Qwen2
// step, qwen.rs:1255-1470, whose projections are linear_i4_out_in,
// lfm.rs:985-1066, over f32 activations).  Same prologue (stage_add_norm, with
// the 32-element chunk sums of xn).  A team of LPR lanes owns RP units of two
// output rows (a RoPE pair, or row n of gate and of up); each lane holds C
// 16-byte chunks of every row, loaded before the prologue.  A chunk is 32
// nibbles of one row: four u32 words, element 8j + e = nibble e of word j.  The
// dot is plain f32: the nibbles widened by v_cvt_f32_ubyteN meet xn in FMA
// chains, and one group scale and bias cover the whole chunk (group >= 32):
//   y[n] = sum_c ( S[n][g(c)] * sum_{k in c} q[n][k] xn[k] + B[n][g(c)] * xsum[c] )
// which is sum_k (q S + B) xn in another summation order.  All MT activation
// rows are computed (padding rows repeat the last one and are never stored), so
// the dot has no per-row branch.  The RP * 2 * MT row sums of a lane are summed
// over the team transposed (team_sum_t); a lane then pairs the two rows of its
// (unit, session) value and runs the epilogue once.

struct DecodeQ4QkvArgs {
    const float* x_prev;
    const float* y;
    float* x_out;
    const float* norm_w;
    float eps;
    const u4_t* w[3];  // q, k, v: u32 words [rows_out][H / 8] as 16-byte chunks
    const float* s[3];  // scales and biases [rows_out][H / group]
    const float* b[3];
    const float* bias[3];  // projection biases [rows_out] or null
    int rows, H, n_heads, n_kv_heads, head_dim, gshift;
    const int32_t* pos;
    const float2* cs;
    int table_positions;
    float* q_out;
    uint16_t* kc;
    uint16_t* vc;
    PagedKv kv;
    int layer;
    int il;
};

struct DecodeQ4GateUpArgs {
    const float* x_prev;
    const float* y;
    float* x_out;
    const float* norm_w;
    float eps;
    const u4_t* wg;
    const float* sg;
    const float* bg;
    const u4_t* wu;
    const float* su;
    const float* bu;
    int rows, H, N, gshift, act;
    float* h;  // [rows][N]
};

// Unit -> its two rows.  QKV: pair p < units of (q heads, k heads, v heads) x
// head_dim / 2, rows i0 and i1 of one head (rope_lo / rope_hi).  Gate/up: row
// n of each matrix.
struct Q4Unit {
    const u4_t* w0;
    const u4_t* w1;
    const float* s0;
    const float* b0;
    const float* s1;
    const float* b1;
    size_t g0, g1;  // first scale/bias index of each row
    int which, head, i, i0, i1, r0, r1;
};

__device__ __forceinline__ Q4Unit q4_unit(const DecodeQ4QkvArgs& a, int p, int cpr, int gpr)
{
    Q4Unit u;
    const int half = a.head_dim >> 1;
    const int hh = p / half;
    u.i = p - hh * half;
    u.which = hh < a.n_heads ? 0 : (hh < a.n_heads + a.n_kv_heads ? 1 : 2);
    u.head = u.which == 0 ? hh : (u.which == 1 ? hh - a.n_heads : hh - a.n_heads - a.n_kv_heads);
    u.i0 = rope_lo(u.i, half, a.il);
    u.i1 = rope_hi(u.i, half, a.il);
    u.r0 = u.head * a.head_dim + u.i0;
    u.r1 = u.head * a.head_dim + u.i1;
    const u4_t* wm = u.which == 0 ? a.w[0] : (u.which == 1 ? a.w[1] : a.w[2]);
    u.s0 = u.s1 = u.which == 0 ? a.s[0] : (u.which == 1 ? a.s[1] : a.s[2]);
    u.b0 = u.b1 = u.which == 0 ? a.b[0] : (u.which == 1 ? a.b[1] : a.b[2]);
    u.w0 = wm + (size_t)u.r0 * cpr;
    u.w1 = wm + (size_t)u.r1 * cpr;
    u.g0 = (size_t)u.r0 * gpr;
    u.g1 = (size_t)u.r1 * gpr;
    return u;
}

__device__ __forceinline__ Q4Unit q4_unit(const DecodeQ4GateUpArgs& a, int n, int cpr, int gpr)
{
    Q4Unit u{};
    u.w0 = a.wg + (size_t)n * cpr;
    u.w1 = a.wu + (size_t)n * cpr;
    u.s0 = a.sg;
    u.b0 = a.bg;
    u.s1 = a.su;
    u.b1 = a.bu;
    u.g0 = u.g1 = (size_t)n * gpr;
    u.r0 = u.r1 = n;
    return u;
}

template <class Args>
__host__ __device__ __forceinline__ int q4_units(const Args& a)
{
    if constexpr (std::is_same<Args, DecodeQ4QkvArgs>::value)
        return (a.n_heads + 2 * a.n_kv_heads) * (a.head_dim >> 1);
    else
        return a.N;
}

// The epilogue's loads for one (unit, session), issued with a kernel's prologue: a lane's
// epilogue unit and session are fixed by its lane (team_sum_t_index), so its position, RoPE row
// and page base (QKV), its projection biases (q4 QKV) and its row scales (int8) need not wait for
// the dot.  QKV: the position is loaded first (*_epi_pos), the RoPE row and the page base after
// the prologue's own loads are issued (rope_prefetch).
struct EpiPre {
    int pr = 0;        // the session's position
    float2 c{};        // cos / sin of the RoPE pair at pr
    long long b = -1;  // K/V element base of (session, pr), or -1
    float s0 = 0.0f, s1 = 0.0f;  // int8 row scales, or q4 projection biases of the unit's two rows
};

template <class A>
__device__ __forceinline__ void rope_prefetch(const A& a, int which, int i, int m, EpiPre& e)
{
    const int half = a.head_dim >> 1;
    e.c = a.cs[(size_t)min(max(e.pr, 0), a.table_positions - 1) * half + i];
    e.b = (which != 0 && e.pr >= 0) ? a.kv.base(m, e.pr, a.layer) : -1;
}

// RoPE on the pair (v0, v1) of head `head`, rows i0 / i1, with the prefetched table row (pair i
// at session m's position), then q into q_out or k / v into the paged cache as f16 (the
// arithmetic of rope_kv_write_kernel).  Shared by the int8 and q4 QKV kernels.
template <class A>
__device__ __forceinline__ void rope_kv_store(const A& a, int which, int head, int i0, int i1, int m, const EpiPre& e,
                                              float v0, float v1)
{
    const float2 c = e.c;
    if (which == 0) {
        float* q = a.q_out + ((size_t)m * a.n_heads + head) * a.head_dim;
        q[i0] = v0 * c.x - v1 * c.y;
        q[i1] = v1 * c.x + v0 * c.y;
        return;
    }
    if (e.b < 0) return;
    const size_t el = (size_t)e.b + (size_t)head * a.head_dim;
    if (which == 1) {
        a.kc[el + i0] = __builtin_bit_cast(uint16_t, (_Float16)(v0 * c.x - v1 * c.y));
        a.kc[el + i1] = __builtin_bit_cast(uint16_t, (_Float16)(v1 * c.x + v0 * c.y));
    } else {
        a.vc[el + i0] = __builtin_bit_cast(uint16_t, (_Float16)v0);
        a.vc[el + i1] = __builtin_bit_cast(uint16_t, (_Float16)v1);
    }
}

// (unit, session m) epilogue with the unit's two row sums v0, v1
// (unit, session m) epilogue of the q4 kernel over its prefetched values (EpiPre: position,
// RoPE row, page base, projection biases)
__device__ __forceinline__ void q4_epi_pos(const DecodeQ4QkvArgs& a, int m, EpiPre& e) { e.pr = a.pos[m]; }
__device__ __forceinline__ void q4_epi_pos(const DecodeQ4GateUpArgs&, int, EpiPre&) {}
__device__ __forceinline__ void q4_epi_prefetch(const DecodeQ4QkvArgs& a, const Q4Unit& u, int m, EpiPre& e)
{
    const float* pb = u.which == 0 ? a.bias[0] : (u.which == 1 ? a.bias[1] : a.bias[2]);
    const float z = 0.0f;
    e.s0 = *(pb ? pb + u.r0 : &z);
    e.s1 = *(pb ? pb + u.r1 : &z);
    rope_prefetch(a, u.which, u.i, m, e);
}
__device__ __forceinline__ void q4_epi_prefetch(const DecodeQ4GateUpArgs&, const Q4Unit&, int, EpiPre&) {}
__device__ __forceinline__ void q4_epilogue(const DecodeQ4QkvArgs& a, const Q4Unit& u, int m, const EpiPre& e,
                                            float v0, float v1)
{
    const float* pb = u.which == 0 ? a.bias[0] : (u.which == 1 ? a.bias[1] : a.bias[2]);
    if (pb) {  // add_projection_bias_if_present, then RoPE
        v0 = v0 + e.s0;
        v1 = v1 + e.s1;
    }
    rope_kv_store(a, u.which, u.head, u.i0, u.i1, m, e, v0, v1);
}
__device__ __forceinline__ void q4_epilogue(const DecodeQ4GateUpArgs& a, const Q4Unit& u, int m, const EpiPre&,
                                            float v0, float v1)
{
    a.h[(size_t)m * a.N + u.r0] = act_mul(a.act, v0, v1);
}

template <int LPR, int C, int RP, int MT, int KR, bool HASY, class Args>
__global__ __launch_bounds__(256) void decode_q4_kernel(Args a)
{
    constexpr int V = RP * 2 * MT;  // row sums per lane: [unit p][row r][session m]
    static_assert(V <= LPR, "one transposed value per lane");
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[kNormThreads / 64][MT];
    const int H = a.H, cpr = H >> 5;
    const int gpr = (H + (1 << a.gshift) - 1) >> a.gshift;
    const int team = threadIdx.x / LPR, lane = threadIdx.x % LPR;
    const int units = q4_units(a);
    const int unit0 = (blockIdx.x * (256 / LPR) + team) * RP;

    NormIn<MT, KR> nin;
    load_add_norm<MT, KR, HASY>(a.x_prev, a.y, a.norm_w, a.rows, H, nin);
    u4_t w[C][RP][2];
    float sb[C][RP][2][2];
#pragma unroll
    for (int p = 0; p < RP; ++p) {
        const Q4Unit u = q4_unit(a, min(unit0 + p, units - 1), cpr, gpr);
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int ch = min(lane + c * LPR, cpr - 1);
            const int gi = (ch << 5) >> a.gshift;
            w[c][p][0] = __builtin_nontemporal_load(u.w0 + ch);
            w[c][p][1] = __builtin_nontemporal_load(u.w1 + ch);
            sb[c][p][0][0] = u.s0[u.g0 + gi];
            sb[c][p][0][1] = u.b0[u.g0 + gi];
            sb[c][p][1][0] = u.s1[u.g1 + gi];
            sb[c][p][1][1] = u.b1[u.g1 + gi];
        }
    }

    float* xsum = xs + MT * xpad(H);
    stage_add_norm<MT, KR, HASY, true>(nin, a.x_out, a.rows, H, a.eps, xs, red, xsum);

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    const int xst = xpad(H);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int ch = lane + c * LPR;
        if (ch >= cpr) break;
        float d[V];
#pragma unroll
        for (int i = 0; i < V; ++i) d[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float q[RP][2][8];
#pragma unroll
            for (int p = 0; p < RP; ++p)
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const uint32_t wd = w[c][p][r][j];
                    const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
                    q[p][r][0] = cvt_ubyte<0>(lo);
                    q[p][r][1] = cvt_ubyte<0>(hi);
                    q[p][r][2] = cvt_ubyte<1>(lo);
                    q[p][r][3] = cvt_ubyte<1>(hi);
                    q[p][r][4] = cvt_ubyte<2>(lo);
                    q[p][r][5] = cvt_ubyte<2>(hi);
                    q[p][r][6] = cvt_ubyte<3>(lo);
                    q[p][r][7] = cvt_ubyte<3>(hi);
                }
            // elements 32 ch + 8 j + 0..7 sit at xpad(...) = 40 ch + 8 j + (j >= 2 ? 4 : 0) + 0..7
            const int xo = 40 * ch + 8 * j + (j >= 2 ? 4 : 0);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const f4_t* xp = reinterpret_cast<const f4_t*>(xs + m * xst + xo);
                const f4_t x0 = xp[0], x1 = xp[1];
                const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int p = 0; p < RP; ++p)
#pragma unroll
                    for (int r = 0; r < 2; ++r)
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            float& dd = d[(p * 2 + r) * MT + m];
                            dd = __builtin_fmaf(q[p][r][e], xv[e], dd);
                        }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float xc = xsum[m * cpr + ch];
#pragma unroll
            for (int p = 0; p < RP; ++p)
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int vi = (p * 2 + r) * MT + m;
                    acc[vi] += sb[c][p][r][0] * d[vi] + sb[c][p][r][1] * xc;
                }
        }
    }
    // lane -> value index (p * 2 + r) * MT + m; the row-1 partner of a row-0 lane is
    // LPR / (2 RP) lanes up (the halving step that split on r)
    const float tot = team_sum_t<LPR, V>(acc);
    constexpr int RO = LPR / (2 * RP);
    float other;
    if constexpr (RO >= 16)
        other = swap_xor<RO>(tot);
    else
        other = lane_xor<RO>(tot, LPR);
    const int vi = team_sum_t_index<LPR, V>(lane);
    const int p = vi / (2 * MT), r = (vi / MT) & 1, m = vi % MT;
    if (r != 0 || (lane & (LPR / V - 1)) != 0 || m >= a.rows || unit0 + p >= units) return;
    // the q4 kernels load the epilogue's values here, after the dot (issued with the prologue they
    // measured 2-6 us slower per Qwen2-shape step)
    const Q4Unit u = q4_unit(a, unit0 + p, cpr, gpr);
    EpiPre epre;
    q4_epi_pos(a, m, epre);
    q4_epi_prefetch(a, u, m, epre);
    q4_epilogue(a, u, m, epre, tot, other);
}

// ---- fused decode-step GEMVs over int8 weights -------------------------------
// One launch replaces "residual add + RMSNorm, int8 GEMV(s), epilogue op" for
// the int8 Llama step (llama_graph.rs:245-327):
//   QKV:     xn = rms_norm(x_prev + y) * w;  q, k, v = W xn;  RoPE on q and k;
//            k and v into the paged cache
//   gate/up: xn = rms_norm(x_prev + y) * w;  h = silu(Wg xn) * (Wu xn)
// The layout of decode_q4_kernel: every block stages the normalised rows
// (stage_add_norm; block 0 also writes x_prev + y to x_out, a different buffer
// from x_prev, so that no block reads a row another has already overwritten),
// a team of LPR lanes owns RP units of two rows, a lane C 16-byte chunks
// (16 int8) of each, loaded after the prologue's inputs and before its work.
// The dot is f32 FMA over the widened bytes; the row sums are summed over the
// team transposed and scaled by the f16 row scale (matmul_i8_f32: the sum,
// then the scale) in the epilogue.

struct I8Unit {
    const u4_t* w0;
    const u4_t* w1;
    const uint16_t* s0;
    const uint16_t* s1;
    int which, head, i, i0, i1, r0, r1;
};

__device__ __forceinline__ I8Unit i8_unit(const DecodeQkvArgs& a, int p, int cpr)
{
    I8Unit u;
    const int half = a.head_dim >> 1;
    const int hh = p / half;
    u.i = p - hh * half;
    u.which = hh < a.n_heads ? 0 : (hh < a.n_heads + a.n_kv_heads ? 1 : 2);
    u.head = u.which == 0 ? hh : (u.which == 1 ? hh - a.n_heads : hh - a.n_heads - a.n_kv_heads);
    u.i0 = rope_lo(u.i, half, a.il);
    u.i1 = rope_hi(u.i, half, a.il);
    u.r0 = u.head * a.head_dim + u.i0;
    u.r1 = u.head * a.head_dim + u.i1;
    const u4_t* wm = reinterpret_cast<const u4_t*>(u.which == 0 ? a.w[0] : (u.which == 1 ? a.w[1] : a.w[2]));
    u.s0 = u.s1 = u.which == 0 ? a.s[0] : (u.which == 1 ? a.s[1] : a.s[2]);
    u.w0 = wm + (size_t)u.r0 * cpr;
    u.w1 = wm + (size_t)u.r1 * cpr;
    return u;
}

__device__ __forceinline__ I8Unit i8_unit(const DecodeGateUpArgs& a, int n, int cpr)
{
    I8Unit u{};
    u.w0 = reinterpret_cast<const u4_t*>(a.wg) + (size_t)n * cpr;
    u.w1 = reinterpret_cast<const u4_t*>(a.wu) + (size_t)n * cpr;
    u.s0 = a.sg;
    u.s1 = a.su;
    u.r0 = u.r1 = n;
    return u;
}

template <class Args>
__host__ __device__ __forceinline__ int i8_units(const Args& a)
{
    if constexpr (std::is_same<Args, DecodeQkvArgs>::value)
        return (a.n_heads + 2 * a.n_kv_heads) * (a.head_dim >> 1);
    else
        return a.N;
}

__device__ __forceinline__ void i8_epi_pos(const DecodeQkvArgs& a, int m, EpiPre& e) { e.pr = a.pos[m]; }
__device__ __forceinline__ void i8_epi_pos(const DecodeGateUpArgs&, int, EpiPre&) {}
__device__ __forceinline__ void i8_epi_prefetch(const DecodeQkvArgs& a, const I8Unit& u, int m, EpiPre& e)
{
    e.s0 = h2f(u.s0[u.r0]);
    e.s1 = h2f(u.s1[u.r1]);
    rope_prefetch(a, u.which, u.i, m, e);
}
__device__ __forceinline__ void i8_epi_prefetch(const DecodeGateUpArgs&, const I8Unit& u, int, EpiPre& e)
{
    e.s0 = h2f(u.s0[u.r0]);
    e.s1 = h2f(u.s1[u.r1]);
}

__device__ __forceinline__ void i8_epilogue(const DecodeQkvArgs& a, const I8Unit& u, int m, const EpiPre& e, float v0,
                                            float v1)
{
    rope_kv_store(a, u.which, u.head, u.i0, u.i1, m, e, v0, v1);
}

// h = silu(g) * u as silu_mul_f32_inplace (metal.rs:235-245): (g * (1 / (1 + exp(-g)))) * u
__device__ __forceinline__ void i8_epilogue(const DecodeGateUpArgs& a, const I8Unit& u, int m, const EpiPre&, float v0,
                                            float v1)
{
    a.h[(size_t)m * a.N + u.r0] = act_mul(ACT_SILU, v0, v1);
}

template <int LPR, int C, int RP, int MT, int KR, bool HASY, class Args>
__global__ __launch_bounds__(256) void decode_i8_kernel(Args a)
{
    constexpr int V = RP * 2 * MT;  // row sums per lane: [unit p][row r][session m]
    static_assert(V <= LPR, "one transposed value per lane");
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[kNormThreads / 64][MT];
    const int H = a.H, cpr = H >> 4;
    const int team = threadIdx.x / LPR, lane = threadIdx.x % LPR;
    const int units = i8_units(a);
    const int unit0 = (blockIdx.x * (256 / LPR) + team) * RP;
    // this lane's epilogue (unit ep, session em): its position first, its row scales, RoPE row and
    // page base after the prologue's loads (EpiPre)
    const int evi = team_sum_t_index<LPR, V>(lane), ep = evi / (2 * MT), em = min(evi % MT, a.rows - 1);
    EpiPre epre;
    i8_epi_pos(a, em, epre);

    NormIn<MT, KR> nin;
    load_add_norm<MT, KR, HASY>(a.x_prev, a.y, a.norm_w, a.rows, H, nin);
    u4_t w[C][RP][2];
#pragma unroll
    for (int p = 0; p < RP; ++p) {
        const I8Unit u = i8_unit(a, min(unit0 + p, units - 1), cpr);
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int ch = min(lane + c * LPR, cpr - 1);
            w[c][p][0] = u.w0[ch];
            w[c][p][1] = u.w1[ch];
        }
    }
    i8_epi_prefetch(a, i8_unit(a, min(unit0 + ep, units - 1), cpr), em, epre);

    stage_add_norm<MT, KR, HASY>(nin, a.x_out, a.rows, H, a.eps, xs, red);

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    const int xst = xpad(H);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int ch = lane + c * LPR;
        if (ch >= cpr) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float q[RP][2][4];
#pragma unroll
            for (int p = 0; p < RP; ++p)
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[p][r][e] = (float)(int8_t)(w[c][p][r][j] >> (8 * e));
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                // elements 16 ch + 4 j + 0..3 sit at xpad(...) = 20 ch + 4 j + 0..3
                const f4_t xv = *reinterpret_cast<const f4_t*>(xs + m * xst + 20 * ch + 4 * j);
#pragma unroll
                for (int p = 0; p < RP; ++p)
#pragma unroll
                    for (int r = 0; r < 2; ++r)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float& dd = acc[(p * 2 + r) * MT + m];
                            dd = __builtin_fmaf(q[p][r][e], xv[e], dd);
                        }
            }
        }
    }
    const float tot = team_sum_t<LPR, V>(acc);
    constexpr int RO = LPR / (2 * RP);
    float other;
    if constexpr (RO >= 16)
        other = swap_xor<RO>(tot);
    else
        other = lane_xor<RO>(tot, LPR);
    const int vi = team_sum_t_index<LPR, V>(lane);
    const int p = vi / (2 * MT), r = (vi / MT) & 1, m = vi % MT;
    if (r != 0 || (lane & (LPR / V - 1)) != 0 || m >= a.rows || unit0 + p >= units) return;
    const I8Unit u = i8_unit(a, unit0 + p, cpr);
    i8_epilogue(a, u, m, epre, tot * epre.s0, other * epre.s1);
}

// ---- MLX q4 affine GEMV over f32 activations (M <= 4), f32 dot ---------------
// y[m][n] = sum_k (q[n][k] S[n][k/g] + B[n][k/g]) x[m][k] for the u32 runners'
// projections that take no prologue (o_proj, down_proj: linear_i4_out_in,
// lfm.rs:985-1066).  x is copied to LDS as f32 (the layout of stage_add_norm,
// with the 32-element chunk sums), and the dot is dot_rows_q4's: no f16
// rounding of x, so nothing to scale per chunk.  A team of LPR lanes owns R
// consecutive rows, C chunks of each per lane (one pass: C * LPR >= K / 32).

// x [M][K] -> xs[MT][xpad(K)], xsum[MT][K / 32]; padding rows m >= M repeat row
// M - 1 (never stored).  Rounds of XU float4 groups per thread, all loads of a
// round issued before its stores; a chunk's eight groups sit in eight adjacent lanes.
template <int MT, int XU, int NT = kNormThreads>
__device__ __forceinline__ void stage_x32(const float* __restrict__ x, int M, int K, float* xs, float* xsum)
{
    const int t = threadIdx.x, K4 = K >> 2, total = MT * K4;
    for (int base = 0; base < total; base += XU * NT) {
        f4_t v[XU];
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            // x rows are contiguous: group g at x + 4 g (padding rows read the last real group)
            v[u] = reinterpret_cast<const f4_t*>(x)[min(base + u * NT + t, min(total, M * K4) - 1)];
        }
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            // row m = g / K4, group k4: LDS m * xpad(K) + xpad(4 k4) = xpad(4 g) and chunk m * cpr +
            // k4 / 8 = g / 8 (K % 32 == 0), so no division
            const int g = base + u * NT + t;
            if (g < total) *reinterpret_cast<f4_t*>(xs + xpad(4 * g)) = v[u];
            // total % 8 == 0 (K4 % 8 == 0): a chunk's groups are all in range or all out
            const float cs = group_sum<8>((v[u][0] + v[u][1]) + (v[u][2] + v[u][3]));
            if (g < total && (t & 7) == 0) xsum[g >> 3] = cs;
        }
    }
    __syncthreads();
}

template <int LPR, int C, int R, int MT, int XU>
__global__ __launch_bounds__(256) void qgemv_q4_x32_kernel(const u4_t* __restrict__ wq, const float* __restrict__ S,
                                                           const float* __restrict__ B, const float* __restrict__ x,
                                                           float* __restrict__ y, int M, int N, int K, int gshift)
{
    extern __shared__ __align__(16) float xs[];
    const int cpr = K >> 5, gpr = (K + (1 << gshift) - 1) >> gshift;
    const int team = threadIdx.x / LPR, lane = threadIdx.x % LPR;
    const int row0 = (blockIdx.x * (256 / LPR) + team) * R;
    u4_t w[C][R];
    float sb[C][R][2];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int ch = min(lane + c * LPR, cpr - 1);
        const int gi = (ch << 5) >> gshift;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(row0 + r, N - 1);
            w[c][r] = __builtin_nontemporal_load(wq + (size_t)n * cpr + ch);
            sb[c][r][0] = S[(size_t)n * gpr + gi];
            sb[c][r][1] = B[(size_t)n * gpr + gi];
        }
    }
    float* xsum = xs + MT * xpad(K);
    stage_x32<MT, XU>(x, M, K, xs, xsum);

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
    const int xst = xpad(K);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int ch = lane + c * LPR;
        if (ch >= cpr) break;
        float d[R][MT];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) d[r][m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float q[R][8];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t lo = w[c][r][j] & 0x0F0F0F0Fu, hi = (w[c][r][j] >> 4) & 0x0F0F0F0Fu;
                q[r][0] = cvt_ubyte<0>(lo);
                q[r][1] = cvt_ubyte<0>(hi);
                q[r][2] = cvt_ubyte<1>(lo);
                q[r][3] = cvt_ubyte<1>(hi);
                q[r][4] = cvt_ubyte<2>(lo);
                q[r][5] = cvt_ubyte<2>(hi);
                q[r][6] = cvt_ubyte<3>(lo);
                q[r][7] = cvt_ubyte<3>(hi);
            }
            const int xo = 40 * ch + 8 * j + (j >= 2 ? 4 : 0);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m >= M) break;
                const f4_t* xp = reinterpret_cast<const f4_t*>(xs + m * xst + xo);
                const f4_t x0 = xp[0], x1 = xp[1];
                const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int e = 0; e < 8; ++e) d[r][m] = __builtin_fmaf(q[r][e], xv[e], d[r][m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= M) break;
            const float xc = xsum[m * cpr + ch];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][m] += sb[c][r][0] * d[r][m] + sb[c][r][1] * xc;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = group_sum<LPR>(acc[r][m]);
    // lane r * MT + m stores (row0 + r, m)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (lane == r * MT + m && m < M && row0 + r < N) y[(size_t)m * N + row0 + r] = acc[r][m];
}

// Long rows (K > 2048, 1..4 activation rows): one block of KS * RB waves
// stages x once (every thread one round of loads) and splits each of its RB
// rows over KS waves, wave (ks, rb) taking chunks [ks * cps, (ks + 1) * cps),
// one per lane (cps <= 64).  Each wave sums its rows transposed
// (team_sum_t<64, MT>), the partials meet in LDS, and one lane per (row,
// session) adds the KS partials in slice order and stores.  Every wave gets
// a 1/KS share of the row's dot, so the block's VALU work spreads over KS
// times more waves than one-wave-per-row teams.
template <int KS, int RB, int MT, int XU>
__global__ __launch_bounds__(KS * RB * 64) void qgemv_q4_x32s_kernel(
    const u4_t* __restrict__ wq, const float* __restrict__ S, const float* __restrict__ B, const float* __restrict__ x,
    float* __restrict__ y, int M, int N, int K, int gshift)
{
    constexpr int NT = KS * RB * 64;
    extern __shared__ __align__(16) float xs[];
    __shared__ float part[KS][RB][MT];
    const int cpr = K >> 5, gpr = (K + (1 << gshift) - 1) >> gshift, cps = (cpr + KS - 1) / KS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ks = wave / RB, rb = wave % RB;
    const int n = min((int)blockIdx.x * RB + rb, N - 1);
    const int ch_raw = ks * cps + lane;
    const bool live = lane < cps && ch_raw < cpr;
    const int ch = min(ch_raw, cpr - 1);
    const int gi = (ch << 5) >> gshift;
    const u4_t wv = __builtin_nontemporal_load(wq + (size_t)n * cpr + ch);
    const float sc = S[(size_t)n * gpr + gi], bc = B[(size_t)n * gpr + gi];
    float* xsum = xs + MT * xpad(K);
    stage_x32<MT, XU, NT>(x, M, K, xs, xsum);

    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    if (live) {
        float d[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) d[m] = 0.0f;
        const int xst = xpad(K);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = wv[j] & 0x0F0F0F0Fu, hi = (wv[j] >> 4) & 0x0F0F0F0Fu;
            const float q[8] = {cvt_ubyte<0>(lo), cvt_ubyte<0>(hi), cvt_ubyte<1>(lo), cvt_ubyte<1>(hi),
                                cvt_ubyte<2>(lo), cvt_ubyte<2>(hi), cvt_ubyte<3>(lo), cvt_ubyte<3>(hi)};
            const int xo = 40 * ch + 8 * j + (j >= 2 ? 4 : 0);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const f4_t* xp = reinterpret_cast<const f4_t*>(xs + m * xst + xo);
                const f4_t x0 = xp[0], x1 = xp[1];
                const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int e = 0; e < 8; ++e) d[m] = __builtin_fmaf(q[e], xv[e], d[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = sc * d[m] + bc * xsum[m * cpr + ch];
    }
    const float tot = team_sum_t<64, MT>(acc);
    if ((lane & (64 / MT - 1)) == 0) part[ks][rb][team_sum_t_index<64, MT>(lane)] = tot;
    __syncthreads();
    if (threadIdx.x < RB * MT) {
        const int r = threadIdx.x / MT, m = threadIdx.x % MT;
        const int row = (int)blockIdx.x * RB + r;
        float v = part[0][r][m];
#pragma unroll
        for (int k = 1; k < KS; ++k) v = v + part[k][r][m];
        if (m < M && row < N) y[(size_t)m * N + row] = v;
    }
}

// Chunk blocks per row: block (c, r) takes elements [c * kArgmaxChunk, (c + 1) * kArgmaxChunk) of
// row r, every thread loading all of its kArgmaxUnroll float4 before it compares any (one memory
// latency per block).  A thread takes the largest of its values (non-finite ones count as -inf,
// llama.rs:1081-1092) and then the lowest index holding it: two short independent passes instead
// of one compare chain.  Waves and the block reduce (value, index) pairs keeping the lower index
// among equal values.  With one chunk the block writes the row's result; otherwise it publishes
// (value, index) with agent-coherent stores, performed before it counts itself on the row's
// counter, and the row's last block combines the chunks (wave 0, one partial per lane) and returns
// the counter to zero.  Every reduction keeps the lower index among equal values, so the result is
// the first maximum in any combining order (topk_from_logits(..)[0], llama.rs:1049-1078).
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxUnroll = 4;
constexpr int kArgmaxChunk = kArgmaxThreads * 4 * kArgmaxUnroll;  // 4096 elements, 16 KB

__device__ __forceinline__ void argmax_pick(float ov, int oi, float& best, int& bi)
{
    if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
    }
}

__device__ __forceinline__ void argmax_wave(float& best, int& bi)
{
    for (int off = 32; off > 0; off >>= 1) argmax_pick(__shfl_xor(best, off), __shfl_xor(bi, off), best, bi);
}

// The first maximum of chunk c of row z (n elements): valid in thread 0 on return; sv/si are the
// block's wave slots.
__device__ __forceinline__ void argmax_chunk(const float* __restrict__ z, int n, int c, float (&sv)[kArgmaxThreads / 64],
                                             int (&si)[kArgmaxThreads / 64], float& best, int& bi)
{
    const int t = threadIdx.x;
    const int beg = c * kArgmaxChunk, end = min(n, beg + kArgmaxChunk);
    best = -INFINITY;
    bi = 0x7fffffff;
    if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(z) & 15) == 0) {
        const float4* z4 = reinterpret_cast<const float4*>(z);
        const int j0 = beg >> 2, j1 = end >> 2;
        float v[kArgmaxUnroll][4];
#pragma unroll
        for (int u = 0; u < kArgmaxUnroll; ++u) {
            const float4 a = z4[min(j0 + u * kArgmaxThreads + t, j1 - 1)];
            v[u][0] = a.x;
            v[u][1] = a.y;
            v[u][2] = a.z;
            v[u][3] = a.w;
        }
#pragma unroll
        for (int u = 0; u < kArgmaxUnroll; ++u) {
            const bool in = j0 + u * kArgmaxThreads + t < j1;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[u][e] = in && isfinite(v[u][e]) ? v[u][e] : -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < kArgmaxUnroll; ++u)
            mx = fmaxf(mx, fmaxf(fmaxf(v[u][0], v[u][1]), fmaxf(v[u][2], v[u][3])));
        // the lowest in-range index holding mx (an all -inf thread: its first in-range element)
#pragma unroll
        for (int u = kArgmaxUnroll - 1; u >= 0; --u) {
            const int j = j0 + u * kArgmaxThreads + t;
            if (j < j1) {
#pragma unroll
                for (int e = 3; e >= 0; --e) bi = v[u][e] == mx ? 4 * j + e : bi;
            }
        }
        best = mx;
    } else {
        for (int i = beg + t; i < end; i += kArgmaxThreads) {
            float x = z[i];
            if (!isfinite(x)) x = -INFINITY;
            argmax_pick(x, i, best, bi);  // ties keep the lower index: the first element counts even at -inf
        }
    }
    argmax_wave(best, bi);
    if ((t & 63) == 0) {
        sv[t >> 6] = best;
        si[t >> 6] = bi;
    }
    __syncthreads();
    if (t == 0)
        for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_pick(sv[w], si[w], best, bi);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits, int n,
                                                                int32_t* __restrict__ idx, float* __restrict__ val,
                                                                uint32_t* __restrict__ cnt, float2* __restrict__ part)
{
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    __shared__ int last;
    const int c = blockIdx.x, r = blockIdx.y, t = threadIdx.x, nch = gridDim.x;
    float best;
    int bi;
    argmax_chunk(logits + (size_t)r * n, n, c, sv, si, best, bi);
    if (t == 0) {
        if (nch == 1) {
            idx[r] = bi == 0x7fffffff ? 0 : bi;
            val[r] = best;
        } else {
            float2* p = part + (size_t)r * nch + c;
            __hip_atomic_store(&p->x, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&p->y, __builtin_bit_cast(float, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // performed before the count
            last = __hip_atomic_fetch_add(cnt + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(nch - 1);
        }
    }
    if (nch == 1) return;
    __syncthreads();
    if (!last || t >= 64) return;
    // wave 0: lane l takes partials l, l + 64, ... of the row
    best = -INFINITY;
    bi = 0x7fffffff;
    for (int k = t; k < nch; k += 64) {
        const float2* p = part + (size_t)r * nch + k;
        argmax_pick(__hip_atomic_load(&p->x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                    __builtin_bit_cast(int, __hip_atomic_load(&p->y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                    best, bi);
    }
    argmax_wave(best, bi);
    if (t == 0) {
        __hip_atomic_store(cnt + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        idx[r] = bi == 0x7fffffff ? 0 : bi;
        val[r] = best;
    }
}

// Packed form of a row's first maximum: the value's bits mapped to an unsigned order (-0 taken as
// +0, so equal values compare equal) in the high word, 0xffffffff - index in the low word.  The
// largest key is the largest value at its lowest index, so one 64-bit atomic max per chunk block
// merges the chunks in any order into the row's first maximum, with no partials, counter or
// combining block.
__device__ __forceinline__ uint64_t argmax_key(float v, int i)
{
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_key_kernel(const float* __restrict__ logits, int n,
                                                                    uint64_t* __restrict__ keys)
{
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const int c = blockIdx.x, r = blockIdx.y;
    float best;
    int bi;
    argmax_chunk(logits + (size_t)r * n, n, c, sv, si, best, bi);
    if (threadIdx.x == 0)
        (void)__hip_atomic_fetch_max(keys + r, argmax_key(best, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_embed_i8(const uint32_t* tokens, int rows, const int8_t* emb, const uint16_t* scale, int vocab,
                           int hidden, float* x, hipStream_t st)
{
    const dim3 grid((unsigned)std::min((hidden + 255) / 256, 64), (unsigned)rows);
    hipLaunchKernelGGL(embed_i8_kernel, grid, dim3(256), 0, st, tokens, emb, scale, vocab, hidden, x);
    return hipGetLastError();
}

hipError_t launch_embed_f16(const uint32_t* tokens, int rows, const uint16_t* emb, int vocab, int hidden, float* x,
                            hipStream_t st)
{
    const dim3 grid((unsigned)std::min((hidden + 255) / 256, 64), (unsigned)rows);
    hipLaunchKernelGGL(embed_f16_kernel, grid, dim3(256), 0, st, tokens, emb, vocab, hidden, x);
    return hipGetLastError();
}

hipError_t launch_embed_i4(const uint32_t* tokens, int rows, const uint8_t* emb, const uint16_t* scale, int vocab,
                           int hidden, float* x, hipStream_t st)
{
    const dim3 grid((unsigned)std::min((hidden + 255) / 256, 64), (unsigned)rows);
    hipLaunchKernelGGL(embed_i4_kernel, grid, dim3(256), 0, st, tokens, emb, scale, vocab, hidden, x);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, const void* w, int wdt, int rows, int n, float eps, float* out,
                           hipStream_t st)
{
    if (wdt == DT_F32)
        hipLaunchKernelGGL((rms_norm_kernel<DT_F32>), dim3(rows), dim3(kNormThreads), 0, st, x, w, out, n, eps);
    else if (wdt == DT_F16)
        hipLaunchKernelGGL((rms_norm_kernel<DT_F16>), dim3(rows), dim3(kNormThreads), 0, st, x, w, out, n, eps);
    else
        hipLaunchKernelGGL((rms_norm_kernel<DT_BF16>), dim3(rows), dim3(kNormThreads), 0, st, x, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_add_rms_norm(float* x, const float* y, const void* w, int wdt, int rows, int n, float eps,
                               float* out, hipStream_t st)
{
    if (wdt == DT_F32)
        hipLaunchKernelGGL((add_rms_norm_kernel<DT_F32>), dim3(rows), dim3(kNormThreads), 0, st, x, y, w, out, n, eps);
    else if (wdt == DT_F16)
        hipLaunchKernelGGL((add_rms_norm_kernel<DT_F16>), dim3(rows), dim3(kNormThreads), 0, st, x, y, w, out, n, eps);
    else
        hipLaunchKernelGGL((add_rms_norm_kernel<DT_BF16>), dim3(rows), dim3(kNormThreads), 0, st, x, y, w, out, n,
                           eps);
    return hipGetLastError();
}

hipError_t launch_rope_kv_write_f16(float* q, float* k, const float* v, int rows, int n_heads, int n_kv_heads,
                                    int head_dim, const int32_t* pos, const float* cos_sin, int table_positions,
                                    uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int max_blocks,
                                    int total_blocks, int n_layers, int tokens_per_block, int layer, int interleaved, hipStream_t st)
{
    const PagedKv kv{block_tables, max_blocks, total_blocks, n_layers, tokens_per_block, n_kv_heads * head_dim};
    const int total = rows * (n_heads + n_kv_heads) * (head_dim / 2);
    const int blocks = std::max(1, std::min((total + 255) / 256, 1024));
    hipLaunchKernelGGL(rope_kv_write_kernel, dim3(blocks), dim3(256), 0, st, q, k, v, rows, n_heads, n_kv_heads,
                       head_dim, pos, reinterpret_cast<const float2*>(cos_sin), table_positions, kcache, vcache, kv,
                       layer, interleaved ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_rope_half(float* x, int rows, int n_heads, int head_dim, const int32_t* pos, const float* cos_sin,
                            int table_positions, int interleaved, hipStream_t st)
{
    const int total = rows * n_heads * (head_dim / 2);
    const int blocks = std::max(1, std::min((total + 255) / 256, 1024));
    hipLaunchKernelGGL(rope_half_kernel, dim3(blocks), dim3(256), 0, st, x, rows, n_heads, head_dim, pos,
                       reinterpret_cast<const float2*>(cos_sin), table_positions, interleaved ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_kv_write_f16(const float* k, const float* v, int rows, int kv_dim, const int32_t* pos,
                               uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int max_blocks,
                               int total_blocks, int n_layers, int tokens_per_block, int layer, hipStream_t st)
{
    const PagedKv kv{block_tables, max_blocks, total_blocks, n_layers, tokens_per_block, kv_dim};
    const int total = rows * kv_dim;
    const int blocks = std::max(1, std::min((total + 255) / 256, 1024));
    hipLaunchKernelGGL(kv_write_kernel, dim3(blocks), dim3(256), 0, st, k, v, rows, pos, kcache, vcache, kv, layer);
    return hipGetLastError();
}

bool attention_supported(int n_heads, int n_kv_heads, int head_dim, int max_seq)
{
    return n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= kAttnGMax &&
           (head_dim == 64 || head_dim == 128) && max_seq >= 1 && max_seq <= kAttnMaxChunks * kAttnChunk;
}

size_t attention_workspace_bytes(int rows, int n_heads, int n_kv_heads, int head_dim, int max_seq)
{
    const int nch = (max_seq + kAttnChunk - 1) / kAttnChunk;
    return kAttnCounterBytes + (size_t)rows * n_heads * nch * (head_dim + 2) * sizeof(float);
}

size_t attention_counter_bytes() { return kAttnCounterBytes; }

hipError_t launch_attention_gqa_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                                      const uint32_t* block_tables, int max_blocks, int total_blocks,
                                      const int32_t* pos, int rows, int n_heads, int n_kv_heads, int head_dim,
                                      int n_layers, int tokens_per_block, int layer, float attn_scale,
                                      float soft_cap, float* out, float* workspace, hipStream_t st, int window)
{
    const PagedKv kv{block_tables, max_blocks, total_blocks, n_layers, tokens_per_block, n_kv_heads * head_dim};
    const int nch = (max_blocks * tokens_per_block + kAttnChunk - 1) / kAttnChunk;
    if (nch > kAttnMaxChunks) return hipErrorInvalidValue;
    // attn_scale None = 1 / sqrt(head_dim) in f32, as kvcache.rs:752 computes it
    const float scale = attn_scale > 0.0f ? attn_scale : 1.0f / std::sqrt((float)head_dim);
    const dim3 pgrid((unsigned)(rows * n_kv_heads), (unsigned)nch);
    const dim3 cgrid((unsigned)(rows * n_kv_heads));
    const int G = n_heads / n_kv_heads;
    // workspace: the group counters (zero between calls), then the partials
    uint32_t* counters = reinterpret_cast<uint32_t*>(workspace);
    float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + kAttnCounterBytes);
    const bool one_launch = rows * n_kv_heads <= kAttnCounters;
    const int cap = max_blocks * tokens_per_block;
    const dim3 hgrid((unsigned)(rows * n_heads));
    auto go = [&](auto hd, auto g) {
        constexpr int HD = decltype(hd)::value, GG = decltype(g)::value;
        // caches of up to 512 positions: the whole sequence in one block per query head
        if (cap <= kAttnBlockSub) {
            hipLaunchKernelGGL((attn_head_kernel<HD, 1>), hgrid, dim3(kAttnBlockThreads), 0, st, q, kcache, vcache,
                               pos, kv, layer, n_heads, GG, scale, soft_cap, window, out);
            return;
        }
        if (cap <= 2 * kAttnBlockSub) {
            hipLaunchKernelGGL((attn_head_kernel<HD, 2>), hgrid, dim3(kAttnBlockThreads), 0, st, q, kcache, vcache,
                               pos, kv, layer, n_heads, GG, scale, soft_cap, window, out);
            return;
        }
        if (one_launch) {
            hipLaunchKernelGGL((attn_partial_kernel<HD, GG, true>), pgrid, dim3(kAttnThreads), 0, st, q, kcache,
                               vcache, pos, kv, layer, n_kv_heads, scale, soft_cap, window, part, nch, counters, out);
            return;
        }
        hipLaunchKernelGGL((attn_partial_kernel<HD, GG>), pgrid, dim3(kAttnThreads), 0, st, q, kcache, vcache, pos, kv,
                           layer, n_kv_heads, scale, soft_cap, window, part, nch, nullptr, nullptr);
        hipLaunchKernelGGL((attn_combine_kernel<HD, GG>), cgrid, dim3(kAttnThreads), 0, st, part, pos, kv,
                           n_kv_heads, nch, window, out);
    };
    auto by_g = [&](auto hd) {
        switch (G) {
        case 1: go(hd, std::integral_constant<int, 1>{}); break;
        case 2: go(hd, std::integral_constant<int, 2>{}); break;
        case 3: go(hd, std::integral_constant<int, 3>{}); break;
        case 4: go(hd, std::integral_constant<int, 4>{}); break;
        case 5: go(hd, std::integral_constant<int, 5>{}); break;
        case 6: go(hd, std::integral_constant<int, 6>{}); break;
        case 7: go(hd, std::integral_constant<int, 7>{}); break;
        default: go(hd, std::integral_constant<int, 8>{}); break;
        }
    };
    if (head_dim == 64)
        by_g(std::integral_constant<int, 64>{});
    else
        by_g(std::integral_constant<int, 128>{});
    return hipGetLastError();
}

// ---- allocation-free attention scratch ---------------------------------------
// The softmax partials of the split-sequence attention, for callers that cannot
// allocate (HIP graph capture, serving loops): a fixed device array that every
// GPU the library runs on holds until the process ends.  Host code never uses
// the array's name as an address (in host code it is a stand-in, not device
// memory): the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) float scratch[kAttnStaticScratchBytes / sizeof(float)];

hipError_t attention_static_scratch(float** out)
{
    static std::mutex mu;
    static std::vector<std::pair<int, float*>> per_device;  // (device, address of its copy)
    *out = nullptr;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const std::lock_guard<std::mutex> lk(mu);
    for (const auto& d : per_device)
        if (d.first == dev) {
            *out = d.second;
            return hipSuccess;
        }
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    // the group counters at its start must read zero before the first call (the calls keep them so)
    if (hipError_t e = hipMemset(p, 0, kAttnCounterBytes); e != hipSuccess) return e;
    per_device.emplace_back(dev, static_cast<float*>(p));
    *out = static_cast<float*>(p);
    return hipSuccess;
}

// Host-side geometry of the fused decode GEMVs (launch_decode): LPR lanes per
// row pair, 64 for rows of more than 16 chunks of 16 bytes, 16 otherwise; C
// chunks per lane; KR registers per thread of the staged row; MT activation rows.
bool decode_fused_supported(int rows, int H)
{
    return rows >= 1 && rows <= 4 && H >= 16 && H % 16 == 0 && H <= 4 * 4 * kNormThreads;
}

size_t decode_fused_lds_bytes(int rows, int H)
{
    const int MT = rows <= 1 ? 1 : (rows <= 2 ? 2 : 4);
    return (size_t)MT * xpad(H) * sizeof(float);
}

namespace {

// Units (a QKV row, or a gate row with its up row) per 64-lane team.  Measured on the configs[4]
// step at 4 sessions (one box, graph replay): gate/up with 1 / 2 / 4 / 8 units 0.882 / 0.854 /
// 0.835 / 0.893 ms; QKV with 2 units 0.879 against 0.854 with 1.
#ifndef CELLM_DI8_RP_QKV
#define CELLM_DI8_RP_QKV 1
#endif
#ifndef CELLM_DI8_RP_GU
#define CELLM_DI8_RP_GU 4
#endif

template <int LPR, int C, int MT, int KR, class Args>
hipError_t launch_decode_fixed(const Args& a, size_t lds, hipStream_t st)
{
    constexpr bool QKV = std::is_same<Args, DecodeQkvArgs>::value;
    constexpr int RPW = QKV ? CELLM_DI8_RP_QKV : CELLM_DI8_RP_GU;  // units per team wanted
    constexpr int RP = RPW * 2 * MT <= LPR ? RPW : (LPR / (2 * MT) >= 1 ? LPR / (2 * MT) : 1);
    const int per_block = (256 / LPR) * RP;
    const dim3 grid((unsigned)((i8_units(a) + per_block - 1) / per_block));
    if (a.y)
        hipLaunchKernelGGL((decode_i8_kernel<LPR, C, RP, MT, KR, true, Args>), grid, dim3(256), lds, st, a);
    else
        hipLaunchKernelGGL((decode_i8_kernel<LPR, C, RP, MT, KR, false, Args>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int LPR, int C, int MT, class Args>
hipError_t launch_decode_kr(int H, const Args& a, size_t lds, hipStream_t st)
{
    const int kr = (H / 4 + kNormThreads - 1) / kNormThreads;  // float4 groups per thread
    if (kr <= 1) return launch_decode_fixed<LPR, C, MT, 1>(a, lds, st);
    if (kr <= 2) return launch_decode_fixed<LPR, C, MT, 2>(a, lds, st);
    return launch_decode_fixed<LPR, C, MT, 4>(a, lds, st);
}

template <int LPR, int C, class Args>
hipError_t launch_decode_mt(int rows, int H, const Args& a, hipStream_t st)
{
    const size_t lds = decode_fused_lds_bytes(rows, H);
    if (rows <= 1) return launch_decode_kr<LPR, C, 1>(H, a, lds, st);
    if (rows <= 2) return launch_decode_kr<LPR, C, 2>(H, a, lds, st);
    return launch_decode_kr<LPR, C, 4>(H, a, lds, st);
}

// chunks per row nchunk = H / 16: 16 lanes up to 16 chunks, else 64 lanes with C = ceil(nchunk / 64)
// (up to 4).  At hidden 960 (60 chunks) 64 lanes of one chunk each beat 32 lanes of two by ~1 % of
// the configs[4] step: twice the waves, each with half the dot work after its loads land.
template <class Args>
hipError_t launch_decode(int rows, int H, const Args& a, hipStream_t st)
{
    const int nchunk = H >> 4;
    if (nchunk <= 16) return launch_decode_mt<16, 1>(rows, H, a, st);
    if (nchunk <= 64) return launch_decode_mt<64, 1>(rows, H, a, st);
    if (nchunk <= 128) return launch_decode_mt<64, 2>(rows, H, a, st);
    return launch_decode_mt<64, 4>(rows, H, a, st);
}

}  // namespace

hipError_t launch_decode_qkv(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                             const int8_t* const w[3], const uint16_t* const s[3], int rows, int H, int n_heads,
                             int n_kv_heads, int head_dim, const int32_t* pos, const float* cos_sin,
                             int table_positions, float* q_out, uint16_t* kcache, uint16_t* vcache,
                             const uint32_t* block_tables, int max_blocks, int total_blocks, int n_layers,
                             int tokens_per_block, int layer, int interleaved, hipStream_t st)
{
    DecodeQkvArgs a{};
    a.x_prev = x_prev;
    a.y = y;
    a.x_out = x_out;
    a.norm_w = norm_w;
    a.eps = eps;
    for (int j = 0; j < 3; ++j) {
        a.w[j] = w[j];
        a.s[j] = s[j];
    }
    a.rows = rows;
    a.H = H;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.pos = pos;
    a.cs = reinterpret_cast<const float2*>(cos_sin);
    a.table_positions = table_positions;
    a.q_out = q_out;
    a.kc = kcache;
    a.vc = vcache;
    a.kv = PagedKv{block_tables, max_blocks, total_blocks, n_layers, tokens_per_block, n_kv_heads * head_dim};
    a.layer = layer;
    a.il = interleaved ? 1 : 0;
    if (H > 64 * 16 * 4) return hipErrorInvalidValue;
    return launch_decode(rows, H, a, st);
}

hipError_t launch_decode_gate_up(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                 const int8_t* wg, const uint16_t* sg, const int8_t* wu, const uint16_t* su, int rows,
                                 int H, int N, float* h, hipStream_t st)
{
    DecodeGateUpArgs a{x_prev, y, x_out, norm_w, eps, wg, sg, wu, su, rows, H, N, h};
    if (H > 64 * 16 * 4) return hipErrorInvalidValue;
    return launch_decode(rows, H, a, st);
}

bool decode_q4_fused_supported(int rows, int H, int group)
{
    return rows >= 1 && rows <= 4 && H >= 32 && H % 32 == 0 && H <= 4096 && group >= 32 && group <= H &&
           (group & (group - 1)) == 0;
}

namespace {

size_t decode_q4_lds_bytes(int MT, int H) { return (size_t)MT * (xpad(H) + (H >> 5)) * sizeof(float); }

// q4 gate/up: 2 units per team (4 and 8 measured 0.786-0.790 against 0.764-0.767 ms on the
// Qwen2-shape step at 4 sessions)
#ifndef CELLM_DQ4_RP_QKV
#define CELLM_DQ4_RP_QKV 1
#endif
#ifndef CELLM_DQ4_RP_GU
#define CELLM_DQ4_RP_GU 2
#endif

template <int LPR, int C, int MT, int KR, class Args>
hipError_t launch_decode_q4_fixed(const Args& a, hipStream_t st)
{
    constexpr bool QKV = std::is_same<Args, DecodeQ4QkvArgs>::value;
    constexpr int RPW = QKV ? CELLM_DQ4_RP_QKV : CELLM_DQ4_RP_GU;  // units per team wanted
    constexpr int RP = RPW * 2 * MT <= LPR ? RPW : (LPR / (2 * MT) >= 1 ? LPR / (2 * MT) : 1);
    const int per_block = (256 / LPR) * RP;
    const dim3 grid((unsigned)((q4_units(a) + per_block - 1) / per_block));
    const size_t lds = decode_q4_lds_bytes(MT, a.H);
    if (a.y)
        hipLaunchKernelGGL((decode_q4_kernel<LPR, C, RP, MT, KR, true, Args>), grid, dim3(256), lds, st, a);
    else
        hipLaunchKernelGGL((decode_q4_kernel<LPR, C, RP, MT, KR, false, Args>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int LPR, int C, int KR, class Args>
hipError_t launch_decode_q4_mt(const Args& a, hipStream_t st)
{
    if (a.rows <= 1) return launch_decode_q4_fixed<LPR, C, 1, KR>(a, st);
    if (a.rows <= 2) return launch_decode_q4_fixed<LPR, C, 2, KR>(a, st);
    return launch_decode_q4_fixed<LPR, C, 4, KR>(a, st);
}

// chunks per row cpr = H / 32, one chunk per lane up to 64 (teams of 16, 32 or 64 lanes), two up to 128;
// KR float4 groups per thread in the prologue (KR * 1024 >= H follows from the same bounds)
template <class Args>
hipError_t launch_decode_q4(const Args& a, hipStream_t st)
{
    const int cpr = a.H >> 5;
    if (cpr <= 16) return launch_decode_q4_mt<16, 1, 1>(a, st);
    if (cpr <= 32) return launch_decode_q4_mt<32, 1, 1>(a, st);
    if (cpr <= 64) return launch_decode_q4_mt<64, 1, 2>(a, st);
    return launch_decode_q4_mt<64, 2, 4>(a, st);
}

int log2_exact(int v)
{
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

}  // namespace

hipError_t launch_decode_q4_qkv(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                const uint32_t* const w[3], const float* const s[3], const float* const b[3],
                                const float* const bias[3], int group, int rows, int H, int n_heads, int n_kv_heads,
                                int head_dim, const int32_t* pos, const float* cos_sin, int table_positions,
                                float* q_out, uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables,
                                int max_blocks, int total_blocks, int n_layers, int tokens_per_block, int layer,
                                int interleaved, hipStream_t st)
{
    if (!decode_q4_fused_supported(rows, H, group)) return hipErrorInvalidValue;
    DecodeQ4QkvArgs a{};
    a.x_prev = x_prev;
    a.y = y;
    a.x_out = x_out;
    a.norm_w = norm_w;
    a.eps = eps;
    for (int j = 0; j < 3; ++j) {
        a.w[j] = reinterpret_cast<const u4_t*>(w[j]);
        a.s[j] = s[j];
        a.b[j] = b[j];
        a.bias[j] = bias[j];
    }
    a.rows = rows;
    a.H = H;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.gshift = log2_exact(group);
    a.pos = pos;
    a.cs = reinterpret_cast<const float2*>(cos_sin);
    a.table_positions = table_positions;
    a.q_out = q_out;
    a.kc = kcache;
    a.vc = vcache;
    a.kv = PagedKv{block_tables, max_blocks, total_blocks, n_layers, tokens_per_block, n_kv_heads * head_dim};
    a.layer = layer;
    a.il = interleaved ? 1 : 0;
    return launch_decode_q4(a, st);
}

hipError_t launch_decode_q4_gate_up(const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
                                    const uint32_t* wg, const float* sg, const float* bg, const uint32_t* wu,
                                    const float* su, const float* bu, int group, int rows, int H, int N, int act,
                                    float* h, hipStream_t st)
{
    if (!decode_q4_fused_supported(rows, H, group)) return hipErrorInvalidValue;
    DecodeQ4GateUpArgs a{x_prev, y, x_out, norm_w, eps, reinterpret_cast<const u4_t*>(wg), sg, bg,
                         reinterpret_cast<const u4_t*>(wu), su, bu, rows, H, N, log2_exact(group), act, h};
    return launch_decode_q4(a, st);
}

// Rows of up to 2048 (64 chunks): one team per row.  Longer rows go to qgemv_q4_x32s_kernel, which
// splits each row over three waves (measured on MI355X, 4864 -> 896 at M = 1 / 2 / 4: 3.9 / 4.3 / 6.2 us
// there, 4.6 / 6.8 / 10.0 us here and 4.7 / 6.5 / 9.3 us on the hi + lo f16 kernels); 896 -> 896 here:
// 2.95 / 3.17 / 4.62 us against 3.25 / 4.07 / 4.59 us on the hi + lo f16 kernels.
bool qgemv_q4_x32_supported(int M, int N, int K, int group)
{
    return M >= 1 && M <= 4 && N >= 1 && K >= 32 && K % 32 == 0 && group >= 32 && group <= K &&
           (group & (group - 1)) == 0 && (size_t)4 * (xpad(K) + (K >> 5)) * sizeof(float) <= 160 * 1024 &&
           K <= 2048;
}

namespace {

template <int LPR, int C, int R, int MT>
hipError_t launch_q4_x32_fixed(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                               int N, int K, int gshift, hipStream_t st)
{
    const int rows_per_block = (256 / LPR) * R;
    const dim3 grid((unsigned)((N + rows_per_block - 1) / rows_per_block));
    const size_t lds = (size_t)MT * (xpad(K) + (K >> 5)) * sizeof(float);
    const int groups = MT * (K >> 2);
    if (groups <= 2 * kNormThreads)
        hipLaunchKernelGGL((qgemv_q4_x32_kernel<LPR, C, R, MT, 2>), grid, dim3(256), lds, st,
                           reinterpret_cast<const u4_t*>(wq), S, B, x, y, M, N, K, gshift);
    else
        hipLaunchKernelGGL((qgemv_q4_x32_kernel<LPR, C, R, MT, 8>), grid, dim3(256), lds, st,
                           reinterpret_cast<const u4_t*>(wq), S, B, x, y, M, N, K, gshift);
    return hipGetLastError();
}

template <int LPR, int C, int R>
hipError_t launch_q4_x32_mt(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                            int N, int K, int gshift, hipStream_t st)
{
    if (M <= 1) return launch_q4_x32_fixed<LPR, C, R, 1>(wq, S, B, x, y, M, N, K, gshift, st);
    if (M <= 2) return launch_q4_x32_fixed<LPR, C, R, 2>(wq, S, B, x, y, M, N, K, gshift, st);
    return launch_q4_x32_fixed<LPR, C, R, 4>(wq, S, B, x, y, M, N, K, gshift, st);
}

}  // namespace

namespace {

template <int KS, int RB, int MT>
hipError_t launch_q4_x32s_fixed(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                                int N, int K, int gshift, hipStream_t st)
{
    constexpr int NT = KS * RB * 64;
    const dim3 grid((unsigned)((N + RB - 1) / RB));
    const size_t lds = (size_t)MT * (xpad(K) + (K >> 5)) * sizeof(float);
    const auto* w4 = reinterpret_cast<const u4_t*>(wq);
    const int rounds = (MT * (K >> 2) + NT - 1) / NT;  // float4 loads per thread
    if (rounds <= 4)
        hipLaunchKernelGGL((qgemv_q4_x32s_kernel<KS, RB, MT, 4>), grid, dim3(NT), lds, st, w4, S, B, x, y, M, N, K,
                           gshift);
    else
        hipLaunchKernelGGL((qgemv_q4_x32s_kernel<KS, RB, MT, 8>), grid, dim3(NT), lds, st, w4, S, B, x, y, M, N, K,
                           gshift);
    return hipGetLastError();
}

template <int KS, int RB>
hipError_t launch_q4_x32s_mt(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                             int N, int K, int gshift, hipStream_t st)
{
    if (M <= 1) return launch_q4_x32s_fixed<KS, RB, 1>(wq, S, B, x, y, M, N, K, gshift, st);
    if (M <= 2) return launch_q4_x32s_fixed<KS, RB, 2>(wq, S, B, x, y, M, N, K, gshift, st);
    return launch_q4_x32s_fixed<KS, RB, 4>(wq, S, B, x, y, M, N, K, gshift, st);
}

}  // namespace

// Waves per row and rows per block of qgemv_q4_x32s_kernel.  4864 -> 896 at 4 rows on MI355X:
// 3 x 4 (768 threads) 6.2 us, 4 x 4 7.2 us, 4 x 2 and 3 x 2 12.7-12.9 us; the hi + lo f16 kernel 9.3 us.
#ifndef CELLM_X32S_KS
#define CELLM_X32S_KS 3
#endif
#ifndef CELLM_X32S_RB
#define CELLM_X32S_RB 4
#endif
bool qgemv_q4_x32s_supported(int M, int N, int K, int group)
{
    const int cpr = K >> 5;
    return M >= 1 && M <= 4 && N >= 1 && K > 2048 && K >= 32 && K % 32 == 0 && group >= 32 && group <= K &&
           (group & (group - 1)) == 0 && (size_t)4 * (xpad(K) + (K >> 5)) * sizeof(float) <= 160 * 1024 &&
           (cpr + CELLM_X32S_KS - 1) / CELLM_X32S_KS <= 64;
}

hipError_t launch_qgemv_q4_x32s(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                                int N, int K, int group, hipStream_t st)
{
    if (!qgemv_q4_x32s_supported(M, N, K, group)) return hipErrorInvalidValue;
    return launch_q4_x32s_mt<CELLM_X32S_KS, CELLM_X32S_RB>(wq, S, B, x, y, M, N, K, log2_exact(group), st);
}

hipError_t launch_qgemv_q4_x32(const uint32_t* wq, const float* S, const float* B, const float* x, float* y, int M,
                               int N, int K, int group, hipStream_t st)
{
    if (!qgemv_q4_x32_supported(M, N, K, group)) return hipErrorInvalidValue;
    const int cpr = K >> 5, gshift = log2_exact(group);
    constexpr int R = 1;  // one row per team: at K <= 1536 faster than two or four (more blocks)
    if (cpr <= 16) return launch_q4_x32_mt<16, 1, R>(wq, S, B, x, y, M, N, K, gshift, st);
    if (cpr <= 32) return launch_q4_x32_mt<32, 1, R>(wq, S, B, x, y, M, N, K, gshift, st);
    return launch_q4_x32_mt<64, 1, R>(wq, S, B, x, y, M, N, K, gshift, st);  // K <= 2048: 64 chunks
}

int argmax_chunks(int n) { return std::max(1, (n + kArgmaxChunk - 1) / kArgmaxChunk); }

size_t argmax_counter_bytes(int rows) { return (((size_t)rows * sizeof(uint32_t)) + 255) & ~(size_t)255; }

size_t argmax_scratch_bytes(int rows, int n)
{
    const int nch = argmax_chunks(n);
    return nch == 1 ? 0 : argmax_counter_bytes(rows) + (size_t)rows * nch * sizeof(float2);
}

hipError_t launch_argmax_keys(const float* logits, int rows, int n, uint64_t* keys, hipStream_t st)
{
    hipLaunchKernelGGL(argmax_key_kernel, dim3(argmax_chunks(n), rows), dim3(kArgmaxThreads), 0, st, logits, n, keys);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int rows, int n, int32_t* idx, float* val, void* scratch, hipStream_t st)
{
    const int nch = argmax_chunks(n);
    if (nch > 1 && !scratch) return hipErrorInvalidValue;
    uint32_t* cnt = reinterpret_cast<uint32_t*>(scratch);
    float2* part = nch > 1 ? reinterpret_cast<float2*>(reinterpret_cast<unsigned char*>(scratch) +
                                                        argmax_counter_bytes(rows))
                           : nullptr;
    hipLaunchKernelGGL(argmax_kernel, dim3(nch, rows), dim3(kArgmaxThreads), 0, st, logits, n, idx, val, cnt, part);
    return hipGetLastError();
}

}  // namespace cellm
