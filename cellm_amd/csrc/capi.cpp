// C ABI of libcellm_hip.so (declarations and contracts in include/cellm_hip.h).
//
// Host-side structure mirrors MetalOps (crates/cellm-kernels/src/metal.rs:637-1267):
// a context owns the device, a stream, a name-keyed weight cache and scratch
// buffers grown on demand (ensure_buf_f32, metal.rs:1247-1253), all behind one
// mutex; kernels are launched asynchronously, and the sync logits_* wrappers
// copy x in, launch, and copy y back.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cellm_hip.h"
#include "api_guard.hpp"
#include "common.hpp"
#include "kernels.hpp"

using namespace cellm;

namespace {

// The calling thread's last error (cellm.h:24-26 documents the reference's as
// thread-local).  A fixed buffer: recording an error never allocates.
thread_local ErrorSlot g_last_error = {};

void store_error(const char* msg, size_t len) { g_last_error.store(msg, len); }

}  // namespace

namespace cellm {
// Lets the other translation units of the library (cellm_file.cpp,
// llama_device.cpp) report through cellm_hip_last_error_message.
int32_t set_error_external(int32_t code, const std::string& msg)
{
    store_error(msg.data(), msg.size());
    return code;
}

// The CELLM_API_END report of this library: records "internal error: <what>"
// without allocating.
int32_t report_exception(int32_t code, const char* what)
{
    char buf[sizeof(g_last_error.msg)];
    const int n = snprintf(buf, sizeof(buf), "internal error: %s", what ? what : "");
    store_error(buf, n < 0 ? 0 : std::min((size_t)n, sizeof(buf) - 1));
    return code;
}
}  // namespace cellm

namespace {

int32_t set_error(int32_t code, const char* fmt, ...)
{
    char buf[sizeof(g_last_error.msg)];
    va_list ap;
    va_start(ap, fmt);
    int n = vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    store_error(buf, n < 0 ? 0 : std::min((size_t)n, sizeof(buf) - 1));
    return code;
}

int32_t hip_error(hipError_t e, const char* what)
{
    if (e == hipErrorOutOfMemory) return set_error(CELLM_HIP_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    return set_error(CELLM_HIP_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                     \
    do {                                        \
        hipError_t e_ = (expr);                 \
        if (e_ != hipSuccess) return hip_error(e_, what); \
    } while (0)

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

bool valid_dtype(int32_t d) { return d == DT_F32 || d == DT_F16 || d == DT_BF16; }
size_t dtype_size(int32_t d) { return d == DT_F32 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

struct cellm_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    std::unordered_map<std::string, DeviceBuffer> weights;
    size_t weight_bytes = 0;
    DeviceBuffer x_buf, y_buf;
    std::unordered_map<hipStream_t, DeviceBuffer> workspaces;  // split-K partials, one per stream
    std::unordered_map<hipStream_t, DeviceBuffer> aux;         // unfused gate/up: the up rows, one per stream
    std::unordered_map<hipStream_t, DeviceBuffer> attn;        // split-sequence attention partials, one per stream
    std::unordered_map<hipStream_t, DeviceBuffer> argmax;      // argmax row counters + chunk partials, one per stream
    float* attn_static = nullptr;  // this device's static attention scratch (cellm_hip_attention_gqa_f16kv_noalloc)
    std::atomic<int> rope_interleaved{0};  // RoPE pairs of the fused decode ops (cellm_hip_set_rope_interleaved)
};

namespace {

// Grow `b` to at least `bytes` (contents not preserved).
int32_t ensure_buffer(DeviceBuffer& b, size_t bytes)
{
    if (b.bytes >= bytes) return CELLM_HIP_OK;
    if (b.ptr) {
        hipError_t e = hipFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
        if (e != hipSuccess) return hip_error(e, "hipFree(scratch)");
    }
    HIP_TRY(hipMalloc(&b.ptr, bytes), "hipMalloc(scratch)");
    b.bytes = bytes;
    return CELLM_HIP_OK;
}

// RAII: make ctx->device current for the duration of a call, restore after.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev)
    {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard()
    {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Async entry points take the caller's stream as is: NULL is HIP's default
// (null) stream, as in the HIP API.  The context's own stream is only used by
// the sync logits_* wrappers (and is available via cellm_hip_get_stream).
hipStream_t pick_stream(cellm_hip_ctx* /*ctx*/, void* stream) { return reinterpret_cast<hipStream_t>(stream); }

int32_t check_ctx(cellm_hip_ctx* ctx)
{
    if (!ctx) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null context");
    return CELLM_HIP_OK;
}

int32_t check_dims(int64_t m, int64_t n, int64_t k)
{
    if (m < 0 || n < 0 || k < 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "negative dimension m=%lld n=%lld k=%lld",
                                                  (long long)m, (long long)n, (long long)k);
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX || m * k > (int64_t)1 << 40 || n * k > (int64_t)1 << 40)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "dimension too large m=%lld n=%lld k=%lld", (long long)m,
                         (long long)n, (long long)k);
    return CELLM_HIP_OK;
}

int32_t check_group(int64_t group)
{
    if (group < 8 || group > (1 << 20) || (group & (group - 1)) != 0)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "group size %lld must be a power of two >= 8", (long long)group);
    return CELLM_HIP_OK;
}

// int8 scale counts: one per tensor, or one per output row (the reference's
// per_channel = "the scale buffer covers every row", metal.rs:900,938-941).
// Counts in between would silently use scale[0] there and are refused here.
int32_t check_n_scales(int64_t n_scales, int64_t n, const char* what)
{
    if (n_scales == 1 || n_scales >= n) return CELLM_HIP_OK;
    return set_error(CELLM_HIP_ERR_INVALID_ARG, "n_scales=%lld%s must be 1 (per tensor) or >= n=%lld (per row)",
                     (long long)n_scales, what, (long long)n);
}

// Per-stream scratch (split-K partials, unfused gate/up rows, attention
// partials), grown on demand.  The caller holds ctx->mu from this call until
// every kernel that uses the buffer is enqueued: calls on one stream then
// queue their scratch users back to back, and a grow (which waits for the
// stream, then frees) cannot happen between a get and its launches.
// zero_prefix: bytes at the start of a freshly allocated buffer that are cleared
// on this stream before first use (the attention's group counters, which its
// kernels then return to zero themselves).
int32_t get_stream_buffer(cellm_hip_ctx* ctx, std::unordered_map<hipStream_t, DeviceBuffer>& map, hipStream_t st,
                          size_t need, float** out, size_t zero_prefix = 0)
{
    *out = nullptr;
    if (need == 0) return CELLM_HIP_OK;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    DeviceBuffer& b = map[st];
    const bool grow = b.bytes < need;
    if (grow) {
        // The old buffer may still be read by queued work on this stream.
        HIP_TRY(hipStreamSynchronize(st), "hipStreamSynchronize(workspace grow)");
    }
    int32_t rc = ensure_buffer(b, need);
    if (rc) return rc;
    if (grow && zero_prefix) HIP_TRY(hipMemsetAsync(b.ptr, 0, std::min(zero_prefix, need), st), "hipMemsetAsync(counters)");
    *out = reinterpret_cast<float*>(b.ptr);
    return CELLM_HIP_OK;
}

// Output rows from which the MFMA batched-decode kernel beats the VALU GEMV at
// 2..4 activation rows (measured on MI355X: 1152->13824 q4 at m=4 7.6 vs 10.3 us;
// 960->2560 int8 at m=4 7.2 vs 4.6 us).
constexpr int64_t kMfmaMinRows = 8192;
#ifndef CELLM_I8FX_MIN_M
#define CELLM_I8FX_MIN_M 3
#endif
constexpr int64_t kI8F32xMfmaMinM = CELLM_I8FX_MIN_M;  // rows from which the int8 f32-x MFMA path runs
// Output rows from which the f32-x q4 GEMV runs on MFMA (the VALU kernels do the dot twice,
// once per f16 part of x; the MFMA form reads each weight once and is HBM-bound).
constexpr int64_t kF32xMfmaMinRows = 32768;

int32_t get_workspace(cellm_hip_ctx* ctx, hipStream_t st, size_t need, float** out)
{
    return get_stream_buffer(ctx, ctx->workspaces, st, need, out);
}

int32_t qgemv_i8_impl(cellm_hip_ctx* ctx, const int8_t* w, const void* scales, int32_t sdt, int64_t n_scales,
                      const void* x, int32_t xdt, const float* bias, float* y, int64_t m, int64_t n, int64_t k,
                      hipStream_t st, bool force_gemm)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (!valid_dtype(sdt) || !valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if (!w && k > 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null weight pointer");
    if (!scales || !y || (!x && k > 0)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null scale/x/y pointer");
    if (int32_t rc = check_n_scales(n_scales, n, "")) return rc;
    const int per_channel = n_scales >= n ? 1 : 0;
    const bool gemm_ok = xdt == DT_F16 && k > 0 && (k % 64) == 0 && aligned16(w) && aligned16(x);
    // 2..64 activation rows: weights streamed once into MFMA operands (exact for
    // int8).  At m <= 4 the VALU GEMV wins until there are rows enough to fill
    // the chip with MFMA tiles.
    if (!force_gemm && gemm_ok && (m > 4 || n >= kMfmaMinRows) && qgemv_mfma_supported(1, (int)m, (int)n, (int)k, 0)) {
        float* ws = nullptr;
        const size_t need = qgemv_mfma_workspace_bytes(1, (int)m, (int)n, (int)k);
        if (int32_t rc = get_workspace(ctx, st, need, &ws)) return rc;
        HIP_TRY(launch_qgemv_mfma_i8(w, scales, sdt, per_channel, reinterpret_cast<const _Float16*>(x), bias, y,
                                     (int)m, (int)n, (int)k, ws, need, st),
                "qgemv_mfma_i8 launch");
        return CELLM_HIP_OK;
    }
    if ((force_gemm || m > 4) && gemm_ok) {
        float* ws = nullptr;
        const size_t need = qgemm_workspace_bytes(1, (int)m, (int)n, (int)k, 64, sdt);
        if (int32_t rc = get_workspace(ctx, st, need, &ws)) return rc;
        HIP_TRY(launch_qgemm_i8_ws(w, scales, sdt, per_channel, reinterpret_cast<const _Float16*>(x), bias, y, (int)m,
                                   (int)n, (int)k, ws, st),
                "qgemm_i8 launch");
        return CELLM_HIP_OK;
    }
    if (force_gemm) return set_error(CELLM_HIP_ERR_UNSUPPORTED, "qgemm_i8 needs f16 x, k %% 64 == 0, 16-byte alignment");
    // f32 x over a long output at several rows (the Llama lm_head of a multi-session step,
    // llama.rs:602-643): exact integer sums on int8 MFMA over three x digits per row
    if (xdt == DT_F32 && m >= kI8F32xMfmaMinM && n >= kF32xMfmaMinRows && aligned16(w) && aligned16(x) &&
        qgemv_i8_f32x_mfma_supported((int)m, (int)n, (int)k)) {
        HIP_TRY(launch_qgemv_i8_f32x_mfma(w, scales, sdt, per_channel, bias, static_cast<const float*>(x), y, (int)m,
                                          (int)n, (int)k, st),
                "qgemv_i8_f32x_mfma launch");
        return CELLM_HIP_OK;
    }
    HIP_TRY(launch_qgemv_i8(w, scales, sdt, per_channel, x, xdt, bias, y, (int)m, (int)n, (int)k, st, k == 0),
            "qgemv_i8 launch");
    return CELLM_HIP_OK;
}

// f16 / i2 / q1_0_g128 row GEMVs (lowbit.hip)
int32_t qgemv_lowbit_impl(int fmt, const void* w, const uint16_t* scales_f16, int32_t scale_mode, const void* x,
                          int32_t xdt, float* y, int64_t m, int64_t n, int64_t k, hipStream_t st)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (!valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (fmt == LB_Q1 && k % 128 != 0)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "q1_0_g128 needs k %% 128 == 0 (k=%lld)", (long long)k);
    if (fmt == LB_I2 && scale_mode != 0 && scale_mode != 1)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "i2 scale_mode must be 0 (at the end) or 1 (per element)");
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if ((k > 0 && (!w || !x)) || !y || (fmt == LB_I2 && !scales_f16))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (fmt == LB_F16 && (reinterpret_cast<uintptr_t>(w) & 1))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "f16 weights must be 2-byte aligned");
    if (k == 0) {
        HIP_TRY(launch_fill_f32(y, 0.0f, (size_t)m * n, st), "zero fill of y");
        return CELLM_HIP_OK;
    }
    HIP_TRY(launch_qgemv_lowbit(fmt, w, scales_f16, scale_mode, x, xdt, y, (int)m, (int)n, (int)k, st),
            "qgemv lowbit launch");
    return CELLM_HIP_OK;
}

int32_t qgemv_q4_impl(cellm_hip_ctx* ctx, const uint32_t* wq, const void* scales, const void* biases, int32_t sbt,
                      int64_t group, const void* x, int32_t xdt, float* y, int64_t m, int64_t n, int64_t k,
                      hipStream_t st, bool force_gemm)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (int32_t rc = check_group(group)) return rc;
    if (!valid_dtype(sbt) || !valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (k % 8 != 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "k=%lld must be a multiple of 8 (u32 nibble words)",
                                     (long long)k);
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if (k > 0 && (!wq || !scales || !biases || !x)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null input pointer");
    if (!y) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null output pointer");
    const bool gemm_ok = xdt == DT_F16 && k > 0 && (k % 64) == 0 && group >= 32 && aligned16(wq) && aligned16(x);
    // f32 x over a long output (the affine lm_head, lfm.rs:700-741): exact nibbles on MFMA
    if (!force_gemm && xdt == DT_F32 && n >= kF32xMfmaMinRows && aligned16(wq) && aligned16(x) &&
        qgemv_q4_f32x_mfma_supported((int)m, (int)n, (int)k, (int)group)) {
        HIP_TRY(launch_qgemv_q4_f32x_mfma(wq, scales, biases, sbt, static_cast<const float*>(x), y, (int)m, (int)n,
                                          (int)k, st),
                "qgemv_q4_f32x_mfma launch");
        return CELLM_HIP_OK;
    }
    // f32 x at m <= 4 with f32 scales and biases (the u32 runners' o_proj and down_proj): x copied to
    // LDS as f32 once per block, an f32 dot (the hi + lo f16 kernels stage and dot x twice)
    if (!force_gemm && xdt == DT_F32 && sbt == DT_F32 && aligned16(wq) && aligned16(x) &&
        qgemv_q4_x32_supported((int)m, (int)n, (int)k, (int)group)) {
        HIP_TRY(launch_qgemv_q4_x32(wq, static_cast<const float*>(scales), static_cast<const float*>(biases),
                                    static_cast<const float*>(x), y, (int)m, (int)n, (int)k, (int)group, st),
                "qgemv_q4_x32 launch");
        return CELLM_HIP_OK;
    }
    // the same over rows longer than 2048 (the down projection): each row split over the waves of a block
    if (!force_gemm && xdt == DT_F32 && sbt == DT_F32 && aligned16(wq) && aligned16(x) &&
        qgemv_q4_x32s_supported((int)m, (int)n, (int)k, (int)group)) {
        HIP_TRY(launch_qgemv_q4_x32s(wq, static_cast<const float*>(scales), static_cast<const float*>(biases),
                                     static_cast<const float*>(x), y, (int)m, (int)n, (int)k, (int)group, st),
                "qgemv_q4_x32s launch");
        return CELLM_HIP_OK;
    }
    // 2..64 activation rows: f16 MFMA tiles dequantized in registers; at m <= 4
    // only for long outputs (else the f32-accumulating VALU GEMV is faster)
    if (!force_gemm && (m > 4 || n >= kMfmaMinRows) && gemm_ok &&
        qgemv_mfma_supported(0, (int)m, (int)n, (int)k, (int)group)) {
        float* ws = nullptr;
        const size_t need = qgemv_mfma_workspace_bytes(0, (int)m, (int)n, (int)k);
        if (int32_t rc = get_workspace(ctx, st, need, &ws)) return rc;
        HIP_TRY(launch_qgemv_mfma_q4(wq, scales, biases, sbt, (int)group, reinterpret_cast<const _Float16*>(x), y,
                                     (int)m, (int)n, (int)k, ws, need, st),
                "qgemv_mfma_q4 launch");
        return CELLM_HIP_OK;
    }
    if ((force_gemm || m > 4) && gemm_ok) {
        float* ws = nullptr;
        const size_t need = qgemm_workspace_bytes(0, (int)m, (int)n, (int)k, (int)group, sbt);
        if (int32_t rc = get_workspace(ctx, st, need, &ws)) return rc;
        HIP_TRY(launch_qgemm_q4_affine_ws(wq, scales, biases, sbt, (int)group, reinterpret_cast<const _Float16*>(x), y,
                                          (int)m, (int)n, (int)k, ws, st),
                "qgemm_q4_affine launch");
        return CELLM_HIP_OK;
    }
    if (force_gemm)
        return set_error(CELLM_HIP_ERR_UNSUPPORTED, "qgemm_q4_affine needs f16 x, k %% 64 == 0, group >= 32, alignment");
    HIP_TRY(launch_qgemv_q4_affine(wq, scales, biases, sbt, (int)group, x, xdt, y, (int)m, (int)n, (int)k, st, k == 0),
            "qgemv_q4_affine launch");
    return CELLM_HIP_OK;
}

// Fused projections (one launch for M <= 4); other shapes run the single-op
// paths, plus the elementwise SiLU * up for gate/up.
int32_t qkv_i8_impl(cellm_hip_ctx* ctx, const int8_t* const w[3], const void* const s[3], const int64_t n_s[3],
                    const float* const b[3], int32_t sdt, const void* x, int32_t xdt, float* const y[3], int64_t m,
                    const int64_t rows[3], int64_t k, hipStream_t st)
{
    for (int i = 0; i < 3; ++i)
        if (int32_t rc = check_dims(m, rows[i], k)) return rc;
    if (!valid_dtype(sdt) || !valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || rows[0] + rows[1] + rows[2] == 0) return CELLM_HIP_OK;
    for (int i = 0; i < 3; ++i) {
        if (rows[i] == 0) continue;
        if ((!w[i] && k > 0) || !s[i] || !y[i] || (!x && k > 0))
            return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer in projection %d", i);
        if (int32_t rc = check_n_scales(n_s[i], rows[i], i == 0 ? " (q)" : i == 1 ? " (k)" : " (v)")) return rc;
    }
    I8FusedSeg segs[3];
    for (int i = 0; i < 3; ++i)
        segs[i] = I8FusedSeg{w[i], s[i], b[i], y[i], (int)rows[i], n_s[i] >= rows[i] ? 1 : 0};
    if (k > 0 && qgemv_i8_fused_supported(xdt, (int)m, (int)k, x, segs, 3)) {
        HIP_TRY(launch_qgemv_i8_fused(segs, 3, false, ACT_SILU, sdt, x, xdt, (int)m, (int)k, st), "qgemv_i8_qkv launch");
        return CELLM_HIP_OK;
    }
    for (int i = 0; i < 3; ++i)
        if (rows[i] > 0)
            if (int32_t rc = qgemv_i8_impl(ctx, w[i], s[i], sdt, n_s[i], x, xdt, b[i], y[i], m, rows[i], k, st, false))
                return rc;
    return CELLM_HIP_OK;
}

int32_t gate_up_i8_impl(cellm_hip_ctx* ctx, const int8_t* wg, const void* sg, int64_t n_sg, const float* bg,
                        const int8_t* wu, const void* su, int64_t n_su, const float* bu, int32_t sdt, const void* x,
                        int32_t xdt, float* h, int64_t m, int64_t n, int64_t k, int act, hipStream_t st)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (!valid_dtype(sdt) || !valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if ((k > 0 && (!wg || !wu || !x)) || !sg || !su || !h) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (int32_t rc = check_n_scales(n_sg, n, " (gate)")) return rc;
    if (int32_t rc = check_n_scales(n_su, n, " (up)")) return rc;
    I8FusedSeg segs[2] = {I8FusedSeg{wg, sg, bg, h, (int)n, n_sg >= n ? 1 : 0},
                          I8FusedSeg{wu, su, bu, nullptr, (int)n, n_su >= n ? 1 : 0}};
    if (k > 0 && qgemv_i8_fused_supported(xdt, (int)m, (int)k, x, segs, 2)) {
        HIP_TRY(launch_qgemv_i8_fused(segs, 2, true, act, sdt, x, xdt, (int)m, (int)k, st), "qgemv_i8 gate/up launch");
        return CELLM_HIP_OK;
    }
    float* up = nullptr;
    if (int32_t rc = get_stream_buffer(ctx, ctx->aux, st, (size_t)m * n * sizeof(float), &up)) return rc;
    if (int32_t rc = qgemv_i8_impl(ctx, wg, sg, sdt, n_sg, x, xdt, bg, h, m, n, k, st, false)) return rc;
    if (int32_t rc = qgemv_i8_impl(ctx, wu, su, sdt, n_su, x, xdt, bu, up, m, n, k, st, false)) return rc;
    HIP_TRY(launch_act_mul(act, h, up, (size_t)m * n, st), "activation * up launch");
    return CELLM_HIP_OK;
}

int32_t gate_up_q4_impl(cellm_hip_ctx* ctx, const uint32_t* wg, const void* sg, const void* bg, const uint32_t* wu,
                        const void* su, const void* bu, int32_t sbt, int64_t group, const void* x, int32_t xdt,
                        float* h, int64_t m, int64_t n, int64_t k, int act, hipStream_t st)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (int32_t rc = check_group(group)) return rc;
    if (!valid_dtype(sbt) || !valid_dtype(xdt)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if (!h) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null output pointer");
    if (k > 0 && (!wg || !sg || !bg || !wu || !su || !bu || !x))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null input pointer");
    if (qgemv_q4_gate_up_supported(xdt, (int)m, (int)k, (int)group, x, wg, wu)) {
        HIP_TRY(launch_qgemv_q4_gate_up_silu(wg, sg, bg, wu, su, bu, sbt, (int)group, x, xdt, h, (int)m, (int)n, (int)k,
                                             act, st),
                "qgemv_q4 gate/up launch");
        return CELLM_HIP_OK;
    }
    float* up = nullptr;
    if (int32_t rc = get_stream_buffer(ctx, ctx->aux, st, (size_t)m * n * sizeof(float), &up)) return rc;
    if (int32_t rc = qgemv_q4_impl(ctx, wg, sg, bg, sbt, group, x, xdt, h, m, n, k, st, false)) return rc;
    if (int32_t rc = qgemv_q4_impl(ctx, wu, su, bu, sbt, group, x, xdt, up, m, n, k, st, false)) return rc;
    HIP_TRY(launch_act_mul(act, h, up, (size_t)m * n, st), "activation * up launch");
    return CELLM_HIP_OK;
}

int32_t upload_locked(cellm_hip_ctx* ctx, const std::string& key, const void* host, size_t nbytes, const void** out)
{
    auto it = ctx->weights.find(key);
    if (it != ctx->weights.end()) {
        if (it->second.bytes != nbytes)
            return set_error(CELLM_HIP_ERR_INVALID_ARG, "weight '%s' cached with %zu bytes, upload has %zu",
                             key.c_str(), it->second.bytes, nbytes);
        *out = it->second.ptr;
        return CELLM_HIP_OK;
    }
    if (!host && nbytes) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null host pointer for '%s'", key.c_str());
    DeviceBuffer b;
    HIP_TRY(hipMalloc(&b.ptr, nbytes ? nbytes : 1), "hipMalloc(weight)");
    b.bytes = nbytes;
    if (nbytes) {
        hipError_t e = hipMemcpyAsync(b.ptr, host, nbytes, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(b.ptr);
            return hip_error(e, "upload weight");
        }
    }
    ctx->weights.emplace(key, b);
    ctx->weight_bytes += nbytes;
    *out = b.ptr;
    return CELLM_HIP_OK;
}

// Shared tail of the logits_* wrappers: x (f32 host) in, launch, y (f32 host) out.
template <typename Launch>
int32_t run_logits(cellm_hip_ctx* ctx, const float* x, size_t cols, size_t rows, float* out, Launch&& launch)
{
    if (int32_t rc = ensure_buffer(ctx->x_buf, (cols ? cols : 1) * sizeof(float))) return rc;
    if (int32_t rc = ensure_buffer(ctx->y_buf, (rows ? rows : 1) * sizeof(float))) return rc;
    if (cols) HIP_TRY(hipMemcpyAsync(ctx->x_buf.ptr, x, cols * sizeof(float), hipMemcpyHostToDevice, ctx->stream), "copy x");
    if (int32_t rc = launch(reinterpret_cast<const float*>(ctx->x_buf.ptr), reinterpret_cast<float*>(ctx->y_buf.ptr)))
        return rc;
    if (rows)
        HIP_TRY(hipMemcpyAsync(out, ctx->y_buf.ptr, rows * sizeof(float), hipMemcpyDeviceToHost, ctx->stream), "copy y");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(logits)");
    return CELLM_HIP_OK;
}

}  // namespace

extern "C" {

size_t cellm_hip_last_error_message(char* buf, size_t buf_len) { return g_last_error.take(buf, buf_len); }

int32_t cellm_hip_device_count(int32_t* out_count)
{
    CELLM_API_BEGIN
    if (!out_count) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null out_count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) n = 0;
    else if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
    *out_count = n;
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_smoke_test(int32_t device)
{
    CELLM_API_BEGIN
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return set_error(CELLM_HIP_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= count) return set_error(CELLM_HIP_ERR_INVALID_ARG, "device %d out of range", device);
    DeviceGuard g(device);
    if (!g.ok) return set_error(CELLM_HIP_ERR_DEVICE, "hipSetDevice(%d) failed", device);
    const int n = 1024;
    std::vector<float> a(n), b(n), c(n, 0.0f);
    for (int i = 0; i < n; ++i) {
        a[i] = (float)i;
        b[i] = (float)(2 * i);
    }
    float *da = nullptr, *db = nullptr, *dc = nullptr;
    int32_t rc = CELLM_HIP_OK;
    if (hipMalloc(&da, n * 4) != hipSuccess || hipMalloc(&db, n * 4) != hipSuccess || hipMalloc(&dc, n * 4) != hipSuccess) {
        rc = set_error(CELLM_HIP_ERR_OUT_OF_MEMORY, "smoke test allocation failed");
    } else if (hipMemcpy(da, a.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess ||
               hipMemcpy(db, b.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess ||
               launch_add_f32(da, db, dc, n, nullptr) != hipSuccess ||
               hipMemcpy(c.data(), dc, n * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        rc = set_error(CELLM_HIP_ERR_DEVICE, "smoke test kernel failed");
    } else {
        for (int i = 0; i < n; ++i)
            if (c[i] != (float)(3 * i)) {
                rc = set_error(CELLM_HIP_ERR_DEVICE, "smoke test mismatch at %d: %f", i, c[i]);
                break;
            }
    }
    if (da) (void)hipFree(da);
    if (db) (void)hipFree(db);
    if (dc) (void)hipFree(dc);
    return rc;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_create(int32_t device, cellm_hip_ctx_t** out_ctx)
{
    CELLM_API_BEGIN
    if (!out_ctx) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null out_ctx");
    *out_ctx = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return set_error(CELLM_HIP_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= count) return set_error(CELLM_HIP_ERR_INVALID_ARG, "device %d out of range", device);
    DeviceGuard g(device);
    if (!g.ok) return set_error(CELLM_HIP_ERR_DEVICE, "hipSetDevice(%d) failed", device);
    auto* ctx = new (std::nothrow) cellm_hip_ctx();
    if (!ctx) return set_error(CELLM_HIP_ERR_OUT_OF_MEMORY, "context allocation failed");
    ctx->device = device;
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_error(e, "hipStreamCreate");
    }
    // The device address of the static attention scratch, with the device current.  Only
    // cellm_hip_attention_gqa_f16kv_noalloc needs it: a failure here leaves it null, and that
    // entry point tries again on its first call and reports the error itself.
    if (attention_static_scratch(&ctx->attn_static) != hipSuccess) {
        ctx->attn_static = nullptr;
        (void)hipGetLastError();
    }
    *out_ctx = ctx;
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

void cellm_hip_destroy(cellm_hip_ctx_t* ctx)
{
    CELLM_API_BEGIN
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto* map : {&ctx->workspaces, &ctx->aux, &ctx->attn, &ctx->argmax})
        for (auto& kv : *map) {
            (void)hipStreamSynchronize(kv.first);
            if (kv.second.ptr) (void)hipFree(kv.second.ptr);
        }
    for (auto& kv : ctx->weights)
        if (kv.second.ptr) (void)hipFree(kv.second.ptr);
    if (ctx->x_buf.ptr) (void)hipFree(ctx->x_buf.ptr);
    if (ctx->y_buf.ptr) (void)hipFree(ctx->y_buf.ptr);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    CELLM_API_END_VOID
}

int32_t cellm_hip_synchronize(cellm_hip_ctx_t* ctx)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_get_stream(cellm_hip_ctx_t* ctx, void** out_stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!out_stream) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null out_stream");
    *out_stream = reinterpret_cast<void*>(ctx->stream);
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_weight_upload(cellm_hip_ctx_t* ctx, const char* key, const void* host, size_t nbytes,
                                const void** out_dev)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!key || !out_dev) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null key or out_dev");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    return upload_locked(ctx, key, host, nbytes, out_dev);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_weight_lookup(cellm_hip_ctx_t* ctx, const char* key, const void** out_dev, size_t* out_nbytes)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!key) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null key");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    auto it = ctx->weights.find(key);
    if (it == ctx->weights.end()) return set_error(CELLM_HIP_ERR_NOT_FOUND, "weight '%s' not cached", key);
    if (out_dev) *out_dev = it->second.ptr;
    if (out_nbytes) *out_nbytes = it->second.bytes;
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_weight_evict(cellm_hip_ctx_t* ctx, const char* key)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!key) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null key");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    auto it = ctx->weights.find(key);
    if (it == ctx->weights.end()) return set_error(CELLM_HIP_ERR_NOT_FOUND, "weight '%s' not cached", key);
    // queued kernels on any stream may still read it
    HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize(evict)");
    HIP_TRY(hipFree(it->second.ptr), "hipFree(weight)");
    ctx->weight_bytes -= it->second.bytes;
    ctx->weights.erase(it);
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_weight_cache_stats(cellm_hip_ctx_t* ctx, size_t* out_entries, size_t* out_bytes)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (out_entries) *out_entries = ctx->weights.size();
    if (out_bytes) *out_bytes = ctx->weight_bytes;
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i8(cellm_hip_ctx_t* ctx, const int8_t* w, const void* scales, int32_t scale_dtype,
                           int64_t n_scales, const void* x, int32_t x_dtype, const float* bias, float* y, int64_t m,
                           int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return qgemv_i8_impl(ctx, w, scales, scale_dtype, n_scales, x, x_dtype, bias, y, m, n, k, pick_stream(ctx, stream),
                         false);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                  int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype, float* y,
                                  int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return qgemv_q4_impl(ctx, wq, scales, biases, sb_dtype, group, x, x_dtype, y, m, n, k, pick_stream(ctx, stream),
                         false);
    CELLM_API_END(report_exception)
}

static int32_t qgemv_i4_impl(const uint8_t* w, const uint16_t* scales_f16, int64_t n_scales, int64_t gs,
                             const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k, hipStream_t st);

int32_t cellm_hip_qgemv_batch(cellm_hip_ctx_t* ctx, const cellm_hip_qgemv_op_t* ops, int64_t n_ops, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (n_ops < 0 || (n_ops > 0 && !ops)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null or negative op list");
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    hipStream_t st = pick_stream(ctx, stream);
    for (int64_t i = 0; i < n_ops; ++i) {
        const cellm_hip_qgemv_op_t& o = ops[i];
        int32_t rc;
        if (o.kind == CELLM_HIP_OP_QGEMV_I8)
            rc = qgemv_i8_impl(ctx, static_cast<const int8_t*>(o.w), o.scales, o.sb_dtype, o.n_scales, o.x, o.x_dtype,
                               o.bias, o.y, o.m, o.n, o.k, st, false);
        else if (o.kind == CELLM_HIP_OP_QGEMV_Q4_AFFINE)
            rc = qgemv_q4_impl(ctx, static_cast<const uint32_t*>(o.w), o.scales, o.biases, o.sb_dtype, o.group, o.x,
                               o.x_dtype, o.y, o.m, o.n, o.k, st, false);
        else if (o.kind == CELLM_HIP_OP_QGEMV_F16)
            rc = qgemv_lowbit_impl(LB_F16, o.w, nullptr, 0, o.x, o.x_dtype, o.y, o.m, o.n, o.k, st);
        else if (o.kind == CELLM_HIP_OP_QGEMV_I2)
            rc = qgemv_lowbit_impl(LB_I2, o.w, static_cast<const uint16_t*>(o.scales), o.group, o.x, o.x_dtype, o.y,
                                   o.m, o.n, o.k, st);
        else if (o.kind == CELLM_HIP_OP_QGEMV_Q1_0_G128)
            rc = qgemv_lowbit_impl(LB_Q1, o.w, nullptr, 0, o.x, o.x_dtype, o.y, o.m, o.n, o.k, st);
        else if (o.kind == CELLM_HIP_OP_QGEMV_I4_SYM)
            rc = qgemv_i4_impl(static_cast<const uint8_t*>(o.w), static_cast<const uint16_t*>(o.scales), o.n_scales,
                               o.group, o.x, o.x_dtype, o.y, o.m, o.n, o.k, st);
        else
            rc = set_error(CELLM_HIP_ERR_INVALID_ARG, "op %lld: unknown kind %d", (long long)i, (int)o.kind);
        if (rc) return rc;
    }
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i8_qkv(cellm_hip_ctx_t* ctx, const int8_t* wq, const void* sq, int64_t n_sq, const float* bq,
                               const int8_t* wk, const void* sk, int64_t n_sk, const float* bk, const int8_t* wv,
                               const void* sv, int64_t n_sv, const float* bv, int32_t scale_dtype, const void* x,
                               int32_t x_dtype, float* q, float* k_out, float* v, int64_t m, int64_t rows_q,
                               int64_t rows_kv, int64_t cols, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    const int8_t* w[3] = {wq, wk, wv};
    const void* s[3] = {sq, sk, sv};
    const int64_t n_s[3] = {n_sq, n_sk, n_sv};
    const float* b[3] = {bq, bk, bv};
    float* y[3] = {q, k_out, v};
    const int64_t rows[3] = {rows_q, rows_kv, rows_kv};
    return qkv_i8_impl(ctx, w, s, n_s, b, scale_dtype, x, x_dtype, y, m, rows, cols, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_q4_affine_qkv(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* sq, const void* bq,
                                      const float* biasq, const uint32_t* wk, const void* sk, const void* bk,
                                      const float* biask, const uint32_t* wv, const void* sv, const void* bv,
                                      const float* biasv, int32_t sb_dtype, int64_t group, const void* x,
                                      int32_t x_dtype, float* q, float* k_out, float* v, int64_t m, int64_t rows_q,
                                      int64_t rows_kv, int64_t cols, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    hipStream_t st = pick_stream(ctx, stream);
    const uint32_t* w[3] = {wq, wk, wv};
    const void* s[3] = {sq, sk, sv};
    const void* b[3] = {bq, bk, bv};
    const float* pb[3] = {biasq, biask, biasv};
    float* y[3] = {q, k_out, v};
    const int64_t rows[3] = {rows_q, rows_kv, rows_kv};
    for (int i = 0; i < 3; ++i)
        if (int32_t rc = check_dims(m, rows[i], cols)) return rc;
    if (int32_t rc = check_group(group)) return rc;
    if (!valid_dtype(sb_dtype) || !valid_dtype(x_dtype)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || rows[0] + rows[1] + rows[2] == 0) return CELLM_HIP_OK;
    for (int i = 0; i < 3; ++i)
        if (rows[i] > 0 && ((cols > 0 && (!w[i] || !s[i] || !b[i] || !x)) || !y[i]))
            return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer in projection %d", i);
    Q4FusedSeg segs[3];
    for (int i = 0; i < 3; ++i) segs[i] = Q4FusedSeg{w[i], s[i], b[i], pb[i], y[i], (int)rows[i]};
    if (cols > 0 && qgemv_q4_segs_supported(x_dtype, (int)m, (int)cols, (int)group, x, segs, 3)) {
        HIP_TRY(launch_qgemv_q4_segs(segs, 3, sb_dtype, (int)group, x, x_dtype, (int)m, (int)cols, st),
                "qgemv_q4_qkv launch");
        return CELLM_HIP_OK;
    }
    // other shapes: one GEMV per projection, then its bias
    for (int i = 0; i < 3; ++i) {
        if (rows[i] == 0) continue;
        if (int32_t rc = qgemv_q4_impl(ctx, w[i], s[i], b[i], sb_dtype, group, x, x_dtype, y[i], m, rows[i], cols, st,
                                       false))
            return rc;
        if (pb[i]) HIP_TRY(launch_add_bias_rows(y[i], pb[i], (int)m, (int)rows[i], st), "add_bias launch");
    }
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i8_gate_up_silu(cellm_hip_ctx_t* ctx, const int8_t* wg, const void* sg, int64_t n_sg,
                                        const float* bg, const int8_t* wu, const void* su, int64_t n_su,
                                        const float* bu, int32_t scale_dtype, const void* x, int32_t x_dtype, float* h,
                                        int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return gate_up_i8_impl(ctx, wg, sg, n_sg, bg, wu, su, n_su, bu, scale_dtype, x, x_dtype, h, m, n, k, ACT_SILU,
                           pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i8_gate_up_gelu(cellm_hip_ctx_t* ctx, const int8_t* wg, const void* sg, int64_t n_sg,
                                        const float* bg, const int8_t* wu, const void* su, int64_t n_su,
                                        const float* bu, int32_t scale_dtype, const void* x, int32_t x_dtype, float* h,
                                        int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return gate_up_i8_impl(ctx, wg, sg, n_sg, bg, wu, su, n_su, bu, scale_dtype, x, x_dtype, h, m, n, k,
                           ACT_GELU_TANH, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_q4_affine_gate_up_silu(cellm_hip_ctx_t* ctx, const uint32_t* wg, const void* sg,
                                               const void* bg, const uint32_t* wu, const void* su, const void* bu,
                                               int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype,
                                               float* h, int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return gate_up_q4_impl(ctx, wg, sg, bg, wu, su, bu, sb_dtype, group, x, x_dtype, h, m, n, k, ACT_SILU,
                           pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_q4_affine_gate_up_gelu(cellm_hip_ctx_t* ctx, const uint32_t* wg, const void* sg,
                                               const void* bg, const uint32_t* wu, const void* su, const void* bu,
                                               int32_t sb_dtype, int64_t group, const void* x, int32_t x_dtype,
                                               float* h, int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return gate_up_q4_impl(ctx, wg, sg, bg, wu, su, bu, sb_dtype, group, x, x_dtype, h, m, n, k, ACT_GELU_TANH,
                           pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

static int32_t qgemv_i4_impl(const uint8_t* w, const uint16_t* scales_f16, int64_t n_scales, int64_t gs,
                             const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k, hipStream_t st)
{
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (!valid_dtype(x_dtype)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if (gs < 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "gs must be >= 1");
    const int64_t spr = n_scales / n;
    if (spr < 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "n_scales=%lld < n=%lld", (long long)n_scales, (long long)n);
    if (k > 0 && (k - 1) / gs >= spr)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "scale index (k-1)/gs=%lld out of range spr=%lld",
                         (long long)((k - 1) / gs), (long long)spr);
    if ((k > 0 && (!w || !scales_f16 || !x)) || !y) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    HIP_TRY(launch_qgemv_i4_sym(w, scales_f16, (int)spr, (int)gs, x, x_dtype, y, (int)m, (int)n, (int)k, st),
            "qgemv_i4_sym launch");
    return CELLM_HIP_OK;
}

// Gemma's MLP over symmetric i4 gate/up weights (gemma.rs:838-846 with the i4 branch of
// linear_f16_out_in, gemma.rs:1446-1471): the two i4 GEMVs, then gelu_tanh(g) * u.
int32_t cellm_hip_qgemv_i4_gate_up_gelu(cellm_hip_ctx_t* ctx, const uint8_t* wg, const uint16_t* sg, int64_t n_sg,
                                        const uint8_t* wu, const uint16_t* su, int64_t n_su, int64_t gs,
                                        const void* x, int32_t x_dtype, float* h, int64_t m, int64_t n, int64_t k,
                                        void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(m, n, k)) return rc;
    if (m == 0 || n == 0) return CELLM_HIP_OK;
    if (!h) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null output pointer");
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    hipStream_t st = pick_stream(ctx, stream);
    float* up = nullptr;
    if (int32_t rc = get_stream_buffer(ctx, ctx->aux, st, (size_t)m * n * sizeof(float), &up)) return rc;
    if (int32_t rc = qgemv_i4_impl(wg, sg, n_sg, gs, x, x_dtype, h, m, n, k, st)) return rc;
    if (int32_t rc = qgemv_i4_impl(wu, su, n_su, gs, x, x_dtype, up, m, n, k, st)) return rc;
    HIP_TRY(launch_act_mul(ACT_GELU_TANH, h, up, (size_t)m * n, st), "gelu_tanh_mul launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i4_sym(cellm_hip_ctx_t* ctx, const uint8_t* w, const uint16_t* scales_f16, int64_t n_scales,
                               int64_t gs, const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k,
                               void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    return qgemv_i4_impl(w, scales_f16, n_scales, gs, x, x_dtype, y, m, n, k, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_f16(cellm_hip_ctx_t* ctx, const uint16_t* w_f16, const void* x, int32_t x_dtype, float* y,
                            int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    return qgemv_lowbit_impl(LB_F16, w_f16, nullptr, 0, x, x_dtype, y, m, n, k, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_i2(cellm_hip_ctx_t* ctx, const uint8_t* w, const uint16_t* scales_f16, int32_t scale_mode,
                           const void* x, int32_t x_dtype, float* y, int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    return qgemv_lowbit_impl(LB_I2, w, scales_f16, scale_mode, x, x_dtype, y, m, n, k, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemv_q1_0_g128(cellm_hip_ctx_t* ctx, const uint8_t* w, const void* x, int32_t x_dtype, float* y,
                                  int64_t m, int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    return qgemv_lowbit_impl(LB_Q1, w, nullptr, 0, x, x_dtype, y, m, n, k, pick_stream(ctx, stream));
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemm_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                  int32_t sb_dtype, int64_t group, const uint16_t* x_f16, float* y, int64_t m,
                                  int64_t n, int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return qgemv_q4_impl(ctx, wq, scales, biases, sb_dtype, group, x_f16, DT_F16, y, m, n, k, pick_stream(ctx, stream),
                         true);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_qgemm_i8(cellm_hip_ctx_t* ctx, const int8_t* w, const void* scales, int32_t scale_dtype,
                           int64_t n_scales, const uint16_t* x_f16, const float* bias, float* y, int64_t m, int64_t n,
                           int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return qgemv_i8_impl(ctx, w, scales, scale_dtype, n_scales, x_f16, DT_F16, bias, y, m, n, k,
                         pick_stream(ctx, stream), true);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_dequant_q4_affine(cellm_hip_ctx_t* ctx, const uint32_t* wq, const void* scales, const void* biases,
                                    int32_t sb_dtype, int64_t group, void* out, int32_t out_dtype, int64_t n,
                                    int64_t k, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(1, n, k)) return rc;
    if (int32_t rc = check_group(group)) return rc;
    if (!valid_dtype(sb_dtype) || (out_dtype != DT_F32 && out_dtype != DT_F16))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (k % 8 != 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "k must be a multiple of 8");
    if (n == 0 || k == 0) return CELLM_HIP_OK;
    if (!wq || !scales || !biases || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (!aligned16(out)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "output must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_dequant_q4_affine(wq, scales, biases, sb_dtype, (int)group, out, out_dtype, (int)n, (int)k,
                                     pick_stream(ctx, stream)),
            "dequant launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_logits_i8(cellm_hip_ctx_t* ctx, const float* x, const int8_t* w, const uint16_t* scales_f16,
                            size_t rows, size_t cols, const char* cache_key, float* out)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!cache_key || (!x && cols) || (!out && rows)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    const void *dw = nullptr, *ds = nullptr;
    const std::string key = cache_key;
    if (int32_t rc = upload_locked(ctx, "logits.w." + key, w, rows * cols, &dw)) return rc;
    if (int32_t rc = upload_locked(ctx, "logits.s." + key, scales_f16, rows * 2, &ds)) return rc;
    return run_logits(ctx, x, cols, rows, out, [&](const float* dx, float* dy) {
        return qgemv_i8_impl(ctx, reinterpret_cast<const int8_t*>(dw), ds, DT_F16, (int64_t)rows, dx, DT_F32, nullptr,
                             dy, 1, (int64_t)rows, (int64_t)cols, ctx->stream, false);
    });
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_logits_i4(cellm_hip_ctx_t* ctx, const float* x, const uint8_t* w, const uint16_t* scales_f16,
                            size_t n_scales, size_t rows, size_t cols, size_t gs, const char* cache_key, float* out)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!cache_key || (!x && cols) || (!out && rows)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    const void *dw = nullptr, *ds = nullptr;
    const std::string key = cache_key;
    if (int32_t rc = upload_locked(ctx, "logits.w." + key, w, rows * ((cols + 1) / 2), &dw)) return rc;
    if (int32_t rc = upload_locked(ctx, "logits.s." + key, scales_f16, n_scales * 2, &ds)) return rc;
    return run_logits(ctx, x, cols, rows, out, [&](const float* dx, float* dy) {
        return cellm_hip_qgemv_i4_sym(ctx, reinterpret_cast<const uint8_t*>(dw), reinterpret_cast<const uint16_t*>(ds),
                                      (int64_t)n_scales, (int64_t)gs, dx, DT_F32, dy, 1, (int64_t)rows, (int64_t)cols,
                                      ctx->stream);
    });
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_logits_q4_affine(cellm_hip_ctx_t* ctx, const float* x, const uint32_t* wq, const void* scales,
                                   const void* biases, int32_t sb_dtype, size_t rows, size_t cols,
                                   const char* cache_key, float* out)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (!cache_key || (!x && cols) || (!out && rows)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (!valid_dtype(sb_dtype)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (cols % 8 != 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "cols must be a multiple of 8");
    DeviceGuard g(ctx->device);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    const size_t groups = (cols + 63) / 64;
    const size_t sb_bytes = rows * groups * dtype_size(sb_dtype);
    const void *dw = nullptr, *ds = nullptr, *db = nullptr;
    const std::string key = cache_key;
    if (int32_t rc = upload_locked(ctx, "logits.w." + key, wq, rows * cols / 2, &dw)) return rc;
    if (int32_t rc = upload_locked(ctx, "logits.s." + key, scales, sb_bytes, &ds)) return rc;
    if (int32_t rc = upload_locked(ctx, "logits.b." + key, biases, sb_bytes, &db)) return rc;
    return run_logits(ctx, x, cols, rows, out, [&](const float* dx, float* dy) {
        return qgemv_q4_impl(ctx, reinterpret_cast<const uint32_t*>(dw), ds, db, sb_dtype, 64, dx, DT_F32, dy, 1,
                             (int64_t)rows, (int64_t)cols, ctx->stream, false);
    });
    CELLM_API_END(report_exception)
}

}  // extern "C"

// ---- decode-step ops (decode.hip): MetalOps::encode_rms_norm_f16w,
// encode_rope_half_f32, encode_add_f32_inplace and MetalKvStorage's
// encode_write_token_f32 / encode_attention (metal.rs, kvcache.rs) ---------

namespace {

int32_t check_paged(int64_t rows, int64_t max_blocks, int64_t total_blocks, int64_t n_layers, int64_t tpb,
                    int64_t layer)
{
    if (rows < 0 || rows > 4096 || max_blocks < 1 || total_blocks < 1 || n_layers < 1 || tpb < 1 || layer < 0 ||
        layer >= n_layers || max_blocks * tpb > INT32_MAX || total_blocks * n_layers * tpb > ((int64_t)1 << 40))
        return set_error(CELLM_HIP_ERR_INVALID_ARG,
                         "bad paged-cache geometry rows=%lld max_blocks=%lld total_blocks=%lld layers=%lld tpb=%lld "
                         "layer=%lld",
                         (long long)rows, (long long)max_blocks, (long long)total_blocks, (long long)n_layers,
                         (long long)tpb, (long long)layer);
    return CELLM_HIP_OK;
}

// Shared by cellm_hip_attention_gqa_f16kv (softmax partials in the context's
// per-stream scratch, grown on demand) and its _noalloc variant (the library's
// static scratch; nothing is allocated).
int32_t attention_impl(cellm_hip_ctx* ctx, const float* q, const uint16_t* kcache, const uint16_t* vcache,
                       const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks, const int32_t* positions,
                       int64_t rows, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t n_layers,
                       int64_t tokens_per_block, int64_t layer, float attn_scale, float soft_cap, float* out,
                       hipStream_t st, bool static_scratch, int64_t window = 0)
{
    if (window < 0 || window > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad window %lld", (long long)window);
    if (int32_t rc = check_paged(rows, max_blocks, total_blocks, n_layers, tokens_per_block, layer)) return rc;
    if (n_heads < 1 || n_kv_heads < 1 || head_dim < 1 || n_heads > 4096 ||
        !attention_supported((int)n_heads, (int)n_kv_heads, (int)head_dim, (int)(max_blocks * tokens_per_block)))
        return set_error(CELLM_HIP_ERR_UNSUPPORTED,
                         "attention needs n_heads %% n_kv_heads == 0, <= 8 query heads per kv head, head_dim 64 or "
                         "128 and max_blocks * tokens_per_block <= 32768 (got %lld/%lld/%lld, %lld positions)",
                         (long long)n_heads, (long long)n_kv_heads, (long long)head_dim,
                         (long long)(max_blocks * tokens_per_block));
    if (!(attn_scale >= 0.0f) || !(soft_cap >= 0.0f) || std::isinf(attn_scale) || std::isinf(soft_cap))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "attn_scale and soft_cap must be finite and >= 0 (0 = none)");
    const size_t need = attention_workspace_bytes((int)rows, (int)n_heads, (int)n_kv_heads, (int)head_dim,
                                                  (int)(max_blocks * tokens_per_block));
    if (static_scratch && need > kAttnStaticScratchBytes)
        return set_error(CELLM_HIP_ERR_INVALID_ARG,
                         "attention_noalloc: %zu bytes of softmax partials (rows x heads x ceil(max_blocks * "
                         "tokens_per_block / 64) x (head_dim + 2) floats) exceed the static scratch of %zu bytes",
                         need, kAttnStaticScratchBytes);
    if (rows == 0) return CELLM_HIP_OK;
    if (!q || !kcache || !vcache || !block_tables || !positions || !out)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (!aligned16(kcache) || !aligned16(vcache)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "K/V must be 16-byte aligned");
    float* ws = nullptr;
    if (static_scratch) {
        if (!ctx->attn_static) {
            std::lock_guard<std::recursive_mutex> lk(ctx->mu);
            if (!ctx->attn_static) HIP_TRY(attention_static_scratch(&ctx->attn_static), "hipGetSymbolAddress(attention scratch)");
        }
        ws = ctx->attn_static;
        if (!ws) return set_error(CELLM_HIP_ERR_DEVICE, "static attention scratch has no device address");
    } else if (int32_t rc = get_stream_buffer(ctx, ctx->attn, st, need, &ws, attention_counter_bytes())) {
        return rc;
    }
    HIP_TRY(launch_attention_gqa_f16kv(q, kcache, vcache, block_tables, (int)max_blocks, (int)total_blocks, positions,
                                       (int)rows, (int)n_heads, (int)n_kv_heads, (int)head_dim, (int)n_layers,
                                       (int)tokens_per_block, (int)layer, attn_scale, soft_cap, out, ws, st,
                                       (int)window),
            "attention launch");
    return CELLM_HIP_OK;
}

}  // namespace

extern "C" {

int32_t cellm_hip_embed_i8(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const int8_t* embed_i8,
                           const uint16_t* scales_f16, int64_t vocab, int64_t hidden, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, vocab, hidden)) return rc;
    if (rows == 0 || hidden == 0) return CELLM_HIP_OK;
    if (vocab < 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "vocab must be >= 1");
    if (!tokens || !embed_i8 || !scales_f16 || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_embed_i8(tokens, (int)rows, embed_i8, scales_f16, (int)vocab, (int)hidden, out,
                            pick_stream(ctx, stream)),
            "embed_i8 launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_embed_f16(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const uint16_t* embed_f16,
                            int64_t vocab, int64_t hidden, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, vocab, hidden)) return rc;
    if (rows == 0 || hidden == 0) return CELLM_HIP_OK;
    if (vocab < 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "vocab must be >= 1");
    if (!tokens || !embed_f16 || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_embed_f16(tokens, (int)rows, embed_f16, (int)vocab, (int)hidden, out, pick_stream(ctx, stream)),
            "embed_f16 launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_embed_i4(cellm_hip_ctx_t* ctx, const uint32_t* tokens, int64_t rows, const uint8_t* embed_i4,
                           const uint16_t* scales_f16, int64_t vocab, int64_t hidden, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, vocab, hidden)) return rc;
    if (rows == 0 || hidden == 0) return CELLM_HIP_OK;
    if (vocab < 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "vocab must be >= 1");
    if (!tokens || !embed_i4 || !scales_f16 || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_embed_i4(tokens, (int)rows, embed_i4, scales_f16, (int)vocab, (int)hidden, out,
                            pick_stream(ctx, stream)),
            "embed_i4 launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_rms_norm(cellm_hip_ctx_t* ctx, const float* x, const void* weight, int32_t weight_dtype,
                           int64_t rows, int64_t n, float eps, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n, 1)) return rc;
    if (!valid_dtype(weight_dtype)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (rows == 0 || n == 0) return CELLM_HIP_OK;
    if (!x || !weight || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_rms_norm(x, weight, weight_dtype, (int)rows, (int)n, eps, out, pick_stream(ctx, stream)),
            "rms_norm launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_add_rms_norm(cellm_hip_ctx_t* ctx, float* x, const float* y, const void* weight,
                               int32_t weight_dtype, int64_t rows, int64_t n, float eps, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n, 1)) return rc;
    if (!valid_dtype(weight_dtype)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad dtype");
    if (rows == 0 || n == 0) return CELLM_HIP_OK;
    if (!x || !y || !weight || !out) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_add_rms_norm(x, y, weight, weight_dtype, (int)rows, (int)n, eps, out, pick_stream(ctx, stream)),
            "add_rms_norm launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_rope_half_f32(cellm_hip_ctx_t* ctx, float* x, int64_t rows, int64_t n_heads, int64_t head_dim,
                                const int32_t* positions, const float* cos_sin, int64_t table_positions, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n_heads, head_dim)) return rc;
    if (rows == 0 || n_heads == 0 || head_dim == 0) return CELLM_HIP_OK;
    if (head_dim % 2 != 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "head_dim must be even");
    if (table_positions < 1 || table_positions > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "table_positions must be >= 1");
    if (rows * n_heads * head_dim > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "tensor too large");
    if (!x || !positions || !cos_sin) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_rope_half(x, (int)rows, (int)n_heads, (int)head_dim, positions, cos_sin, (int)table_positions, 0,
                             pick_stream(ctx, stream)),
            "rope_half launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_rope_interleaved_f32(cellm_hip_ctx_t* ctx, float* x, int64_t rows, int64_t n_heads, int64_t head_dim,
                                       const int32_t* positions, const float* cos_sin, int64_t table_positions,
                                       void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n_heads, head_dim)) return rc;
    if (rows == 0 || n_heads == 0 || head_dim == 0) return CELLM_HIP_OK;
    if (head_dim % 2 != 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "head_dim must be even");
    if (table_positions < 1 || table_positions > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "table_positions must be >= 1");
    if (rows * n_heads * head_dim > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "tensor too large");
    if (!x || !positions || !cos_sin) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_rope_half(x, (int)rows, (int)n_heads, (int)head_dim, positions, cos_sin, (int)table_positions, 1,
                             pick_stream(ctx, stream)),
            "rope_interleaved launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_set_rope_interleaved(cellm_hip_ctx_t* ctx, int32_t interleaved)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (interleaved != 0 && interleaved != 1) return set_error(CELLM_HIP_ERR_INVALID_ARG, "interleaved must be 0 or 1");
    ctx->rope_interleaved.store(interleaved);
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_kv_write_f16(cellm_hip_ctx_t* ctx, const float* k, const float* v, int64_t rows, int64_t kv_dim,
                               const int32_t* positions, uint16_t* kcache, uint16_t* vcache,
                               const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                               int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_paged(rows, max_blocks, total_blocks, n_layers, tokens_per_block, layer)) return rc;
    if (kv_dim < 1 || rows * kv_dim > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad kv_dim");
    if (rows == 0) return CELLM_HIP_OK;
    if (!k || !v || !positions || !kcache || !vcache || !block_tables)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_kv_write_f16(k, v, (int)rows, (int)kv_dim, positions, kcache, vcache, block_tables, (int)max_blocks,
                                (int)total_blocks, (int)n_layers, (int)tokens_per_block, (int)layer,
                                pick_stream(ctx, stream)),
            "kv_write launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_rope_kv_write_f16(cellm_hip_ctx_t* ctx, float* q, float* k, const float* v, int64_t rows,
                                    int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const int32_t* positions,
                                    const float* cos_sin, int64_t table_positions, uint16_t* kcache, uint16_t* vcache,
                                    const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                                    int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_paged(rows, max_blocks, total_blocks, n_layers, tokens_per_block, layer)) return rc;
    if (n_heads < 1 || n_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 ||
        rows * (n_heads + n_kv_heads) * head_dim > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad head geometry %lld/%lld/%lld", (long long)n_heads,
                         (long long)n_kv_heads, (long long)head_dim);
    if (table_positions < 1 || table_positions > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "table_positions must be >= 1");
    if (rows == 0) return CELLM_HIP_OK;
    if (!q || !k || !v || !positions || !cos_sin || !kcache || !vcache || !block_tables)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_rope_kv_write_f16(q, k, v, (int)rows, (int)n_heads, (int)n_kv_heads, (int)head_dim, positions,
                                     cos_sin, (int)table_positions, kcache, vcache, block_tables, (int)max_blocks,
                                     (int)total_blocks, (int)n_layers, (int)tokens_per_block, (int)layer,
                                     ctx->rope_interleaved.load(), pick_stream(ctx, stream)),
            "rope_kv_write launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_decode_qkv_rope_kv(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out,
                                     const float* norm_w, float eps, const int8_t* wq, const uint16_t* sq,
                                     const int8_t* wk, const uint16_t* sk, const int8_t* wv, const uint16_t* sv,
                                     int64_t rows, int64_t hidden, int64_t n_heads, int64_t n_kv_heads,
                                     int64_t head_dim, const int32_t* positions, const float* cos_sin,
                                     int64_t table_positions, float* q_out, uint16_t* kcache, uint16_t* vcache,
                                     const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
                                     int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_paged(rows, max_blocks, total_blocks, n_layers, tokens_per_block, layer)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (hidden > INT32_MAX || !decode_fused_supported((int)rows, (int)hidden) || hidden > 4096)
        return set_error(CELLM_HIP_ERR_UNSUPPORTED, "fused decode QKV needs 1..4 rows and hidden %% 16 == 0, <= 4096 "
                                                    "(got rows=%lld hidden=%lld)", (long long)rows, (long long)hidden);
    if (n_heads < 1 || n_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || n_heads > 4096 || n_kv_heads > 4096 ||
        head_dim > 4096)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad head geometry %lld/%lld/%lld", (long long)n_heads,
                         (long long)n_kv_heads, (long long)head_dim);
    if (table_positions < 1 || table_positions > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "table_positions must be >= 1");
    if (!x_prev || !x_out || !norm_w || !wq || !sq || !wk || !sk || !wv || !sv || !positions || !cos_sin || !q_out ||
        !kcache || !vcache || !block_tables)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (x_out == x_prev || x_out == y)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "x_out must not alias x_prev or y (other blocks still read them)");
    if (!aligned16(wq) || !aligned16(wk) || !aligned16(wv))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "weights must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    const int8_t* w[3] = {wq, wk, wv};
    const uint16_t* sc[3] = {sq, sk, sv};
    HIP_TRY(launch_decode_qkv(x_prev, y, x_out, norm_w, eps, w, sc, (int)rows, (int)hidden, (int)n_heads,
                              (int)n_kv_heads, (int)head_dim, positions, cos_sin, (int)table_positions, q_out, kcache,
                              vcache, block_tables, (int)max_blocks, (int)total_blocks, (int)n_layers,
                              (int)tokens_per_block, (int)layer, ctx->rope_interleaved.load(), pick_stream(ctx, stream)),
            "decode_qkv launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_decode_gate_up_silu(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out,
                                      const float* norm_w, float eps, const int8_t* wg, const uint16_t* sg,
                                      const int8_t* wu, const uint16_t* su, int64_t rows, int64_t hidden,
                                      int64_t inter, float* h, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (rows < 0 || hidden > INT32_MAX || !decode_fused_supported((int)rows, (int)hidden) || hidden > 4096)
        return set_error(CELLM_HIP_ERR_UNSUPPORTED, "fused decode gate/up needs 1..4 rows and hidden %% 16 == 0, "
                                                    "<= 4096 (got rows=%lld hidden=%lld)", (long long)rows,
                         (long long)hidden);
    if (inter < 1 || inter > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad intermediate size");
    if (!x_prev || !x_out || !norm_w || !wg || !sg || !wu || !su || !h)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (x_out == x_prev || x_out == y)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "x_out must not alias x_prev or y (other blocks still read them)");
    if (!aligned16(wg) || !aligned16(wu)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "weights must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_decode_gate_up(x_prev, y, x_out, norm_w, eps, wg, sg, wu, su, (int)rows, (int)hidden, (int)inter, h,
                                  pick_stream(ctx, stream)),
            "decode_gate_up launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

namespace {

// Shared checks of the two fused q4 decode entry points.
int32_t check_decode_q4(const float* x_prev, const float* y, const float* x_out, const float* norm_w,
                        int32_t sb_dtype, int64_t group, int64_t rows, int64_t hidden, const char* what)
{
    if (sb_dtype != CELLM_HIP_DTYPE_F32)
        return set_error(CELLM_HIP_ERR_UNSUPPORTED, "%s: scales and biases must be f32 (got dtype %d)", what,
                         (int)sb_dtype);
    if (rows < 1 || hidden > 4096 || group < 1 || group > hidden ||
        !decode_q4_fused_supported((int)rows, (int)hidden, (int)group))
        return set_error(CELLM_HIP_ERR_UNSUPPORTED, "%s needs 1..4 rows, hidden %% 32 == 0, <= 4096 and a power-of-two "
                                                    "group >= 32 (got rows=%lld hidden=%lld group=%lld)",
                         what, (long long)rows, (long long)hidden, (long long)group);
    if (!x_prev || !x_out || !norm_w) return set_error(CELLM_HIP_ERR_INVALID_ARG, "%s: null pointer", what);
    if (x_out == x_prev || x_out == y)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "x_out must not alias x_prev or y (other blocks still read them)");
    if (!aligned16(x_prev) || (y && !aligned16(y)) || !aligned16(x_out) || !aligned16(norm_w))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "%s: x_prev, y, x_out and norm_w must be 16-byte aligned", what);
    return CELLM_HIP_OK;
}

}  // namespace

int32_t cellm_hip_decode_q4_affine_qkv_rope_kv(
    cellm_hip_ctx_t* ctx, const float* x_prev, const float* y, float* x_out, const float* norm_w, float eps,
    const uint32_t* wq, const void* sq, const void* bq, const float* biasq, const uint32_t* wk, const void* sk,
    const void* bk, const float* biask, const uint32_t* wv, const void* sv, const void* bv, const float* biasv,
    int32_t sb_dtype, int64_t group, int64_t rows, int64_t hidden, int64_t n_heads, int64_t n_kv_heads,
    int64_t head_dim, const int32_t* positions, const float* cos_sin, int64_t table_positions, float* q_out,
    uint16_t* kcache, uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks, int64_t total_blocks,
    int64_t n_layers, int64_t tokens_per_block, int64_t layer, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_paged(rows, max_blocks, total_blocks, n_layers, tokens_per_block, layer)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (int32_t rc = check_decode_q4(x_prev, y, x_out, norm_w, sb_dtype, group, rows, hidden, "fused q4 decode QKV"))
        return rc;
    if (n_heads < 1 || n_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || n_heads > 4096 || n_kv_heads > 4096 ||
        head_dim > 4096)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad head geometry %lld/%lld/%lld", (long long)n_heads,
                         (long long)n_kv_heads, (long long)head_dim);
    if (table_positions < 1 || table_positions > INT32_MAX)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "table_positions must be >= 1");
    if (!wq || !sq || !bq || !wk || !sk || !bk || !wv || !sv || !bv || !positions || !cos_sin || !q_out || !kcache ||
        !vcache || !block_tables)
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (!aligned16(wq) || !aligned16(wk) || !aligned16(wv))
        return set_error(CELLM_HIP_ERR_INVALID_ARG, "weights must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    const uint32_t* w[3] = {wq, wk, wv};
    const float* s[3] = {static_cast<const float*>(sq), static_cast<const float*>(sk), static_cast<const float*>(sv)};
    const float* b[3] = {static_cast<const float*>(bq), static_cast<const float*>(bk), static_cast<const float*>(bv)};
    const float* bias[3] = {biasq, biask, biasv};
    HIP_TRY(launch_decode_q4_qkv(x_prev, y, x_out, norm_w, eps, w, s, b, bias, (int)group, (int)rows, (int)hidden,
                                 (int)n_heads, (int)n_kv_heads, (int)head_dim, positions, cos_sin,
                                 (int)table_positions, q_out, kcache, vcache, block_tables, (int)max_blocks,
                                 (int)total_blocks, (int)n_layers, (int)tokens_per_block, (int)layer,
                                 ctx->rope_interleaved.load(), pick_stream(ctx, stream)),
            "decode_q4_qkv launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_decode_q4_affine_gate_up_silu(cellm_hip_ctx_t* ctx, const float* x_prev, const float* y,
                                                float* x_out, const float* norm_w, float eps, const uint32_t* wg,
                                                const void* sg, const void* bg, const uint32_t* wu, const void* su,
                                                const void* bu, int32_t sb_dtype, int64_t group, int64_t rows,
                                                int64_t hidden, int64_t inter, float* h, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (int32_t rc =
            check_decode_q4(x_prev, y, x_out, norm_w, sb_dtype, group, rows, hidden, "fused q4 decode gate/up"))
        return rc;
    if (inter < 1 || inter > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad intermediate size");
    if (!wg || !sg || !bg || !wu || !su || !bu || !h) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (!aligned16(wg) || !aligned16(wu)) return set_error(CELLM_HIP_ERR_INVALID_ARG, "weights must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_decode_q4_gate_up(x_prev, y, x_out, norm_w, eps, wg, static_cast<const float*>(sg),
                                     static_cast<const float*>(bg), wu, static_cast<const float*>(su),
                                     static_cast<const float*>(bu), (int)group, (int)rows, (int)hidden, (int)inter,
                                     ACT_SILU, h, pick_stream(ctx, stream)),
            "decode_q4_gate_up launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_attention_gqa_f16kv(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                      const uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks,
                                      int64_t total_blocks, const int32_t* positions, int64_t rows, int64_t n_heads,
                                      int64_t n_kv_heads, int64_t head_dim, int64_t n_layers, int64_t tokens_per_block,
                                      int64_t layer, float attn_scale, float soft_cap, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return attention_impl(ctx, q, kcache, vcache, block_tables, max_blocks, total_blocks, positions, rows, n_heads,
                          n_kv_heads, head_dim, n_layers, tokens_per_block, layer, attn_scale, soft_cap, out,
                          pick_stream(ctx, stream), false);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_attention_gqa_f16kv_window(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                             const uint16_t* vcache, const uint32_t* block_tables, int64_t max_blocks,
                                             int64_t total_blocks, const int32_t* positions, int64_t rows,
                                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t n_layers,
                                             int64_t tokens_per_block, int64_t layer, float attn_scale, float soft_cap,
                                             int64_t window, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch users are enqueued
    return attention_impl(ctx, q, kcache, vcache, block_tables, max_blocks, total_blocks, positions, rows, n_heads,
                          n_kv_heads, head_dim, n_layers, tokens_per_block, layer, attn_scale, soft_cap, out,
                          pick_stream(ctx, stream), false, window);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_attention_gqa_f16kv_noalloc(cellm_hip_ctx_t* ctx, const float* q, const uint16_t* kcache,
                                              const uint16_t* vcache, const uint32_t* block_tables,
                                              int64_t max_blocks, int64_t total_blocks, const int32_t* positions,
                                              int64_t rows, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                              int64_t n_layers, int64_t tokens_per_block, int64_t layer,
                                              float attn_scale, float soft_cap, float* out, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    DeviceGuard g(ctx->device);
    return attention_impl(ctx, q, kcache, vcache, block_tables, max_blocks, total_blocks, positions, rows, n_heads,
                          n_kv_heads, head_dim, n_layers, tokens_per_block, layer, attn_scale, soft_cap, out,
                          pick_stream(ctx, stream), true);
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_silu_mul_f32(cellm_hip_ctx_t* ctx, float* gate, const float* up, int64_t n, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (n < 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad length");
    if (n == 0) return CELLM_HIP_OK;
    if (!gate || !up) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_silu_mul(gate, up, (size_t)n, pick_stream(ctx, stream)), "silu_mul launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_gelu_tanh_mul_f32(cellm_hip_ctx_t* ctx, float* gate, const float* up, int64_t n, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (n < 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad length");
    if (n == 0) return CELLM_HIP_OK;
    if (!gate || !up) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_act_mul(ACT_GELU_TANH, gate, up, (size_t)n, pick_stream(ctx, stream)), "gelu_tanh_mul launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_add_f32_inplace(cellm_hip_ctx_t* ctx, float* x, const float* y, int64_t n, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (n < 0 || n > INT32_MAX) return set_error(CELLM_HIP_ERR_INVALID_ARG, "bad length");
    if (n == 0) return CELLM_HIP_OK;
    if (!x || !y) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_add_f32(x, y, x, (int)n, pick_stream(ctx, stream)), "add launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_argmax_f32(cellm_hip_ctx_t* ctx, const float* logits, int64_t rows, int64_t n, int32_t* out_index,
                             float* out_value, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n, 1)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (n == 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "empty logits");
    if (!logits || !out_index || !out_value) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (rows > 65535) return set_error(CELLM_HIP_ERR_INVALID_ARG, "rows=%lld > 65535", (long long)rows);
    DeviceGuard g(ctx->device);
    const std::lock_guard<std::recursive_mutex> lk(ctx->mu);  // held until the scratch user is enqueued
    hipStream_t st = pick_stream(ctx, stream);
    // rows longer than one chunk: per-stream scratch, its row counters cleared when it is allocated
    // and returned to zero by every launch
    float* scratch = nullptr;
    if (int32_t rc = get_stream_buffer(ctx, ctx->argmax, st, argmax_scratch_bytes((int)rows, (int)n), &scratch,
                                       argmax_counter_bytes((int)rows)))
        return rc;
    HIP_TRY(launch_argmax(logits, (int)rows, (int)n, out_index, out_value, scratch, st), "argmax launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

int32_t cellm_hip_argmax_key_index(uint64_t key) { return (int32_t)(0xffffffffu - (uint32_t)key); }

float cellm_hip_argmax_key_value(uint64_t key)
{
    const uint32_t o = (uint32_t)(key >> 32);
    return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

int32_t cellm_hip_argmax_f32_keys(cellm_hip_ctx_t* ctx, const float* logits, int64_t rows, int64_t n,
                                  uint64_t* out_keys, void* stream)
{
    CELLM_API_BEGIN
    if (int32_t rc = check_ctx(ctx)) return rc;
    if (int32_t rc = check_dims(rows, n, 1)) return rc;
    if (rows == 0) return CELLM_HIP_OK;
    if (n == 0) return set_error(CELLM_HIP_ERR_INVALID_ARG, "empty logits");
    if (!logits || !out_keys) return set_error(CELLM_HIP_ERR_INVALID_ARG, "null pointer");
    if (rows > 65535) return set_error(CELLM_HIP_ERR_INVALID_ARG, "rows=%lld > 65535", (long long)rows);
    if (reinterpret_cast<uintptr_t>(out_keys) & 7) return set_error(CELLM_HIP_ERR_INVALID_ARG, "keys not 8-byte aligned");
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_argmax_keys(logits, (int)rows, (int)n, out_keys, pick_stream(ctx, stream)), "argmax launch");
    return CELLM_HIP_OK;
    CELLM_API_END(report_exception)
}

}  // extern "C"
