// .cellm model files on the host side of the boundary, and their upload into
// the HIP weight cache (declared in include/cellm_hip.h).
//
// Format (crates/cellm-model/src/cellm_file.rs:58-124; writer
// tools/convert_lfm.py:15-90):
//   bytes 0..5   "CELLM"
//   byte  5      version (1)
//   bytes 6..10  header length, u32 little endian
//   JSON header  {"model_type": ..., "vocab_size": ..., ..., "tensors": [
//                  {"name", "offset_bytes", "nbytes", "shape", "dtype"}, ...]}
//   tensor data  at absolute file offsets (64-byte aligned by the writers)
// The file is mapped read-only; every tensor range is checked against the
// file size and every 4 KiB page is touched once at open, as the reference
// pre-warms its mapping (cellm_file.rs:91-105).  The header is parsed by the
// small JSON reader below (objects, arrays, strings with escapes, numbers,
// true / false / null), which keeps the raw text for callers that want the
// other fields.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/cellm_hip.h"
#include "api_guard.hpp"

namespace cellm {
int32_t set_error_external(int32_t code, const std::string& msg);  // capi.cpp: the thread's last error
int32_t report_exception(int32_t code, const char* what);           // capi.cpp: the same, without allocating
}

namespace {

int32_t fail(int32_t code, const char* fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return cellm::set_error_external(code, buf);
}

// ---- a small JSON reader -------------------------------------------------

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const char* key) const
    {
        if (kind != Obj) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
public:
    JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Json& out, std::string& err)
    {
        if (!value(out, 0)) {
            err = err_.empty() ? "malformed JSON" : err_;
            char at[64];
            snprintf(at, sizeof(at), " at byte %zu", (size_t)(p_ - begin()));
            err += at;
            return false;
        }
        ws();
        if (p_ != end_) {
            err = "trailing characters after the JSON header";
            return false;
        }
        return true;
    }

private:
    const char* p_;
    const char* end_;
    const char* start_ = p_;
    std::string err_;

    const char* begin() const { return start_; }
    void ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s)
    {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t c)
    {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& v)
    {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s)
    {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            const char c = *p_++;
            if ((unsigned char)c < 0x20) {
                err_ = "control character in a JSON string";
                return false;
            }
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
            switch (e) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    uint32_t lo;
                    if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                put_utf8(s, cp);
                break;
            }
            default: err_ = "bad escape in a JSON string"; return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(double& v)
    {
        const char* b = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || !((*p_ >= '0' && *p_ <= '9'))) return false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                             *p_ == '-'))
            ++p_;
        const std::string t(b, p_);
        char* e = nullptr;
        v = strtod(t.c_str(), &e);
        return e && *e == '\0';
    }
    bool value(Json& out, int depth)
    {
        if (depth > 64) {
            err_ = "JSON nested too deeply";
            return false;
        }
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            out.kind = Json::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Json v;
                if (!value(v, depth + 1)) return false;
                out.obj.emplace_back(std::move(key), std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            out.kind = Json::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Json v;
                if (!value(v, depth + 1)) return false;
                out.arr.push_back(std::move(v));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            out.kind = Json::Str;
            return string(out.str);
        }
        if (lit("true")) {
            out.kind = Json::Bool;
            out.b = true;
            return true;
        }
        if (lit("false")) {
            out.kind = Json::Bool;
            return true;
        }
        if (lit("null")) {
            out.kind = Json::Null;
            return true;
        }
        out.kind = Json::Num;
        return number(out.num);
    }
};

bool as_u64(const Json* j, uint64_t& v)
{
    if (!j || j->kind != Json::Num || j->num < 0 || j->num != std::floor(j->num) || j->num > 9007199254740992.0)
        return false;
    v = (uint64_t)j->num;
    return true;
}

}  // namespace

struct cellm_file {
    int fd = -1;
    const unsigned char* map = nullptr;
    size_t size = 0;
    std::string header_text;
    Json header;
    std::vector<cellm_file_tensor_t> tensors;  // name/dtype point into names_/dtypes_
    std::vector<std::unique_ptr<std::string>> names_, dtypes_;
    std::unordered_map<std::string, size_t> by_name;
    cellm_file_config_t config{};

    ~cellm_file()
    {
        if (map) munmap(const_cast<unsigned char*>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int32_t read_config(cellm_file* f)
{
    cellm_file_config_t& c = f->config;
    const Json& h = f->header;
    const Json* mt = h.get("model_type");
    if (!mt || mt->kind != Json::Str) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: model_type missing");
    snprintf(c.model_type, sizeof(c.model_type), "%s", mt->str.c_str());
    struct {
        const char* key;
        int64_t* dst;
        bool required;
    } ints[] = {{"vocab_size", &c.vocab_size, true},
                {"hidden_dim", &c.hidden_dim, true},
                {"intermediate_size", &c.intermediate_size, true},
                {"num_layers", &c.num_layers, true},
                {"num_heads", &c.num_heads, true},
                {"num_kv_heads", &c.num_kv_heads, true},
                {"head_dim", &c.head_dim, false},
                {"bos_token_id", &c.bos_token_id, false},
                {"eos_token_id", &c.eos_token_id, false},
                {"max_position_embeddings", &c.max_position_embeddings, false}};
    for (auto& e : ints) {
        const Json* j = h.get(e.key);
        uint64_t v = 0;
        if (!j || j->kind == Json::Null) {
            if (e.required) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: %s missing", e.key);
            *e.dst = -1;
            continue;
        }
        if (!as_u64(j, v)) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: %s is not a count", e.key);
        *e.dst = (int64_t)v;
    }
    const Json* eps = h.get("rms_norm_eps");
    const Json* theta = h.get("rope_theta");
    if (!eps || eps->kind != Json::Num || !theta || theta->kind != Json::Num)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: rms_norm_eps / rope_theta missing");
    c.rms_norm_eps = (float)eps->num;  // serde's f32 from the JSON number
    c.rope_theta = (float)theta->num;
    const Json* tie = h.get("tie_word_embeddings");
    c.tie_word_embeddings = (tie && tie->kind == Json::Bool) ? (tie->b ? 1 : 0) : -1;
    return CELLM_HIP_OK;
}

}  // namespace

extern "C" {

int32_t cellm_file_open(const char* path, cellm_file_t** out)
{
    CELLM_API_BEGIN
    if (!path || !out) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    std::unique_ptr<cellm_file> f(new cellm_file());
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: open failed: %s", strerror(errno));
    struct stat st;
    if (fstat(f->fd, &st) != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: stat failed: %s", strerror(errno));
    f->size = (size_t)st.st_size;
    if (f->size < 10) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: file too small");
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: mmap failed: %s", strerror(errno));
    f->map = static_cast<const unsigned char*>(m);
    if (memcmp(f->map, "CELLM", 5) != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: bad magic");
    if (f->map[5] != 1) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: unsupported version %u", f->map[5]);
    const uint32_t hlen = (uint32_t)f->map[6] | ((uint32_t)f->map[7] << 8) | ((uint32_t)f->map[8] << 16) |
                          ((uint32_t)f->map[9] << 24);
    if ((uint64_t)10 + hlen > f->size) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: header length out of range");
    f->header_text.assign(reinterpret_cast<const char*>(f->map + 10), hlen);
    std::string err;
    JsonParser jp(f->header_text.data(), f->header_text.size());
    if (!jp.parse(f->header, err) || f->header.kind != Json::Obj)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: header json parse failed: %s",
                    err.empty() ? "not an object" : err.c_str());
    if (int32_t rc = read_config(f.get())) return rc;
    const Json* ts = f->header.get("tensors");
    if (!ts || ts->kind != Json::Arr) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: tensors missing");
    f->tensors.reserve(ts->arr.size());
    for (size_t i = 0; i < ts->arr.size(); ++i) {
        const Json& t = ts->arr[i];
        const Json* name = t.get("name");
        const Json* dtype = t.get("dtype");
        const Json* shape = t.get("shape");
        uint64_t off = 0, nb = 0;
        if (!name || name->kind != Json::Str || !dtype || dtype->kind != Json::Str || !shape ||
            shape->kind != Json::Arr || !as_u64(t.get("offset_bytes"), off) || !as_u64(t.get("nbytes"), nb))
            return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: tensor entry %zu is malformed", i);
        if (shape->arr.size() > 8) return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: tensor %s has rank > 8",
                                               name->str.c_str());
        if (off > f->size || nb > f->size - off)  // cellm_file.rs:108-119
            return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm load: tensor %s out of range (end=%llu file_len=%zu)",
                        name->str.c_str(), (unsigned long long)(off + nb), f->size);
        cellm_file_tensor_t e{};
        f->names_.emplace_back(new std::string(name->str));
        f->dtypes_.emplace_back(new std::string(dtype->str));
        e.name = f->names_.back()->c_str();
        e.dtype = f->dtypes_.back()->c_str();
        e.ndim = (int32_t)shape->arr.size();
        for (size_t d = 0; d < shape->arr.size(); ++d) {
            uint64_t v;
            if (!as_u64(&shape->arr[d], v))
                return fail(CELLM_HIP_ERR_INVALID_ARG, "cellm header: tensor %s has a bad shape", name->str.c_str());
            e.shape[d] = (int64_t)v;
        }
        e.offset_bytes = off;
        e.nbytes = nb;
        // A name seen again replaces the earlier entry (cellm_file.rs:89-92 builds
        // its index with HashMap::insert, so the last entry wins); every entry,
        // shadowed or not, has passed the range check above.
        const auto ins = f->by_name.emplace(name->str, f->tensors.size());
        if (ins.second)
            f->tensors.push_back(e);
        else
            f->tensors[ins.first->second] = e;
    }
    // one read per 4 KiB page brings the file into the page cache now
    (void)madvise(m, f->size, MADV_WILLNEED);
    volatile unsigned char sink = 0;
    for (size_t i = 0; i < f->size; i += 4096) sink = sink | f->map[i];
    (void)sink;
    *out = f.release();
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

void cellm_file_close(cellm_file_t* f) { delete f; }

int32_t cellm_file_config(const cellm_file_t* f, cellm_file_config_t* out)
{
    CELLM_API_BEGIN
    if (!f || !out) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *out = f->config;
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

int32_t cellm_file_header_json(const cellm_file_t* f, const char** out_text, size_t* out_len)
{
    CELLM_API_BEGIN
    if (!f || !out_text || !out_len) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    *out_text = f->header_text.data();
    *out_len = f->header_text.size();
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

int64_t cellm_file_tensor_count(const cellm_file_t* f) { return f ? (int64_t)f->tensors.size() : -1; }

int32_t cellm_file_tensor_at(const cellm_file_t* f, int64_t index, cellm_file_tensor_t* out)
{
    CELLM_API_BEGIN
    if (!f || !out) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (index < 0 || index >= (int64_t)f->tensors.size())
        return fail(CELLM_HIP_ERR_INVALID_ARG, "tensor index %lld out of range", (long long)index);
    *out = f->tensors[(size_t)index];
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

int32_t cellm_file_find(const cellm_file_t* f, const char* name, cellm_file_tensor_t* out)
{
    CELLM_API_BEGIN
    if (!f || !name) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return fail(CELLM_HIP_ERR_NOT_FOUND, "cellm: unknown tensor %s", name);
    if (out) *out = f->tensors[it->second];
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

int32_t cellm_file_tensor_bytes(const cellm_file_t* f, const char* name, const void** out_host, size_t* out_nbytes)
{
    CELLM_API_BEGIN
    cellm_file_tensor_t t;
    if (int32_t rc = cellm_file_find(f, name, &t)) return rc;
    if (out_host) *out_host = f->map + t.offset_bytes;
    if (out_nbytes) *out_nbytes = (size_t)t.nbytes;
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}

int32_t cellm_hip_upload_cellm_file(cellm_hip_ctx_t* ctx, const cellm_file_t* f, const char* name_prefix,
                                    int64_t* out_count, size_t* out_bytes)
{
    CELLM_API_BEGIN
    if (!ctx || !f) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    const size_t plen = name_prefix ? strlen(name_prefix) : 0;
    int64_t count = 0;
    size_t bytes = 0;
    for (const cellm_file_tensor_t& t : f->tensors) {
        if (plen && strncmp(t.name, name_prefix, plen) != 0) continue;
        const void* dev = nullptr;
        if (int32_t rc = cellm_hip_weight_upload(ctx, t.name, f->map + t.offset_bytes, (size_t)t.nbytes, &dev))
            return rc;
        ++count;
        bytes += (size_t)t.nbytes;
    }
    if (out_count) *out_count = count;
    if (out_bytes) *out_bytes = bytes;
    return CELLM_HIP_OK;
    CELLM_API_END(cellm::report_exception)
}


// One projection by the dtype of its .cellm weight tensor, with the rules of
// the runner family's linear_f16_out_in.  The tensors it reads go into the
// context's weight cache under their file names on first use (blocking
// upload), as the Metal ops cache weights by name; later calls only enqueue.
int32_t cellm_hip_linear_file(cellm_hip_ctx_t* ctx, const cellm_file_t* f, const char* weight_name, int32_t family,
                              const float* x, float* y, int64_t m, int64_t out_dim, int64_t in_dim, void* stream)
{
    CELLM_API_BEGIN
    if (!ctx || !f || !weight_name) return fail(CELLM_HIP_ERR_INVALID_ARG, "null argument");
    if (family < CELLM_HIP_FAMILY_LLAMA || family > CELLM_HIP_FAMILY_LFM)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "unknown runner family %d", family);
    if (m < 0 || out_dim < 1 || in_dim < 1 || out_dim > INT32_MAX || in_dim > INT32_MAX)
        return fail(CELLM_HIP_ERR_INVALID_ARG, "bad dimensions m=%lld out=%lld in=%lld", (long long)m,
                    (long long)out_dim, (long long)in_dim);
    if (m > 0 && (!x || !y)) return fail(CELLM_HIP_ERR_INVALID_ARG, "null x or y");
    const std::string name = weight_name;
    const long long o = out_dim, i = in_dim;
    auto find = [&](const std::string& n) -> const cellm_file_tensor_t* {
        auto it = f->by_name.find(n);
        return it == f->by_name.end() ? nullptr : &f->tensors[it->second];
    };
    auto on_device = [&](const cellm_file_tensor_t* t, const void** dev) -> int32_t {
        return cellm_hip_weight_upload(ctx, t->name, f->map + t->offset_bytes, (size_t)t->nbytes, dev);
    };
    // "<w>.qscale" as f16 row scales of at least one per row; `exact` requires exactly one per row
    auto qscale = [&](bool exact, const void** dev, int64_t* count) -> int32_t {
        const cellm_file_tensor_t* s = find(name + ".qscale");
        if (!s) return fail(CELLM_HIP_ERR_NOT_FOUND, "unknown tensor %s.qscale", weight_name);
        *count = (int64_t)(s->nbytes / 2);
        if (exact && *count != out_dim)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s qscale len mismatch: %lld expected %lld", weight_name,
                        (long long)*count, o);
        if (*count < out_dim)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s qscale holds %lld scales for %lld rows", weight_name,
                        (long long)*count, o);
        return on_device(s, dev);
    };
    auto len_check = [&](const cellm_file_tensor_t* t, uint64_t want, long long elems, long long want_elems) {
        return t->nbytes == want ? CELLM_HIP_OK
                                 : fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s len mismatch: %lld expected %lld",
                                        weight_name, elems, want_elems);
    };
    const cellm_file_tensor_t* t = find(name);
    const int fam = family;
    if (!t) {
        if (fam == CELLM_HIP_FAMILY_QWEN)  // qwen.rs:1035-1036
            return fail(CELLM_HIP_ERR_NOT_FOUND, "linear_f16_out_in: unknown tensor '%s'", weight_name);
        return fail(CELLM_HIP_ERR_NOT_FOUND, "unknown tensor %s", weight_name);
    }
    const std::string dt = t->dtype;
    if (fam == CELLM_HIP_FAMILY_LLAMA || fam == CELLM_HIP_FAMILY_GEMMA) {
        // [out, in] check of llama.rs:764-776 / gemma.rs:1366-1391
        std::string shape = "[";
        for (int32_t d = 0; d < t->ndim; ++d) shape += (d ? ", " : "") + std::to_string(t->shape[d]);
        shape += "]";
        if (t->ndim != 2) return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s expected 2D, got %s", weight_name, shape.c_str());
        if (t->shape[0] != out_dim || t->shape[1] != in_dim)
            return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s shape mismatch: %s expected [%lld,%lld]", weight_name,
                        shape.c_str(), o, i);
    }
    const void *w = nullptr, *s = nullptr, *b = nullptr;
    int64_t ns = 0;
    if (fam == CELLM_HIP_FAMILY_LFM) {
        // lfm.rs:924-981: "u32" with "<base>.scales" and "<base>.biases" is the MLX affine GEMV (group 64,
        // f32 scales and biases); any other tensor is read as f16
        const std::string base = name.size() > 7 && name.compare(name.size() - 7, 7, ".weight") == 0
                                     ? name.substr(0, name.size() - 7)
                                     : name;
        const cellm_file_tensor_t *ts = find(base + ".scales"), *tb = find(base + ".biases");
        if (dt == "u32" && ts && tb) {
            const uint64_t groups = (uint64_t)(i + 63) / 64;
            if (i % 8 != 0 || t->nbytes != (uint64_t)o * i / 2 || ts->nbytes != (uint64_t)o * groups * 4 ||
                tb->nbytes != (uint64_t)o * groups * 4)
                return fail(CELLM_HIP_ERR_INVALID_ARG,
                            "%s: u32 words / f32 scales / biases do not match [%lld, %lld] in groups of 64",
                            weight_name, o, i);
            if (int32_t rc = on_device(t, &w)) return rc;
            if (int32_t rc = on_device(ts, &s)) return rc;
            if (int32_t rc = on_device(tb, &b)) return rc;
            return cellm_hip_qgemv_q4_affine(ctx, static_cast<const uint32_t*>(w), s, b, CELLM_HIP_DTYPE_F32, 64, x,
                                             CELLM_HIP_DTYPE_F32, y, m, out_dim, in_dim, stream);
        }
        if (t->nbytes % 2 != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "tensor %s nbytes not even", weight_name);
        if (t->nbytes != (uint64_t)o * i * 2)
            return fail(CELLM_HIP_ERR_INVALID_ARG,
                        "linear_f16_out_in: weight shape mismatch for %s: got %llu elements, expected %lld (%lldx%lld "
                        "f16)",
                        weight_name, (unsigned long long)(t->nbytes / 2), o * i, o, i);
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_f16(ctx, static_cast<const uint16_t*>(w), x, CELLM_HIP_DTYPE_F32, y, m, out_dim,
                                   in_dim, stream);
    }
    if (dt == "f16") {
        if (int32_t rc = len_check(t, (uint64_t)o * i * 2, (long long)(t->nbytes / 2), o * i)) return rc;
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_f16(ctx, static_cast<const uint16_t*>(w), x, CELLM_HIP_DTYPE_F32, y, m, out_dim,
                                   in_dim, stream);
    }
    if (dt == "i8") {
        // matmul_i8_f32: the row scale applied to the row sum
        if (int32_t rc = len_check(t, (uint64_t)o * i, (long long)t->nbytes, o * i)) return rc;
        if (int32_t rc = qscale(fam != CELLM_HIP_FAMILY_QWEN, &s, &ns)) return rc;
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_i8(ctx, static_cast<const int8_t*>(w), s, CELLM_HIP_DTYPE_F16, out_dim, x,
                                  CELLM_HIP_DTYPE_F32, nullptr, y, m, out_dim, in_dim, stream);
    }
    if (dt == "i4") {
        // matmul_i4_f32 with gs = in_dim (llama.rs:932, gemma.rs:1471), or one scale per group of
        // in_dim / (scales per row) when there are more scales than rows (qwen.rs:1076-1077)
        const uint64_t row_bytes = (uint64_t)(i + 1) / 2;
        if (int32_t rc = len_check(t, (uint64_t)o * row_bytes, (long long)t->nbytes, o * (long long)row_bytes))
            return rc;
        if (int32_t rc = qscale(fam == CELLM_HIP_FAMILY_GEMMA, &s, &ns)) return rc;
        const int64_t gs = (fam == CELLM_HIP_FAMILY_QWEN && ns > out_dim) ? in_dim / (ns / out_dim) : in_dim;
        if (gs < 1) return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s: more scale groups than columns", weight_name);
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_i4_sym(ctx, static_cast<const uint8_t*>(w), static_cast<const uint16_t*>(s), ns, gs,
                                      x, CELLM_HIP_DTYPE_F32, y, m, out_dim, in_dim, stream);
    }
    if (dt == "i2" && fam != CELLM_HIP_FAMILY_LLAMA) {
        // Qwen's dot_i2_scaled_row scales the row sum (qwen.rs:1591-1606); Gemma's each element
        // (gemma.rs:1673-1687)
        if (int32_t rc = len_check(t, (uint64_t)o * ((i + 3) / 4), (long long)t->nbytes, o * ((i + 3) / 4)))
            return rc;
        if (int32_t rc = qscale(false, &s, &ns)) return rc;
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_i2(ctx, static_cast<const uint8_t*>(w), static_cast<const uint16_t*>(s),
                                  fam == CELLM_HIP_FAMILY_GEMMA ? 1 : 0, x, CELLM_HIP_DTYPE_F32, y, m, out_dim, in_dim,
                                  stream);
    }
    if (dt == "q1_0_g128" && fam == CELLM_HIP_FAMILY_QWEN) {
        // dot_row (qwen.rs:1004-1022): in_dim / 128 blocks of 18 bytes per row
        if (i % 128 != 0) return fail(CELLM_HIP_ERR_INVALID_ARG, "weight %s: q1_0_g128 needs in %% 128 == 0", weight_name);
        if (int32_t rc = len_check(t, (uint64_t)o * (i / 128) * 18, (long long)t->nbytes, o * (i / 128) * 18))
            return rc;
        if (int32_t rc = on_device(t, &w)) return rc;
        return cellm_hip_qgemv_q1_0_g128(ctx, static_cast<const uint8_t*>(w), x, CELLM_HIP_DTYPE_F32, y, m, out_dim,
                                         in_dim, stream);
    }
    if (fam == CELLM_HIP_FAMILY_QWEN)  // qwen.rs:1101
        return fail(CELLM_HIP_ERR_UNSUPPORTED, "linear fallback unsupported dtype %s", dt.c_str());
    return fail(CELLM_HIP_ERR_UNSUPPORTED, "unsupported weight dtype for %s: %s", weight_name, dt.c_str());
    CELLM_API_END(cellm::report_exception)
}

}  // extern "C"
