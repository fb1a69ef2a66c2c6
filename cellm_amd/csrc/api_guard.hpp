// Error slot and exception guard shared by the library's C-ABI entry points.
//
// The reference turns Rust panics into status codes at its FFI boundary
// (catch_unwind, crates/cellm-sdk/src/ffi.rs:142); here every extern "C" body
// runs between CELLM_API_BEGIN and CELLM_API_END, so no C++ exception
// (std::bad_alloc from a std::string or container, or anything else) crosses
// the C ABI: it becomes CELLM_HIP_ERR_OUT_OF_MEMORY or CELLM_HIP_ERR_DEVICE
// with a message.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <exception>
#include <new>

namespace cellm {

// One thread's last error message.  A fixed buffer: recording an error never
// allocates, so a guard can report even after an allocation failure.
struct ErrorSlot {
    char msg[1024];
    size_t len;

    void store(const char* s, size_t n)
    {
        if (n >= sizeof(msg)) n = sizeof(msg) - 1;
        memcpy(msg, s, n);
        msg[n] = '\0';
        len = n;
    }

    // cellm_last_error_message (crates/cellm-sdk/src/ffi.rs:126-138): nothing
    // for a NULL or empty buffer; otherwise the message is taken (cleared),
    // copied truncated to buf_len - 1 bytes plus a NUL, and the number of
    // bytes written is returned.
    size_t take(char* buf, size_t buf_len)
    {
        if (!buf || buf_len == 0) return 0;
        const size_t n = len < buf_len - 1 ? len : buf_len - 1;
        memcpy(buf, msg, n);
        buf[n] = '\0';
        len = 0;
        msg[0] = '\0';
        return n;
    }
};

}  // namespace cellm

#define CELLM_API_BEGIN try {
// `report(int32_t code, const char* what)` records the error without allocating
// and returns `code`.
#define CELLM_API_END(report)                                                          \
    }                                                                                  \
    catch (const std::bad_alloc&) { return report(CELLM_HIP_ERR_OUT_OF_MEMORY, "host allocation failed"); } \
    catch (const std::exception& e_) { return report(CELLM_HIP_ERR_DEVICE, e_.what()); }                   \
    catch (...) { return report(CELLM_HIP_ERR_DEVICE, "unknown C++ exception"); }
// For entry points that return nothing (destroy/close): the exception is dropped.
#define CELLM_API_END_VOID \
    }                      \
    catch (...) {}
