// Host-side launch helpers shared by the kernel files.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

namespace cellm {

// Raises the dynamic LDS limit of one kernel, once per device.
template <typename Kern>
hipError_t allow_big_lds(Kern kern, int bytes)
{
    // keyed by (device, kernel): every instantiation of a kernel template has the same pointer type
    struct Done {
        int dev;
        const void* fn;
        int bytes;
    };
    static std::mutex mu;
    static std::vector<Done> done;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const void* fn = reinterpret_cast<const void*>(kern);
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& d : done)
        if (d.dev == dev && d.fn == fn && d.bytes >= bytes) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done.push_back(Done{dev, fn, bytes});
    return e;
}

}  // namespace cellm
