// launch_util.h — host-side launch helpers shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>

namespace moe {

// Dynamic shared memory above 64 KiB needs the kernel's hipFuncAttributeMaxDynamicSharedMemorySize raised.  The
// attribute belongs to the kernel function for the whole process, so it is only ever raised (to the largest size any
// launch asked for), under a lock: a launch never runs with a limit that another thread's smaller launch lowered.
inline hipError_t raise_lds_limit(const void* fn, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> set;
    std::lock_guard<std::mutex> lock(mu);
    size_t& cur = set[fn];
    if (lds <= cur) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) cur = lds;
    return e;
}

}  // namespace moe
