// runtime.hip — status plumbing for the C-ABI. The last error is per host
// thread, so threads that drive different streams do not see each other's.

#include "../../include/ds4hip.h"
#include "ds4hip_common.h"

#include <map>
#include <mutex>
#include <utility>

namespace {
thread_local int t_last_error = 0;
}

extern "C" int ds4hip_set_last_error(int code) {
    if (code != 0) t_last_error = code;
    return code;
}

extern "C" int ds4hip_get_last_error(void) { return t_last_error; }

extern "C" int ds4hip_version(void) { return (0 << 16) | 2; }

extern "C" int ds4hip_clear_last_error(void) {
    const int e = t_last_error;
    t_last_error = 0;
    return e;
}

namespace ds4hip {

int stream_scratch(hipStream_t stream, size_t bytes, void **out) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return kHipErrBase - (int)e;
    std::lock_guard<std::mutex> lock(mu);
    auto &slot = cache[{dev, stream}];
    if (slot.second < bytes) {
        if (slot.first) {
            e = hipFreeAsync(slot.first, stream);
            slot.first = nullptr;
            slot.second = 0;
            if (e != hipSuccess) return kHipErrBase - (int)e;
        }
        const size_t want = bytes < 4096 ? 4096 : bytes;
        e = hipMallocAsync(&slot.first, want, stream);
        if (e != hipSuccess) {
            slot.first = nullptr;
            return kHipErrBase - (int)e;
        }
        slot.second = want;
    }
    *out = slot.first;
    return 0;
}

}  // namespace ds4hip
