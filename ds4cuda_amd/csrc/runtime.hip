// runtime.hip — library-wide status plumbing for the C-ABI.

#include <atomic>

#include "../../include/ds4hip.h"

namespace {
std::atomic<int> g_last_error{0};
}

extern "C" int ds4hip_set_last_error(int code) {
    if (code != 0) g_last_error.store(code, std::memory_order_relaxed);
    return code;
}

extern "C" int ds4hip_get_last_error(void) { return g_last_error.load(std::memory_order_relaxed); }

extern "C" int ds4hip_version(void) { return (0 << 16) | 1; }

extern "C" int ds4hip_clear_last_error(void) {
    return g_last_error.exchange(0, std::memory_order_relaxed);
}
