// Compiles a caller against the ds4cuda:: launcher shims and runs the paths
// that are decided on the host (no GPU work is launched).
#include "ds4hip_launchers.h"

#include <cstdio>

int main() {
    ds4hip_clear_last_error();
    ds4cuda::launch_indexer_allowed_short_circuit_i32(nullptr, 0, 512);  // no-op
    if (ds4hip_get_last_error() != 0) return 1;
    ds4cuda::ds4hip_abort_on_misuse() = false;
    ds4cuda::launch_indexer_allowed_short_circuit_i32(nullptr, 600, 512);  // misuse
    if (ds4hip_get_last_error() != -22) return 2;
    ds4hip_clear_last_error();
    ds4cuda::launch_flash_attn_decode_raw_f32(nullptr, nullptr, nullptr, nullptr, nullptr, 64, 4,
                                              256);  // head_dim 256 rejected
    if (ds4hip_get_last_error() != -22) return 3;
    ds4hip_clear_last_error();
    ds4cuda::launch_fp8_kv_quantize_round_trip_f32(nullptr, nullptr, 0, 512, 64);  // no rows
    if (ds4hip_get_last_error() != 0) return 4;
    std::printf("shim ok\n");
    return 0;
}
