// Exhaustive host check of the device FP8 helpers in ds4hip_common.h:
//  1. ceil_log2_cr(y) == ceil((float)log2((double)y)) for every fp32 y in
//     [2^-30, 2^30) (the reference evaluates ceil(log2(amax/448)) in fp32;
//     a correctly rounded log2 is the definition the integer rule restates);
//  2. fp8_block_exp(amax) == the oracle's scale exponent for every fp32 amax
//     in [2^-17, 2^24);
//  3. e4m3_encode(v) == the oracle's nearest-code picker (binary search over
//     the value table, ties to the even code) for every fp32 v in [0, 448],
//     and the sign rule for the negated values.
// Built with hipcc (host pass only) and linked against the oracle library.
#include "ds4hip_common.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "ds4_oracle.h"

using namespace ds4hip;

static float from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

int main() {
    const int n_thr = 8;
    std::vector<long> bad_log(n_thr, 0), bad_enc(n_thr, 0);
    std::vector<std::thread> th;
    const uint32_t lo = 0x30800000u, hi = 0x4E800000u;   // 2^-30 .. 2^30
    const uint32_t enc_hi = 0x43E00000u;                  // 448.0
    for (int t = 0; t < n_thr; ++t)
        th.emplace_back([&, t] {
            for (uint32_t u = lo + t; u < hi; u += n_thr) {
                const float y = from_bits(u);
                const int ref = (int)std::ceil((float)std::log2((double)y));
                if (ceil_log2_cr(y) != ref) ++bad_log[t];
            }
            // block exponent from amax (floor 1e-4, quotient by 448) vs the oracle
            for (uint32_t u = 0x37000000u + t; u < 0x4B800000u; u += n_thr) {
                const float a = from_bits(u);
                if (fp8_block_exp(a) != orc_fp8_scale_exp(a)) ++bad_log[t];
            }
            for (uint32_t u = t; u <= enc_hi; u += n_thr) {
                const float v = from_bits(u);
                const uint32_t ref = (uint32_t)orc_e4m3fn_nearest_index(v);
                if (e4m3_encode(v) != ref) ++bad_enc[t];
                if (u && e4m3_encode(-v) != (ref | 0x80u)) ++bad_enc[t];
            }
        });
    for (auto &x : th) x.join();
    long bl = 0, be = 0;
    for (int t = 0; t < n_thr; ++t) bl += bad_log[t], be += bad_enc[t];
    std::printf("log2 rule mismatches %ld, encoder mismatches %ld\n", bl, be);
    return (bl || be) ? 1 : 0;
}
