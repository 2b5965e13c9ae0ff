// rope.h — the tail RoPE (YaRN) of the model's rows: host-side parameters per
// layer and the device rotation of one pair, shared by the RoPE kernels
// (rope_matvec.hip) and the decode merge's rotated Q8_0 output (flash_attn.hip).
#pragma once

#include "ds4hip_common.h"

#include <cmath>

namespace ds4hip {

struct RopeParams {
    float theta_scale;
    float freq_scale;
    float ext_factor;
    float attn_factor;
    float corr_low;
    float corr_high;
    float sin_sign;
};

// cuda/rope.cu:123-126
inline int compress_ratio_of(int il) { return il < 2 ? 0 : ((il & 1) == 0 ? 4 : 128); }

// cuda/rope.cu:214-250 (host-side parameter routing)
inline RopeParams rope_params(int n_rot, int il, bool inverse) {
    constexpr float kFreqBase = 10000.0f, kScale = 16.0f, kBetaFast = 32.0f, kBetaSlow = 1.0f;
    constexpr float kCompressBase = 160000.0f;
    constexpr int kOrigCtx = 65536;
    const bool compressed = compress_ratio_of(il) != 0;
    RopeParams P;
    const float freq_base = compressed ? kCompressBase : kFreqBase;
    P.freq_scale = compressed ? 1.0f / kScale : 1.0f;
    P.ext_factor = compressed ? 1.0f : 0.0f;
    P.attn_factor = 1.0f;
    if (P.ext_factor != 0.0f) P.attn_factor /= 1.0f + 0.1f * logf(1.0f / P.freq_scale);
    P.corr_low = P.corr_high = 0.0f;
    if (P.ext_factor != 0.0f) {
        const float pi = 3.14159265358979323846f;
        auto corr_dim = [&](float target) {
            return (float)n_rot * logf((float)kOrigCtx / (target * 2.0f * pi)) /
                   (2.0f * logf(freq_base));
        };
        P.corr_low = fmaxf(0.0f, floorf(corr_dim(kBetaFast)));
        P.corr_high = fminf((float)(n_rot - 1), ceilf(corr_dim(kBetaSlow)));
    }
    P.theta_scale = powf(freq_base, -2.0f / (float)n_rot);
    P.sin_sign = inverse ? -1.0f : 1.0f;
    return P;
}

// Rotation of pair t (dims n_nope + 2t, n_nope + 2t + 1) at position pos:
// its coefficients c, s (rope_cs), then y = (x0 c - x1 s, x0 s + x1 c).
__device__ inline void rope_cs(int t, int pos, const RopeParams &P, float &c_out, float &s_out) {
    float theta_extrap = (float)pos;
    for (int k = 0; k < t; ++k) theta_extrap *= P.theta_scale;   // running product (rope.cu:172-177)
    const float theta_interp = P.freq_scale * theta_extrap;
    float theta = theta_interp;
    float mscale = P.attn_factor;
    if (P.ext_factor != 0.0f) {
        // cuda/rope.cu:130-133 ramp, then the YaRN mix
        const float y = ((float)((2 * t) / 2) - P.corr_low) / fmaxf(0.001f, P.corr_high - P.corr_low);
        const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * P.ext_factor;
        theta = theta_interp * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / P.freq_scale);
    }
    c_out = cosf(theta) * mscale;
    s_out = P.sin_sign * sinf(theta) * mscale;
}
__device__ inline void rope_apply(float x0, float x1, float c, float s, float &y0, float &y1) {
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}
__device__ inline void rope_pair(float x0, float x1, int t, int pos, const RopeParams &P, float &y0, float &y1) {
    float c, s;
    rope_cs(t, pos, P, c, s);
    rope_apply(x0, x1, c, s, y0, y1);
}

}  // namespace ds4hip
