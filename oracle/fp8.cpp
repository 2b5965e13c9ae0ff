// fp8.cpp — oracle: f16/bf16 scalar conversions and the E4M3FN KV quantizer.
// TEST INFRASTRUCTURE ONLY (see ds4_oracle.h).

#include "ds4_oracle.h"

#include <cmath>
#include <cstring>

static inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// IEEE binary32 -> binary16, round to nearest even, overflow -> inf, NaN kept
// quiet. Written from the IEEE 754 encoding definitions.
extern "C" uint16_t orc_f32_to_f16(float x) {
    const uint32_t u = f2u(x);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t ax = u & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       // inf / nan
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    const int e = (int)(ax >> 23) - 127;           // unbiased exponent
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;  // 24-bit significand
    if (ax < 0x00800000u) return sign;             // fp32 subnormal -> 0 (|x| < 2^-126)
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    int shift;                                      // bits to drop from 24-bit significand
    uint32_t base;
    if (e >= -14) {                                 // normal f16
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        mant &= 0x7FFFFFu;                          // drop hidden bit; carry handles rounding
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        const uint32_t h = base + r;                // mantissa carry bumps the exponent
        if (h >= 0x7C00u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | h);
    }
    // subnormal f16: value = m * 2^-24, m = round(|x| * 2^24)
    shift = 13 + (-14 - e);                         // >= 14
    if (shift > 24) return sign;                    // below half of the smallest subnormal
    uint32_t r = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);                    // r == 0x400 rolls into the smallest normal
}

extern "C" float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        const float v = std::ldexp((float)m, -24);
        return (h & 0x8000u) ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

extern "C" float orc_f16_round(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

extern "C" float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

extern "C" uint16_t orc_f32_to_bf16(float x) {
    const uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    const uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

// ---- E4M3FN ---------------------------------------------------------------

// Per-exponent scale of the E4M3FN table (cuda/fp8_kv.cu:75-80).
static const float kExpScale[16] = {
    0.0f,   0.015625f, 0.03125f, 0.0625f, 0.125f, 0.25f,  0.5f,   1.0f,
    2.0f,   4.0f,      8.0f,     16.0f,   32.0f,  64.0f,  128.0f, 256.0f,
};

// cuda/fp8_kv.cu:88-94
extern "C" float orc_e4m3fn_value(int i) {
    const int ex = (i >> 3) & 0xF;
    const int mant = i & 0x7;
    return ex == 0 ? (float)mant * 0.001953125f
                   : (1.0f + (float)mant * 0.125f) * kExpScale[ex];
}

// cuda/fp8_kv.cu:102-131: largest index with value <= ax, then step up when
// the upper neighbour is strictly closer or equally close with an even index.
extern "C" int orc_e4m3fn_nearest_index(float ax) {
    int lo = 0, hi = 126;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (orc_e4m3fn_value(mid) <= ax) lo = mid; else hi = mid - 1;
    }
    int best = lo;
    if (best < 126) {
        const float bd = std::fabs(ax - orc_e4m3fn_value(best));
        const float nd = std::fabs(ax - orc_e4m3fn_value(best + 1));
        if (nd < bd || (nd == bd && ((best + 1) & 1) == 0 && (best & 1) != 0)) ++best;
    }
    return best;
}

// cuda/fp8_kv.cu:174-176. log2 is evaluated in double and rounded to fp32,
// i.e. a correctly rounded fp32 log2 of the fp32 quotient amax/448; the
// quotient itself is an fp32 division (RNE).
extern "C" int orc_fp8_scale_exp(float amax) {
    const float a = amax > 1.0e-4f ? amax : 1.0e-4f;
    const float y = a / 448.0f;
    const float l = (float)std::log2((double)y);
    return (int)std::ceil(l);
}

extern "C" float orc_fp8_deq(uint8_t code, int e) {
    const float v = std::ldexp(orc_e4m3fn_value(code & 0x7F), e);
    return orc_f16_round((code & 0x80) ? -v : v);
}

// cuda/fp8_kv.cu:144-195 for one row.
extern "C" void orc_fp8_quant_row(const float *x, int head_dim, int n_rot,
                                  uint8_t *codes, int8_t *sexp, uint16_t *tail,
                                  float *deq) {
    const int n_nope = head_dim - n_rot;
    for (int off = 0, b = 0; off < n_nope; off += 64, ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 64; ++j) amax = std::fmax(amax, std::fabs(x[off + j]));
        const int e = orc_fp8_scale_exp(amax);
        const float scale = std::ldexp(1.0f, e);
        if (sexp) sexp[b] = (int8_t)e;
        for (int j = 0; j < 64; ++j) {
            const float xv = x[off + j];
            float v = xv / scale;
            v = std::fmin(std::fmax(v, -448.0f), 448.0f);
            const bool neg = v < 0.0f;
            const int idx = orc_e4m3fn_nearest_index(std::fmin(std::fabs(v), 448.0f));
            if (codes) codes[off + j] = (uint8_t)((neg ? 0x80 : 0) | idx);
            if (deq) {
                const float q = (neg ? -1.0f : 1.0f) * orc_e4m3fn_value(idx);
                deq[off + j] = q * scale;
            }
        }
    }
    for (int j = 0; j < n_rot; ++j) {
        if (deq) deq[n_nope + j] = x[n_nope + j];
        if (tail) tail[j] = orc_f32_to_f16(x[n_nope + j]);
    }
}

extern "C" void orc_fp8_quant_rows(const float *x, int n_rows, int head_dim, int n_rot,
                                   uint8_t *codes, int8_t *sexp, uint16_t *tail,
                                   float *deq) {
    const int n_nope = head_dim - n_rot;
    for (int r = 0; r < n_rows; ++r) {
        orc_fp8_quant_row(x + (size_t)r * head_dim, head_dim, n_rot,
                          codes ? codes + (size_t)r * n_nope : nullptr,
                          sexp ? sexp + (size_t)r * 8 : nullptr,
                          tail ? tail + (size_t)r * n_rot : nullptr,
                          deq ? deq + (size_t)r * head_dim : nullptr);
    }
}
