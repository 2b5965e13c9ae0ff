// ds4hip_common.h — shared device helpers for the gfx950 attention-path
// kernels: vector types, the exact E4M3FN encoder, the power-of-two scale
// rule, bf16/f16 conversions and the C-ABI error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ds4hip {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int uint4_t __attribute__((ext_vector_type(4)));
typedef unsigned int uint2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kEINVAL = -22;
constexpr int kHipErrBase = -1000;   // returned as kHipErrBase - hipError_t

// Scratch memory the library keeps per (device, stream) for entry points whose
// reference counterparts take no workspace (the fp32 decode launchers, the
// indexer top-k launchers): *out receives at least `bytes` of device memory
// owned by the library, reused by every later call on the same stream, so the
// steady state allocates nothing. It grows (stream-ordered free + allocation)
// only when a call needs more than any earlier one on that stream. Calls on one
// stream are ordered, so they never share it concurrently; distinct streams get
// distinct buffers. Returns 0 or a status.
int stream_scratch(hipStream_t stream, size_t bytes, void **out);

// ---- scale rule -------------------------------------------------------------
// The reference picks scale = 2^ceil(log2(amax/448)) per 64-element block
// (cuda/fp8_kv.cu:174-176). With log2 evaluated as a correctly rounded fp32
// function of the fp32 quotient y = fl(amax/448), ceil(fl(log2 y)) equals
//   k       when y = 2^k exactly,
//   k       when y = 2^k (1 + M 2^-23) and log2(1 + M 2^-23) is below half the
//           fp32 spacing next to k (fl(k + t) rounds back to k),
//   k + 1   otherwise.
// The rounding-back case only happens for a few mantissas M just above a power
// of two. For y in [2^-126, 2^127) the bound M <= limit(s) with
// s = -log2(half spacing) is the integer part of (2^(2^-s) - 1) 2^23:
//   s=18 -> 22, s=19 -> 11, s=20 -> 5, s=21 -> 2, s=22 -> 1, s>=23 -> 0.
// tests/test_fp8_rule.py checks this rule against ceil(float(log2(double y)))
// for every fp32 y in [2^-30, 2^30).
__host__ __device__ inline int floor_log2_u32(uint32_t a) {
    int r = 0;
    while (a >>= 1) ++r;
    return r;
}

__host__ __device__ inline int ceil_log2_cr(float y) {
    uint32_t u;
    __builtin_memcpy(&u, &y, 4);
    const int k = (int)((u >> 23) & 0xFF) - 127;
    const uint32_t M = u & 0x7FFFFFu;
    if (M == 0) return k;
    if (k == 0) return 1;
    int s;
    if (k > 0) {
        s = 24 - floor_log2_u32((uint32_t)k);
    } else {
        const uint32_t a = (uint32_t)(-k);
        const int fl = floor_log2_u32(a);
        s = ((a & (a - 1)) == 0) ? 25 - fl : 24 - fl;
    }
    uint32_t limit = 0;
    switch (s) {
    case 18: limit = 22; break;
    case 19: limit = 11; break;
    case 20: limit = 5; break;
    case 21: limit = 2; break;
    case 22: limit = 1; break;
    default: limit = s < 18 ? 0xFFFFFFFFu : 0; break;   // s < 18 unreachable for y < 2^127
    }
    return (M <= limit) ? k : k + 1;
}

// Scale exponent of one 64-block from its max |x| (floor 1e-4, fp8_kv.cu:175).
__host__ __device__ inline int fp8_block_exp(float amax) {
    const float a = amax > 1.0e-4f ? amax : 1.0e-4f;
    // fl(a / 448): the double quotient rounded to fp32 equals the fp32 quotient
    // because a / 7 never lies within 2^-53 of an fp32 rounding midpoint.
    const float y = (float)((double)a / 448.0);
    return ceil_log2_cr(y);
}

// ---- E4M3FN encoder -------------------------------------------------------------
// Nearest E4M3FN code of v, |v| <= 448, ties to the even code (the picker of
// cuda/fp8_kv.cu:102-131 is round-to-nearest-even in code space). Sign bit set
// when v < 0 (the reference takes the sign from v < 0, so -0 encodes as +0).
__host__ __device__ inline uint32_t e4m3_encode(float v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    const uint32_t sign = (v < 0.0f) ? 0x80u : 0u;
    const uint32_t au = u & 0x7FFFFFFFu;
    float av;
    __builtin_memcpy(&av, &au, 4);
    uint32_t mag;
    if (au < 0x3C800000u) {                    // |v| < 2^-6: subnormal codes m * 2^-9
        mag = (uint32_t)__builtin_rintf(av * 512.0f);   // exact scaling, RNE
    } else {
        const uint32_t e8 = au >> 23;          // >= 121
        const uint32_t m = au & 0x7FFFFFu;
        uint32_t r = m >> 20;
        const uint32_t rem = m & 0xFFFFFu;
        if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ++r;
        mag = ((e8 - 120u) << 3) + r;          // carry of r into the exponent is intended
    }
    return sign | mag;
}

// ---- conversions ------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

__device__ inline uint16_t f32_to_f16_bits(float x) {
    const half_t h = (half_t)x;                // v_cvt_f16_f32, RNE
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ inline float f16_bits_to_f32(uint16_t b) {
    half_t h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__host__ inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : kHipErrBase - (int)e; }


// x[0, n) into LDS xs by a 256-thread block: 16-byte loads, eight per thread
// issued before any is written, so a block pays one memory latency per 8192
// floats instead of one per 256 (a loop of dependent 4-byte copies). Ends
// without a barrier.
__device__ inline void stage_to_lds(float *xs, const float *x, int n) {
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(xs)) & 15) == 0 && (n & 3) == 0) {
        const int n4 = n >> 2;
        const float4_t *x4 = reinterpret_cast<const float4_t *>(x);
        float4_t *s4 = reinterpret_cast<float4_t *>(xs);
        for (int b = 0; b < n4; b += 256 * 8) {
            float4_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)   // clamped, not branched: no wait between the loads
                v[u] = x4[min(b + 256 * u + (int)threadIdx.x, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = b + 256 * u + (int)threadIdx.x;
                if (i < n4) s4[i] = v[u];
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += 256) xs[i] = x[i];
    }
}

// ---- wave-per-rows GEMV ---------------------------------------------------------
// acc[r] += dot(row r of W, x) for kRows rows held by one wave, x staged in LDS.
// Each lane reads 16-byte chunks (8 f16 or 4 fp32 weights) of every row at
// chunk index lane + 64 j; kUnroll chunks of each of the kRows rows are
// loaded before any is used, so a wave keeps kRows * kUnroll loads in flight
// and every x value read from LDS serves all kRows rows. in_dim must be a
// multiple of the chunk width. The per-lane sums are left to the caller's
// reduction (lane order is fixed, so results are reproducible).
template <int kRows, int kUnroll, bool kF32>
__device__ inline void wave_rows_dot(const void *const (&rows)[kRows], const float *xs, int in_dim, int lane,
                                     float (&acc)[kRows]) {
    constexpr int kPer = kF32 ? 4 : 8;
    const int n_chunks = in_dim / kPer;
    for (int c0 = lane; c0 < n_chunks; c0 += 64 * kUnroll) {
        uint4_t v[kRows][kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int r = 0; r < kRows; ++r)
                v[r][u] = c < n_chunks ? reinterpret_cast<const uint4_t *>(rows[r])[c] : uint4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + 64 * u;
            if (c >= n_chunks) break;
            float xv[kPer];
#pragma unroll
            for (int e = 0; e < kPer; ++e) xv[e] = xs[c * kPer + e];
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (kF32) {
                        acc[r] = fmaf(__uint_as_float(v[r][u][k]), xv[k], acc[r]);
                    } else {
                        acc[r] = fmaf(f16_bits_to_f32((uint16_t)(v[r][u][k] & 0xFFFF)), xv[2 * k], acc[r]);
                        acc[r] = fmaf(f16_bits_to_f32((uint16_t)(v[r][u][k] >> 16)), xv[2 * k + 1], acc[r]);
                    }
                }
            }
        }
    }
}

}  // namespace ds4hip

// Library-internal launchers shared between translation units (rope_matvec.hip).
// Batched fp32-weight projection Y[b][r] = sum_c W[r][c] X[b][c] (n_cols % 32
// == 0, n_batch <= 16) as k-group partials: k-group g writes
// part[g][b][r]; the caller sums the ds4hip_mm_k_groups(n_rows, n_cols,
// n_mats) groups in g order. (W2, part2): a second matrix of the same shape on
// the same X, in the same launch (n_mats = 2).
int ds4hip_mm_k_groups(int n_rows, int n_cols, int n_mats);
int ds4hip_mm_f32_parts(const float *W, const float *X, float *part, int n_rows, int n_cols,
                        int n_batch, hipStream_t st, const float *W2 = nullptr,
                        float *part2 = nullptr);
// The k-slice (columns per wave) ds4hip_mm_f32_parts uses for that shape, and
// up to four matrices of their own row counts and k-slices over one X in one
// launch (matrix z's partials exactly as a launch of it alone with ks[z]).
int ds4hip_mm_kslice(int n_rows, int n_cols, int n_mats);
int ds4hip_mm_f32_parts_mats(const float *const *W, float *const *part, const int *n_rows, const int *ks,
                             int n_mats, const float *X, int n_cols, int n_batch, hipStream_t st);

// Records the last failing status for the void-returning C++ shims.
extern "C" int ds4hip_set_last_error(int code);
