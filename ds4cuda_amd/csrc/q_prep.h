// q_prep.h — the FP8 form of one decode query as the producer lanes of the
// flat-stage decode kernel (flash_attn.hip) use it, shared by that kernel, by
// ds4hip_flash_attn_q_prep_f32 and by the per-token prologue kernel
// (rope_matvec.hip): a layer's query converted ahead of its decode leaves the
// decode's producers one load instead of the conversion, with the same bits.
#pragma once

#include "ds4hip_common.h"

namespace ds4hip {

__device__ inline float qp_pow2f(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// max over lanes l, l^16, l^32, l^48
__device__ inline float qp_xmax_16_32(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// One k-step of q_prep_lane (below): qf8[part][w] and the E8M0 scale byte
// sc[part] of k-step ks.
template <bool kQf32, bool kLean>
__device__ inline void q_prep_ks(const void *qrow, int q, int ks, uint32_t (&qf8)[kQf32 ? 3 : 2][8],
                                 int (&sc)[kQf32 ? 3 : 2]) {
    constexpr int kParts = kQf32 ? 3 : 2;
    const uint16_t *qsrc = static_cast<const uint16_t *>(qrow);
    const float *qsrc32 = static_cast<const float *>(qrow);
    float x[32];
#pragma unroll
    for (int hv = 0; hv < 2; ++hv) {
        const bool live = ks < 3 || hv == 0;
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int off = 128 * ks + 64 * hv + 16 * q + 8 * v;
            if constexpr (kQf32) {
                float4_t a = float4_t{0, 0, 0, 0}, b = a;
                if (live) {
                    a = *reinterpret_cast<const float4_t *>(qsrc32 + off);
                    b = *reinterpret_cast<const float4_t *>(qsrc32 + off + 4);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[16 * hv + 8 * v + i] = a[i];
                    x[16 * hv + 8 * v + 4 + i] = b[i];
                }
            } else {
                uint4_t w = uint4_t{0, 0, 0, 0};
                if (live) w = *reinterpret_cast<const uint4_t *>(qsrc + off);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[16 * hv + 8 * v + 2 * i] = bf16_to_f32((uint16_t)(w[i] & 0xFFFF));
                    x[16 * hv + 8 * v + 2 * i + 1] = bf16_to_f32((uint16_t)(w[i] >> 16));
                }
            }
        }
    }
#pragma unroll
    for (int part = 0; part < kParts; ++part) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
        amax = qp_xmax_16_32(amax);   // one scale for the head's 128 dims
        // scale 2^e with amax / 2^e in [128, 256): no E4M3 overflow
        int e = amax > 0.0f ? ((int)((__float_as_uint(amax) >> 23) & 0xFF) - 127 - 7) : 0;
        if constexpr (kLean) e = max(e, -126);
        const float inv = qp_pow2f(-e), scl = qp_pow2f(e);
        sc[part] = e + (kLean ? 126 : 127);
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            int pk = 0;
            pk = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w] * inv, x[4 * w + 1] * inv, pk, false);
            pk = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * w + 2] * inv, x[4 * w + 3] * inv, pk, true);
            qf8[part][w] = (uint32_t)pk;
            if (part < kParts - 1) {   // the residual goes to the next part
                x[4 * w] -= __builtin_amdgcn_cvt_f32_fp8(pk, 0) * scl;
                x[4 * w + 1] -= __builtin_amdgcn_cvt_f32_fp8(pk, 1) * scl;
                x[4 * w + 2] -= __builtin_amdgcn_cvt_f32_fp8(pk, 2) * scl;
                x[4 * w + 3] -= __builtin_amdgcn_cvt_f32_fp8(pk, 3) * scl;
            }
        }
    }
}

// The f16 tail fragments of q_prep_lane (dims 448 + 32 s2 + 8 q + [0, 8)).
template <bool kQf32>
__device__ inline void q_prep_tail(const void *qrow, int q, half8_t (&qt)[2], half8_t (&qtl)[2]) {
    const uint16_t *qsrc = static_cast<const uint16_t *>(qrow);
    const float *qsrc32 = static_cast<const float *>(qrow);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        half8_t h;
        if constexpr (kQf32) {
            const float4_t a = *reinterpret_cast<const float4_t *>(qsrc32 + 448 + 32 * s2 + 8 * q);
            const float4_t b = *reinterpret_cast<const float4_t *>(qsrc32 + 448 + 32 * s2 + 8 * q + 4);
            half8_t l;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = (half_t)a[i];
                l[i] = (half_t)(a[i] - (float)h[i]);
                h[4 + i] = (half_t)b[i];
                l[4 + i] = (half_t)(b[i] - (float)h[4 + i]);
            }
            qtl[s2] = l;
        } else {
            const uint4_t w = *reinterpret_cast<const uint4_t *>(qsrc + 448 + 32 * s2 + 8 * q);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[2 * i] = (half_t)bf16_to_f32((uint16_t)(w[i] & 0xFFFF));
                h[2 * i + 1] = (half_t)bf16_to_f32((uint16_t)(w[i] >> 16));
            }
        }
        qt[s2] = h;
    }
}

// Q of head 16 d + j (lane (j, q), j = lane & 15, q = lane >> 4) as the B
// operand of the scaled FP8 MFMA. k-step ks covers dims 128 ks + [0, 128);
// the MFMA takes lane (j, q)'s 32 bytes as dims 128 ks + 16 q + [0, 16) and
// 128 ks + 64 + 16 q + [0, 16) (lane q supplies the scale of dims 128 ks +
// 32 q + [0, 32)). Q ~ sum of kParts E4M3 parts, each with one E8M0 scale per
// head and k-step (a bf16 value has 8 significant bits: two parts hold it;
// an fp32 value takes three, about 12 bits). Dims >= 448 (the f16 RoPE tail)
// are zero here and take the f16 MFMA instead: qt[s] = dims 448 + 32 s + 8 q
// + [0, 8) (an fp32 Q: f16 hi qt + lo qtl; one f16 rounding there would
// dominate the error of the three parts). qrow: the head's 512 elements
// (bf16 bits or fp32). qsc[part] byte ks: the E8M0 scale of k-step ks.
// kLean: the cache rows' E8M0 scales are 2^(e_row + 1), so Q's scale carries
// the compensating 2^-1.
template <bool kQf32, bool kLean>
__device__ inline void q_prep_lane(const void *qrow, int q, uint32_t (&qf8)[4][kQf32 ? 3 : 2][8],
                                   int (&qsc)[kQf32 ? 3 : 2], half8_t (&qt)[2], half8_t (&qtl)[2]) {
    constexpr int kParts = kQf32 ? 3 : 2;
#pragma unroll
    for (int part = 0; part < kParts; ++part) qsc[part] = 0;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        int sc[kParts];
        q_prep_ks<kQf32, kLean>(qrow, q, ks, qf8[ks], sc);
#pragma unroll
        for (int part = 0; part < kParts; ++part) qsc[part] |= sc[part] << (8 * ks);
    }
    q_prep_tail<kQf32>(qrow, q, qt, qtl);
}

// The converted fp32 query of one problem in memory: kQPrepVecs 16-byte
// vectors per producer lane (lane index 64 d + lane), vector-major
// ([vec][256 lanes], so each vector is one coalesced 4 KB row): per part
// 0..2, k-steps 0-2 as two vectors and k-step 3's lower half as one (its
// upper half is zeros), then {qsc[0], qsc[1], qsc[2], 0}, then qt[0], qt[1],
// qtl[0], qtl[1].
constexpr int kQPrepVecs = 26;
constexpr int kQPrepLanes = 256;
constexpr long long kQPrepWords = (long long)kQPrepVecs * kQPrepLanes * 4;   // 32-bit words per problem

__device__ inline void q_prep_store(uint4_t *dst, int lane256, const uint32_t (&qf8)[4][3][8], const int (&qsc)[3],
                                    const half8_t (&qt)[2], const half8_t (&qtl)[2]) {
    int v = 0;
#pragma unroll
    for (int part = 0; part < 3; ++part)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int h = 0; h < (ks < 3 ? 2 : 1); ++h)
                dst[(v++) * kQPrepLanes + lane256] = uint4_t{qf8[ks][part][4 * h], qf8[ks][part][4 * h + 1],
                                                             qf8[ks][part][4 * h + 2], qf8[ks][part][4 * h + 3]};
    dst[(v++) * kQPrepLanes + lane256] = uint4_t{(uint32_t)qsc[0], (uint32_t)qsc[1], (uint32_t)qsc[2], 0u};
    dst[(v++) * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qt[0]);
    dst[(v++) * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qt[1]);
    dst[(v++) * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qtl[0]);
    dst[(v++) * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qtl[1]);
}

__device__ inline void q_prep_load(const uint4_t *src, int lane256, uint32_t (&qf8)[4][3][8], int (&qsc)[3],
                                   half8_t (&qt)[2], half8_t (&qtl)[2]) {
    uint4_t r[kQPrepVecs];
#pragma unroll
    for (int v = 0; v < kQPrepVecs; ++v) r[v] = src[v * kQPrepLanes + lane256];
    int v = 0;
#pragma unroll
    for (int part = 0; part < 3; ++part)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint4_t w = (ks < 3 || h == 0) ? r[v++] : uint4_t{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < 4; ++i) qf8[ks][part][4 * h + i] = w[i];
            }
#pragma unroll
    for (int part = 0; part < 3; ++part) qsc[part] = (int)r[v][part];
    ++v;
    qt[0] = __builtin_bit_cast(half8_t, r[v++]);
    qt[1] = __builtin_bit_cast(half8_t, r[v++]);
    qtl[0] = __builtin_bit_cast(half8_t, r[v++]);
    qtl[1] = __builtin_bit_cast(half8_t, r[v++]);
}

// The stored form written by parts (q_prep_store's layout): one k-step's
// vectors and scale bytes, or the tail vectors with the scale vector's
// unused word. Together they write exactly what q_prep_store writes.
__device__ inline void q_prep_store_ks(uint4_t *dst, int lane256, int ks, const uint32_t (&qf8)[3][8],
                                       const int (&sc)[3]) {
#pragma unroll
    for (int part = 0; part < 3; ++part) {
        const int v0 = 7 * part + 2 * ks;
        dst[v0 * kQPrepLanes + lane256] = uint4_t{qf8[part][0], qf8[part][1], qf8[part][2], qf8[part][3]};
        if (ks < 3)
            dst[(v0 + 1) * kQPrepLanes + lane256] = uint4_t{qf8[part][4], qf8[part][5], qf8[part][6], qf8[part][7]};
        reinterpret_cast<uint8_t *>(&dst[21 * kQPrepLanes + lane256])[4 * part + ks] = (uint8_t)sc[part];
    }
}
__device__ inline void q_prep_store_tail(uint4_t *dst, int lane256, const half8_t (&qt)[2], const half8_t (&qtl)[2]) {
    reinterpret_cast<uint32_t *>(&dst[21 * kQPrepLanes + lane256])[3] = 0u;
    dst[22 * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qt[0]);
    dst[23 * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qt[1]);
    dst[24 * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qtl[0]);
    dst[25 * kQPrepLanes + lane256] = __builtin_bit_cast(uint4_t, qtl[1]);
}

}  // namespace ds4hip
