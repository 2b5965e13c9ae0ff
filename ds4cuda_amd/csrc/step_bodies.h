// step_bodies.h — device bodies shared by a kernel of its own and by the
// fused per-token prologue kernel (rope_matvec.hip), so both run the same
// instructions: the FP8 row quantizer (fp8_kv.hip) and the compressor's
// projection rows (compressor.hip).
#pragma once

#include "ds4hip_common.h"

namespace ds4hip {

// One 512-dim (or smaller) row by 64 lanes (lane t: dims [8t, 8t+8)), into
// cache row prow (append) or into kv_out row `row` (round trip).
template <bool kRoundTrip>
__device__ inline void fp8_row_body(const float *__restrict__ kv_in, float *__restrict__ kv_out,
                                    uint8_t *__restrict__ codes, int8_t *__restrict__ sexp,
                                    uint16_t *__restrict__ tail, int row, int head_dim, int n_rot,
                                    long long prow, int t) {
    const int n_nope = head_dim - n_rot;
    const int d0 = t * 8;

    const float4_t *src = reinterpret_cast<const float4_t *>(kv_in + (size_t)row * head_dim + d0);
    float4_t a = src[0], b = src[1];
    float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};

    const bool is_nope = d0 < n_nope;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
    // reduce over the 8 lanes of this 64-dim block (all 8 lanes are in the
    // same class because n_nope is a multiple of 64)
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));

    if (is_nope) {
        const int e = fp8_block_exp(amax);
        uint32_t c[8];
        float q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = ldexpf(x[i], -e);                 // x / 2^e, exact division by a power of two
            v = fminf(fmaxf(v, -448.0f), 448.0f);
            c[i] = e4m3_encode(v);
            if (kRoundTrip) {
                // value of the code times the scale: rebuild from the code bits
                const uint32_t mag = c[i] & 0x7Fu;
                float val;
                if (mag < 8) {
                    val = (float)mag * 0.001953125f;
                } else {
                    const uint32_t bits = ((mag >> 3) + 120u) << 23 | (mag & 7u) << 20;
                    __builtin_memcpy(&val, &bits, 4);
                }
                q[i] = ldexpf((c[i] & 0x80u) ? -val : val, e);
            }
        }
        if (kRoundTrip) {
            float4_t *dst = reinterpret_cast<float4_t *>(kv_out + (size_t)row * head_dim + d0);
            dst[0] = float4_t{q[0], q[1], q[2], q[3]};
            dst[1] = float4_t{q[4], q[5], q[6], q[7]};
        } else {
            uint2_t packed;
            packed[0] = c[0] | c[1] << 8 | c[2] << 16 | c[3] << 24;
            packed[1] = c[4] | c[5] << 8 | c[6] << 16 | c[7] << 24;
            *reinterpret_cast<uint2_t *>(codes + (size_t)prow * n_nope + d0) = packed;
            if ((t & 7) == 0) sexp[(size_t)prow * 8 + (d0 >> 6)] = (int8_t)e;
            // without a tail, the lane of dim 0 zeroes the unused scale slots
            if (n_rot == 0 && d0 == 0)
                for (int s = n_nope / 64; s < 8; ++s) sexp[(size_t)prow * 8 + s] = 0;
        }
    } else {
        if (kRoundTrip) {
            float4_t *dst = reinterpret_cast<float4_t *>(kv_out + (size_t)row * head_dim + d0);
            dst[0] = a;
            dst[1] = b;
        } else {
            uint4_t h;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                h[i] = (uint32_t)f32_to_f16_bits(x[2 * i]) | (uint32_t)f32_to_f16_bits(x[2 * i + 1]) << 16;
            *reinterpret_cast<uint4_t *>(tail + (size_t)prow * n_rot + (d0 - n_nope)) = h;
            // zero the unused scale slots once per row
            if (d0 == n_nope)
                for (int s = n_nope / 64; s < 8; ++s) sexp[(size_t)prow * 8 + s] = 0;
        }
    }
}

constexpr int kCompMaxIn = 8192;   // compressor input dims staged in LDS
constexpr int kCpRows = 1;

// Rows [4 vblock, 4 vblock + 4) of the two projections (rows [0, width) of
// w_kv, then [0, width) of w_gate), one per wave, over the staged input xs:
// eight 16-byte weight chunks per lane in flight (wave_rows_dot), then the APE
// row and the state row (cuda/compressor.cu:78-110).
template <bool kW32>
__device__ inline void comp_project_rows(const float *xs, const void *__restrict__ w_kv,
                                         const void *__restrict__ w_gate, const uint16_t *__restrict__ w_ape,
                                         int in_dim, int width, int ratio, int pos_mod,
                                         float *__restrict__ state_kv, float *__restrict__ state_score,
                                         float *__restrict__ kv_cur, float *__restrict__ sc_cur, int vblock) {
    const int lane = threadIdx.x & 63;
    const int r0 = (vblock * 4 + (threadIdx.x >> 6)) * kCpRows;   // rows of [0, 2*width)
    if (r0 >= 2 * width) return;
    const void *rows[kCpRows];
#pragma unroll
    for (int k = 0; k < kCpRows; ++k) {
        const int r = min(r0 + k, 2 * width - 1);
        const bool gate = r >= width;
        const size_t o = (size_t)(gate ? r - width : r) * in_dim;
        rows[k] = kW32 ? static_cast<const void *>(static_cast<const float *>(gate ? w_gate : w_kv) + o)
                       : static_cast<const void *>(static_cast<const uint16_t *>(gate ? w_gate : w_kv) + o);
    }
    float acc[kCpRows] = {0.0f};
    wave_rows_dot<kCpRows, 8, kW32>(rows, xs, in_dim, lane, acc);
#pragma unroll
    for (int k = 0; k < kCpRows; ++k) {
        float a = acc[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
        const int r = r0 + k;
        if (lane == 0 && r < 2 * width) {
            const bool gate = r >= width;
            const int o = gate ? r - width : r;
            const int row = ratio == 4 ? ratio + pos_mod : pos_mod;   // cuda/compressor.cu:85
            const size_t off = (size_t)row * width + o;
            if (gate) {
                const float s = a + f16_bits_to_f32(w_ape[(size_t)pos_mod * width + o]);
                state_score[off] = s;
                if (sc_cur) sc_cur[o] = s;
            } else {
                state_kv[off] = a;
                if (kv_cur) kv_cur[o] = a;
            }
        }
    }
}

// Row r of src [n][width] fp32 to row dst_rows[r] of dst, by one 64-lane
// wave (lane t: 16-byte chunks t, t + 64, ...). width % 4 == 0.
__device__ inline void row_copy_body(const float *__restrict__ src, int r, int width, float *__restrict__ dst,
                                     const long long *__restrict__ dst_rows, int t) {
    const float4_t *s = reinterpret_cast<const float4_t *>(src + (size_t)r * width);
    float4_t *d = reinterpret_cast<float4_t *>(dst + (size_t)dst_rows[r] * width);
    for (int i = t; i < width / 4; i += 64) d[i] = s[i];
}

}  // namespace ds4hip
