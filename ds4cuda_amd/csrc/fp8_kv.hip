// fp8_kv.hip — FP8 E4M3FN KV quantizer for gfx950.
//
// One 64-lane wave quantizes one 512-dim row: lane t owns dims [8t, 8t+8),
// so a 64-element scale block is 8 adjacent lanes and its max |x| is three
// DPP-class xor shuffles. The encoder is the exact bit-level
// round-to-nearest-even of ds4hip_common.h, not a table search. Loads and
// stores are 32 B / 16 B / 8 B per lane and fully coalesced per row.
//
// Two entry points:
//   * round trip (reference launcher, cuda/fp8_kv.cuh:62): fp32 in, fake-quant
//     fp32 out, tail copied through;
//   * append: writes the cache layout used by the decode kernels —
//     codes u8 [row][n_nope], scale exponents i8 [row][8] (7 used + 1 zero pad),
//     tail f16 [row][n_rot] — at caller-chosen physical rows.

#include "ds4hip_common.h"
#include "../../include/ds4hip.h"

using namespace ds4hip;

namespace {

constexpr int kRowsPerBlock = 4;   // 256 threads, 64 lanes per 512-dim row

// head_dim = 8 * lanes_per_row; lanes_per_row <= 64 and a multiple of 8.
template <bool kRoundTrip>
__global__ __launch_bounds__(256) void fp8_rows_kernel(
        const float *__restrict__ kv_in, float *__restrict__ kv_out,
        uint8_t *__restrict__ codes, int8_t *__restrict__ sexp, uint16_t *__restrict__ tail,
        int n_rows, int head_dim, int n_rot, long long row0,
        const long long *__restrict__ dst_rows) {
    const int lanes_per_row = head_dim >> 3;
    const int rows_per_block = 256 / 64;
    const int sub = threadIdx.x >> 6;              // row slot in the block
    const int t = threadIdx.x & 63;                // lane within the row
    const int row = blockIdx.x * rows_per_block + sub;
    if (row >= n_rows || t >= lanes_per_row) return;
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

    const long long prow = dst_rows ? dst_rows[row] : row0 + row;
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

bool shape_ok(int head_dim, int n_rot) {
    return head_dim > 0 && head_dim <= 512 && head_dim % 64 == 0 && n_rot >= 0 &&
           n_rot % 8 == 0 && n_rot < head_dim && (head_dim - n_rot) % 64 == 0 &&
           (head_dim - n_rot) / 64 <= 8;
}

}  // namespace

extern "C" int ds4hip_fp8_kv_quantize_round_trip_f32(const float *kv_in, float *kv_out,
                                                     int n_rows, int head_dim, int n_rot,
                                                     void *stream) {
    if (n_rows < 0 || !shape_ok(head_dim, n_rot) || (n_rows > 0 && (!kv_in || !kv_out)))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    const int grid = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(fp8_rows_kernel<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       kv_in, kv_out, nullptr, nullptr, nullptr, n_rows, head_dim, n_rot, 0LL,
                       nullptr);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_fp8_kv_quantize_append(const float *kv_in, int n_rows, int head_dim,
                                             int n_rot, uint8_t *codes, int8_t *sexp,
                                             uint16_t *tail, long long row0,
                                             const long long *dst_rows, void *stream) {
    if (n_rows < 0 || !shape_ok(head_dim, n_rot) || row0 < 0 ||
        (n_rows > 0 && (!kv_in || !codes || !sexp || (n_rot > 0 && !tail))))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    const int grid = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(fp8_rows_kernel<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       kv_in, nullptr, codes, sexp, tail, n_rows, head_dim, n_rot, row0,
                       dst_rows);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
