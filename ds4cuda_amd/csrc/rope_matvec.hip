// rope_matvec.hip — tail RoPE YaRN (forward / inverse) and the matvecs of the
// attention path: f16 x fp32 (compressor / indexer projections), Q8_0 x Q8_0
// grouped and dense (attention output chain), bf16 x fp32 batched (the
// forward_batch output projection).
//
// RoPE (cuda/rope.cu:114-259, cuda/attn_out.cu:54-107,207-251): the per-layer
// YaRN parameters and theta_scale = powf(base, -2/n_rot) are computed on the
// host, so every caller sees the same fp32 constants; each pair thread then
// forms theta_extrap = pos * theta_scale^k by the same sequential fp32
// multiplications as the reference. One 64-lane wave rotates one head's
// 32 pairs (lanes 32..63 copy the untouched dims when out != in).
//
// Matvecs are weight-bandwidth bound: one wave per output row, 16-byte
// loads, activations staged once per workgroup in LDS, fp32 accumulation and
// a wave reduction. The Q8_0 dot products use v_dot4_i32_iu8 on int8 pairs,
// exact in int32, scaled per 32-element block as the reference does.

#include "ds4hip_common.h"
#include "step_bodies.h"
#include "q_prep.h"
#include "rope.h"
#include "../../include/ds4hip.h"

#include <algorithm>
#include <cmath>

using namespace ds4hip;

namespace {

// ---- tail RoPE YaRN ---------------------------------------------------------------

// pos_dev (optional): position per group of heads_per_pos consecutive heads.
__global__ __launch_bounds__(64) void rope_tail_kernel(const float *__restrict__ x_in,
                                                       float *__restrict__ x_out, int head_dim,
                                                       int n_rot, int pos, RopeParams P,
                                                       const int *__restrict__ pos_dev,
                                                       int heads_per_pos) {
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    if (pos_dev) pos = pos_dev[head / heads_per_pos];
    const int n_nope = head_dim - n_rot;
    const float *xi = x_in + (size_t)head * head_dim;
    float *xo = x_out + (size_t)head * head_dim;
    const int half = n_rot / 2;
    if (xi != xo)
        for (int d = t; d < n_nope; d += 64) xo[d] = xi[d];
    if (t >= half) return;
    float y0, y1;
    rope_pair(xi[n_nope + 2 * t], xi[n_nope + 2 * t + 1], t, pos, P, y0, y1);
    xo[n_nope + 2 * t] = y0;
    xo[n_nope + 2 * t + 1] = y1;
}

int launch_rope(const float *x_in, float *x_out, int n_heads, int head_dim, int n_rot, int pos,
                int il, bool inverse, hipStream_t st, const int *pos_dev = nullptr,
                int heads_per_pos = 1) {
    if (!x_in || !x_out || n_heads < 0 || head_dim <= 0 || n_rot <= 0 || n_rot > 128 ||
        (n_rot & 1) || n_rot > head_dim)
        return kEINVAL;
    if (n_heads == 0) return 0;
    const RopeParams P = rope_params(n_rot, il, inverse);
    hipLaunchKernelGGL(rope_tail_kernel, dim3(n_heads), dim3(64), 0, st, x_in, x_out, head_dim,
                       n_rot, pos, P, pos_dev, heads_per_pos);
    return hip_status(hipGetLastError());
}

// ---- wave reduction helpers ----------------------------------------------------------

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// ---- f16 x fp32 matvec (cuda/router.cu:69-97) -----------------------------------------
// 256 threads = 4 waves, 2 rows per wave; x staged in LDS as fp32.
constexpr int kMvMaxIn = 16384;

// One wave per 4 rows (16 rows per workgroup): every weight chunk of the four
// rows is loaded before the fmas that use it, and each x value read from LDS
// serves the four rows (wave_rows_dot). Lane-strided fp32 partial sums, then
// the wave's butterfly, as cuda/router.cu:69-97 reduces a warp's lanes.
constexpr int kMvRows = 4;
// Epilogues (each the arithmetic of the separate launch it replaces, so the
// results are bit-identical to that pair of launches):
//   kMvPlain: y = W x;
//   kMvScale: y = (W x) * scale (the indexer's head weights, then
//             ds4hip_scale_inplace_f32);
//   kMvRope:  y = W x, then the forward tail RoPE of every head of head_dim
//             rows (the indexer query, then ds4hip_tail_rope_yarn_f32): a
//             wave's four rows hold two whole pairs, rotated before the store.
enum { kMvPlain = 0, kMvScale = 1, kMvRope = 2 };
struct MvEpilogue {
    float scale = 1.0f;
    int head_dim = 0, n_rot = 0, pos = 0;
    RopeParams P{};
};
// Rows [4 kRows vblock, 4 kRows (vblock + 1)) of y = W x over the staged
// input xs (kRows per wave, kUnroll chunks of each in flight), with the
// epilogue kEpi (kMvRope: kRows even). Each row's sum is the same for any
// kRows and kUnroll: a lane takes chunks lane, lane + 64, ... in that order.
template <int kEpi, int kRows = kMvRows, int kUnroll = 2>
__device__ inline void mv_f16_rows(const float *xs, const uint16_t *__restrict__ w, float *__restrict__ y,
                                   int out_dim, int in_dim, const MvEpilogue &E, int vblock) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (vblock * 4 + wave) * kRows;
    if (row0 >= out_dim) return;
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = 0.0f;
    if ((in_dim & 7) == 0) {
        const void *rows[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) rows[r] = w + (size_t)min(row0 + r, out_dim - 1) * in_dim;
        wave_rows_dot<kRows, kUnroll, false>(rows, xs, in_dim, lane, acc);
    } else {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const uint16_t *wr = w + (size_t)min(row0 + r, out_dim - 1) * in_dim;
            for (int i = lane; i < in_dim; i += 64) acc[r] = fmaf(f16_bits_to_f32(wr[i]), xs[i], acc[r]);
        }
    }
    float a[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) a[r] = wave_sum(acc[r]);
    if (kEpi == kMvScale) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) a[r] = a[r] * E.scale;
    }
    if (kEpi == kMvRope) {
        const int d0 = row0 % E.head_dim, n_nope = E.head_dim - E.n_rot;
#pragma unroll
        for (int r = 0; r < kRows; r += 2)
            if (d0 + r >= n_nope) rope_pair(a[r], a[r + 1], (d0 + r - n_nope) / 2, E.pos, E.P, a[r], a[r + 1]);
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r)
        if (lane == 0 && row0 + r < out_dim) y[row0 + r] = a[r];
}

template <int kEpi>
__global__ __launch_bounds__(256) void mv_f16_kernel(const uint16_t *__restrict__ w,
                                                     const float *__restrict__ x,
                                                     float *__restrict__ y, int out_dim,
                                                     int in_dim, MvEpilogue E) {
    extern __shared__ __attribute__((aligned(16))) float xs[];
    stage_to_lds(xs, x, in_dim);
    __syncthreads();
    mv_f16_rows<kEpi>(xs, w, y, out_dim, in_dim, E, blockIdx.x);
}

// ---- Q8_0 activation quantization (cuda/attn_out.cu:119-145, dense_q8.cu) ---------------
// One 32-lane half-wave per 32-element block: amax, d = amax/127, id = 1/d,
// q = clamp(rint(x*id), -128, 127); the scale is kept fp32 as the reference does.
__global__ __launch_bounds__(256) void q8_quant_kernel(const float *__restrict__ x,
                                                       int8_t *__restrict__ xq,
                                                       float *__restrict__ xscale, int n_blocks) {
    const int b = (blockIdx.x * 256 + threadIdx.x) >> 5;
    const int l = threadIdx.x & 31;
    if (b >= n_blocks) return;
    const float v = x[(size_t)b * 32 + l];
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    const float d = a / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q = (int)__builtin_rintf(v * id);
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    xq[(size_t)b * 32 + l] = (int8_t)q;
    if (l == 0) xscale[b] = d;
}

// ---- Q8_0 x Q8_0 matvec --------------------------------------------------------------------
// Weight rows of n_blocks 34-byte blocks (f16 d + 32 int8). Lane l of a wave
// handles blocks l, l+64, ...: it reads the 34 bytes with 2-byte-aligned
// loads, the quantized activations from LDS, and accumulates
// sum_b (d_w * d_x) * isum_b with isum_b an exact int32 dot product.
// Rows of group g = row / rank read activation group g (cuda/attn_out.cu:171-174).
__device__ inline int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// One wave per row. With an even block count (rows of n_blocks * 34 bytes stay
// 4-byte aligned) a lane takes a pair of blocks, 68 bytes = 17 dwords, with
// dword loads (two pairs per lane in flight): the f16 scale and the int8
// values of the even block start at bytes 0 and 2 of the pair, those of the odd
// block at bytes 66 and 34. Otherwise a lane reads one block as 17 halfwords.
// Per block: the exact int32 dot of the int8 values, scaled by d_w * d_x in
// fp32 (cuda/attn_out.cu:171-197).
__device__ inline float q8_block_term(float dw, float dx, const uint32_t *q, const int *xb) {
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) isum = dot4((int)q[k], xb[k], isum);
    return dw * dx * (float)isum;
}

// kR rows per wave, all their weight loads in flight before any is used;
// row r's sum is accumulated exactly as with one row per wave.
template <int kR>
__device__ inline void q8_rows(const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
                               const float *__restrict__ xscale, const int (&row)[kR], int n_blocks, int rank,
                               int grouped, int lane, float (&out)[kR]) {
    const int8_t *xg[kR];
    const float *sg[kR];
    const uint8_t *wr[kR];
    float acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int g = grouped ? row[r] / rank : 0;
        xg[r] = xq + (size_t)g * n_blocks * 32;
        sg[r] = xscale + (size_t)g * n_blocks;
        wr[r] = W + (size_t)row[r] * n_blocks * 34;
        acc[r] = 0.0f;
    }
    if ((n_blocks & 1) == 0 && (reinterpret_cast<uintptr_t>(W) & 3) == 0) {
        const int n_pairs = n_blocks / 2;
        for (int p0 = lane; p0 < n_pairs; p0 += 128) {
            uint32_t d[kR][2][17];
#pragma unroll
            for (int r = 0; r < kR; ++r)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int p = min(p0 + 64 * u, n_pairs - 1);
                    const uint32_t *wp = reinterpret_cast<const uint32_t *>(wr[r]);
#pragma unroll
                    for (int k = 0; k < 17; ++k) d[r][u][k] = wp[(size_t)p * 17 + k];
                }
#pragma unroll
            for (int r = 0; r < kR; ++r)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int p = p0 + 64 * u;
                    if (p >= n_pairs) break;
                    const int b = 2 * p;
                    uint32_t qe[8], qo[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        qe[k] = __builtin_amdgcn_alignbyte(d[r][u][k + 1], d[r][u][k], 2);   // bytes 2 + 4k ..
                        qo[k] = d[r][u][k + 9];
                    }
                    const float dwe = f16_bits_to_f32((uint16_t)(d[r][u][0] & 0xFFFF));
                    const float dwo = f16_bits_to_f32((uint16_t)(d[r][u][8] >> 16));
                    acc[r] += q8_block_term(dwe, sg[r][b], qe, reinterpret_cast<const int *>(xg[r] + (size_t)b * 32));
                    acc[r] += q8_block_term(dwo, sg[r][b + 1], qo,
                                            reinterpret_cast<const int *>(xg[r] + (size_t)(b + 1) * 32));
                }
        }
    } else {
#pragma unroll
        for (int r = 0; r < kR; ++r)
            for (int b = lane; b < n_blocks; b += 64) {
                const uint16_t *blk = reinterpret_cast<const uint16_t *>(wr[r] + (size_t)b * 34);
                const float dw = f16_bits_to_f32(blk[0]);
                uint32_t q[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) q[k] = (uint32_t)blk[1 + 2 * k] | ((uint32_t)blk[2 + 2 * k] << 16);
                acc[r] += q8_block_term(dw, sg[r][b], q, reinterpret_cast<const int *>(xg[r] + (size_t)b * 32));
            }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) out[r] = wave_sum(acc[r]);
}

__global__ __launch_bounds__(256) void mv_q8_kernel(const uint8_t *__restrict__ W,
                                                    const int8_t *__restrict__ xq,
                                                    const float *__restrict__ xscale,
                                                    float *__restrict__ y, int n_rows,
                                                    int n_blocks, int rank, int grouped) {
    const int lane = threadIdx.x & 63;
    const int row[1] = {(int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)};
    if (row[0] >= n_rows) return;
    float acc[1];
    q8_rows<1>(W, xq, xscale, row, n_blocks, rank, grouped, lane, acc);
    if (lane == 0) y[row[0]] = acc[0];
}

// mv_q8_kernel and q8_quant_kernel of its output in one launch: a workgroup
// of 32 / kRpw waves computes 32 consecutive rows (kRpw per wave), then
// quantizes them as one Q8_0 block (q8_quant_kernel's arithmetic) into yq /
// yscale. n_rows a multiple of 32.
constexpr int kQuantRpw = 2;   // rows per wave (1024-thread workgroups)
template <int kRpw>
__global__ __launch_bounds__(64 * 32 / kRpw) void mv_q8_quant_kernel(const uint8_t *__restrict__ W,
                                                                     const int8_t *__restrict__ xq,
                                                                     const float *__restrict__ xscale,
                                                                     int8_t *__restrict__ yq,
                                                                     float *__restrict__ yscale, int n_blocks,
                                                                     int rank, int grouped) {
    __shared__ float s_y[32];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int row[kRpw];
#pragma unroll
    for (int r = 0; r < kRpw; ++r) row[r] = (int)blockIdx.x * 32 + kRpw * wave + r;
    float acc[kRpw];
    q8_rows<kRpw>(W, xq, xscale, row, n_blocks, rank, grouped, lane, acc);
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < kRpw; ++r) s_y[kRpw * wave + r] = acc[r];
    __syncthreads();
    if (threadIdx.x >= 32) return;
    const int l = threadIdx.x;
    const float v = s_y[l];
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    const float d = a / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q = (int)__builtin_rintf(v * id);
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    yq[(size_t)blockIdx.x * 32 + l] = (int8_t)q;
    if (l == 0) yscale[blockIdx.x] = d;
}

// Steps 14 + 15a in one launch: the inverse tail RoPE of a head's attention
// output and the Q8_0 quantization of the rotated row (one workgroup per
// head, thread t on dims 2t and 2t + 1; a 32-dim block is 16 threads). The
// rotation is rope_tail_kernel's and the quantization q8_quant_kernel's, in
// registers, so the int8 values and scales equal those of the two launches.
__global__ __launch_bounds__(256) void rope_q8_kernel(const float *__restrict__ x, int8_t *__restrict__ xq,
                                                      float *__restrict__ xscale, int head_dim, int n_rot,
                                                      int pos, RopeParams P) {
    const int head = blockIdx.x;
    const int t = threadIdx.x;
    const int d = 2 * t;
    if (d >= head_dim) return;
    const float *xi = x + (size_t)head * head_dim;
    float v0 = xi[d], v1 = xi[d + 1];
    const int n_nope = head_dim - n_rot;
    if (d >= n_nope) rope_pair(v0, v1, (d - n_nope) / 2, pos, P, v0, v1);
    float a = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 16));
    const float dq = a / 127.0f;
    const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
    int q0 = (int)__builtin_rintf(v0 * id), q1 = (int)__builtin_rintf(v1 * id);
    q0 = q0 > 127 ? 127 : (q0 < -128 ? -128 : q0);
    q1 = q1 > 127 ? 127 : (q1 < -128 ? -128 : q1);
    const size_t o = (size_t)head * head_dim + d;
    xq[o] = (int8_t)q0;
    xq[o + 1] = (int8_t)q1;
    if ((t & 15) == 0) xscale[o / 32] = dq;
}

int launch_q8(const uint8_t *W, const float *x, float *y, int n_groups, int group_dim, int rank,
              int8_t *xq, float *xs, bool grouped, hipStream_t st) {
    const int bpg = group_dim / 32;
    const int nb_total = n_groups * bpg;
    hipLaunchKernelGGL(q8_quant_kernel, dim3((nb_total * 32 + 255) / 256), dim3(256), 0, st, x,
                       xq, xs, nb_total);
    int e = hip_status(hipGetLastError());
    if (e) return e;
    const int n_rows = grouped ? n_groups * rank : rank;
    hipLaunchKernelGGL(mv_q8_kernel, dim3((n_rows + 3) / 4), dim3(256), 0, st, W, xq, xs, y,
                       n_rows, bpg, rank, grouped ? 1 : 0);
    return hip_status(hipGetLastError());
}

// ---- RMSNorm (cuda/norm.cu) and the decode Q / KV producer chain ---------------------------
// (cuda/forward_layer.cu:827-913, Steps 3-10). RMSNorm: one 256-thread block
// per row; thread t accumulates x[i]^2 for i = t, t + 256, ... in order, the
// wave sums are added in wave order, scale = 1 / sqrtf(ss / n + eps) and
// y = x * scale * w (w NULL: unit gain), the reference's operation order.
constexpr float kRmsEps = 1.0e-6f;

__device__ inline float block_sum_256(float v, float *part) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = v;
    __syncthreads();
    return ((part[0] + part[1]) + part[2]) + part[3];
}

__global__ __launch_bounds__(256) void rms_norm_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ w, int weight_dim,
                                                       float *__restrict__ y, int n, float eps) {
    __shared__ float part[4];
    const int row = blockIdx.x;
    const float *xr = x + (size_t)row * n;
    float *yr = y + (size_t)row * n;
    const float *wr = weight_dim == 0 ? nullptr : (weight_dim == n ? w : w + (size_t)row * n);
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    const float scale = 1.0f / sqrtf(block_sum_256(ss, part) / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) yr[i] = wr ? xr[i] * scale * wr[i] : xr[i] * scale;
}

// RMSNorm of one row of n = 256 k elements (weight w), then the Q8_0
// activation quantization of the normed row (the q_b matvec's input): element
// i = t + 256 k sits in thread t, so each 32-element block is one half-wave.
__global__ __launch_bounds__(256) void norm_q8_kernel(const float *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      float *__restrict__ y, int8_t *__restrict__ xq,
                                                      float *__restrict__ xscale, int n, float eps) {
    __shared__ float part[4];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(x[i], x[i], ss);
    const float scale = 1.0f / sqrtf(block_sum_256(ss, part) / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = x[i] * scale * w[i];
        y[i] = v;
        float a = fabsf(v);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
        const float d = a / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int q = (int)__builtin_rintf(v * id);
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        xq[i] = (int8_t)q;
        if ((threadIdx.x & 31) == 0) xscale[i >> 5] = d;
    }
}

// Per-head RMSNorm over 512 dims (optional weight shared by the heads), then
// the tail RoPE of dims 448..511: one wave per head, lane l holds dims
// 8 l .. 8 l + 7 (so lanes 56..63 hold the 32 rotated pairs, 4 each).
__global__ __launch_bounds__(64) void head_norm_rope_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ w,
                                                            float *__restrict__ y, int pos,
                                                            RopeParams P, float eps) {
    constexpr int kHd = 512, kNope = 448;
    const int l = threadIdx.x;
    const float *xr = x + (size_t)blockIdx.x * kHd + 8 * l;
    float *yr = y + (size_t)blockIdx.x * kHd + 8 * l;
    float v[8];
    const float4_t a = *reinterpret_cast<const float4_t *>(xr);
    const float4_t b = *reinterpret_cast<const float4_t *>(xr + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
    const float scale = 1.0f / sqrtf(wave_sum(ss) / (float)kHd + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = w ? v[i] * scale * w[8 * l + i] : v[i] * scale;
    if (8 * l >= kNope) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            rope_pair(v[2 * i], v[2 * i + 1], (8 * l - kNope) / 2 + i, pos, P, v[2 * i], v[2 * i + 1]);
    }
    *reinterpret_cast<float4_t *>(yr) = float4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<float4_t *>(yr + 4) = float4_t{v[4], v[5], v[6], v[7]};
}

// Workspace of the decode producer chain, 256-byte aligned pieces.
struct QkvWs {
    int8_t *xq;       // [4096] attn_norm as int8
    float *xs;        // [128]
    float *q_lora;    // [1024]
    float *kv_raw;    // [512]
    int8_t *xq2;      // [1024] q_lora_norm as int8
    float *xs2;       // [32]
    float *q_raw;     // [64 * 512]
    size_t bytes;
};
constexpr int kEmbd = 4096, kQLora = 1024, kKvDim = 512, kQDim = 64 * 512;

QkvWs qkv_ws(void *base) {   // base NULL: only the size is wanted
    auto al = [](size_t n) { return (n + 255) & ~size_t(255); };
    static uint8_t size_only[1];
    uint8_t *p = base ? static_cast<uint8_t *>(base) : size_only;
    QkvWs W;
    size_t o = 0;
    W.xq = reinterpret_cast<int8_t *>(p + o); o += al(kEmbd);
    W.xs = reinterpret_cast<float *>(p + o); o += al(kEmbd / 32 * 4);
    W.q_lora = reinterpret_cast<float *>(p + o); o += al(kQLora * 4);
    W.kv_raw = reinterpret_cast<float *>(p + o); o += al(kKvDim * 4);
    W.xq2 = reinterpret_cast<int8_t *>(p + o); o += al(kQLora);
    W.xs2 = reinterpret_cast<float *>(p + o); o += al(kQLora / 32 * 4);
    W.q_raw = reinterpret_cast<float *>(p + o); o += al((size_t)kQDim * 4);
    W.bytes = o;
    return W;
}

// ---- bf16 batched matvec / skinny GEMM: Y[b][r] = sum_c W[r][c] X[b][c] -----------------
// For the forward_batch output projection (16 sequences x 32768 -> 4096). Each
// wave owns 16 output rows; v_mfma_f32_16x16x32_bf16 with A = W rows (16 rows
// x 32 cols per step, read straight from HBM) and B = X^T from LDS. X is split
// into bf16 hi + lo parts (two MFMAs) so the activations keep ~16 mantissa
// bits. Column chunks (split-K) are summed in a fixed order (deterministic).
// n_batch <= 16, n_cols % 32 == 0.
typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));

// Batched projection Y[b][r] = sum_c W[r][c] X[b][c] for n_batch <= 16,
// streamed: weight-bandwidth bound, every weight is read once. One wave owns
// 64 rows (4 MFMA row tiles) and a k-range of kslice columns; lane (i, q)
// loads 8 consecutive columns of W row 16t+i and of X row i per 32-column
// step, so the four row tiles share one B fragment. bf16 W: X is split into
// bf16 hi + lo on the fly and multiplied with v_mfma_f32_16x16x32_bf16 twice
// (~16 bits of X kept); fp32 W: v_mfma_f32_16x16x4f32 on the exact fp32 values,
// element j of the 8 columns feeding MFMA step j. Each workgroup's k-range
// (k-group) stores a partial; the k-groups are summed in order afterwards.
template <bool kF32W>
struct MmFrag {
    float4_t xa, xb;           // X[batch i][8 columns]
    float4_t wa[4], wb[4];     // fp32 W: 8 columns of the 4 rows
    bf16x8_t w[4];             // bf16 W: 8 columns of the 4 rows
};

template <bool kF32W>
__device__ inline void mm_load(MmFrag<kF32W> &f, const void *Wv, const float *xr,
                               const size_t *roff, int k) {
    f.xa = *reinterpret_cast<const float4_t *>(xr + k);
    f.xb = *reinterpret_cast<const float4_t *>(xr + k + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (kF32W) {
            const float *W = static_cast<const float *>(Wv) + roff[t] + k;
            f.wa[t] = *reinterpret_cast<const float4_t *>(W);
            f.wb[t] = *reinterpret_cast<const float4_t *>(W + 4);
        } else {
            f.w[t] = *reinterpret_cast<const bf16x8_t *>(static_cast<const uint16_t *>(Wv) +
                                                         roff[t] + k);
        }
    }
}

template <bool kF32W>
__device__ inline void mm_compute(const MmFrag<kF32W> &f, bool bok, float4_t *acc) {
    const float4_t xa = bok ? f.xa : float4_t{0, 0, 0, 0};
    const float4_t xb = bok ? f.xb : float4_t{0, 0, 0, 0};
    if (kF32W) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.wa[t][j], xa[j], acc[t], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.wb[t][j], xb[j], acc[t], 0, 0, 0);
        }
    } else {
        // X = hi + lo in bf16 (hardware round-to-nearest-even conversions)
        bf16x8_t xh, xl;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float v0 = e < 4 ? xa[e] : xb[e - 4];
            const float v1 = e < 4 ? xa[e + 1] : xb[e - 3];
            const bf16x2_t h = bf16x2_t{(__bf16)v0, (__bf16)v1};
            const bf16x2_t l = bf16x2_t{(__bf16)(v0 - (float)h[0]), (__bf16)(v1 - (float)h[1])};
            const short2_t hs = __builtin_bit_cast(short2_t, h), ls = __builtin_bit_cast(short2_t, l);
            xh[e] = hs[0];
            xh[e + 1] = hs[1];
            xl[e] = ls[0];
            xl[e + 1] = ls[1];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.w[t], xh, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.w[t], xl, acc[t], 0, 0, 0);
        }
    }
}

// grid.z selects the (W, Y) pair (MmMats, below). The four
// waves of a workgroup take the same 64 rows and four consecutive k-slices;
// their partial sums are added in LDS in wave order, and the workgroup stores
// the k-group's partial to Y + blockIdx.y * n_batch * n_rows (no atomics): the
// k-groups are summed afterwards in k order, so the result is the same on
// every run.
// Up to four matrices over the same X and column count, one per blockIdx.z,
// each with its own row count and k-slice (workgroups past a matrix's row
// tiles or k-groups exit at once).
struct MmMats {
    const void *W[4];
    float *Y[4];
    int n_rows[4];
    int ks[4];
};

template <bool kF32W>
__global__ __launch_bounds__(256) void mm_stream_kernel(const MmMats M, const float *__restrict__ X, int n_cols,
                                                        int n_batch) {
    constexpr int kDepth = 4;   // 32-column steps in flight
    __shared__ float4_t red[4][4][64];   // [wave][row tile][lane]
    const void *Wv = M.W[blockIdx.z];
    float *Y = M.Y[blockIdx.z];
    const int n_rows = M.n_rows[blockIdx.z];
    const int kslice = M.ks[blockIdx.z];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 64;
    if (r0 >= n_rows || (long long)blockIdx.y * 4 * kslice >= n_cols) return;   // workgroup-uniform
    const int i = lane & 15, q = lane >> 4;
    const int k0 = (blockIdx.y * 4 + wave) * kslice;
    const int k1 = min(k0 + kslice, n_cols);
    const bool bok = i < n_batch;
    float4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = float4_t{0, 0, 0, 0};
    if (k0 < n_cols) {
        const float *xr = X + (size_t)(bok ? i : 0) * n_cols + 8 * q;
        size_t roff[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) roff[t] = (size_t)min(r0 + 16 * t + i, n_rows - 1) * n_cols + 8 * q;
        // steps past k1 re-read the last step (never used)
        auto clampk = [&](int k) { return k < k1 ? k : k1 - 32; };
        MmFrag<kF32W> f[kDepth];
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            mm_load(f[u], Wv, xr, roff, clampk(k0 + 32 * u));
            __builtin_amdgcn_sched_barrier(0);   // issue order = use order
        }
        for (int k = k0; k < k1; k += 32 * kDepth) {
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                // past k1 the fragment is a re-read of the last step: X is zeroed
                // instead of branching, so the load pipeline never drains
                mm_compute(f[u], bok && k + 32 * u < k1, acc);
                mm_load(f[u], Wv, xr, roff, clampk(k + 32 * (u + kDepth)));
                // keeps each refill where it is: otherwise the compiler sinks
                // the loads next to their use and the ring drains
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    // wave w adds row tile w of the four partials: D[row 4q+r of tile][batch i]
    const float4_t sum = ((red[0][wave][lane] + red[1][wave][lane]) + red[2][wave][lane]) + red[3][wave][lane];
    if (!bok) return;
    float *Yp = Y + (size_t)blockIdx.y * n_batch * n_rows + (size_t)i * n_rows;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int rr = r0 + 16 * wave + 4 * q + r;
        if (rr < n_rows) Yp[rr] = sum[r];
    }
}

// Y[j] = sum over k-groups g = 0 .. n_kg-1 of P[g * n + j], in g order.
__global__ __launch_bounds__(256) void mm_reduce_kernel(const float *__restrict__ P,
                                                        float *__restrict__ Y, size_t n,
                                                        int n_kg) {
    for (size_t j = (size_t)blockIdx.x * 256 + threadIdx.x; j < n; j += (size_t)gridDim.x * 256) {
        float acc = P[j];
        for (int g = 1; g < n_kg; ++g) acc += P[(size_t)g * n + j];
        Y[j] = acc;
    }
}

// k-slice so that the launch has about 2048 waves (two per SIMD; a multiple
// of 128 columns).
int mm_kslice(int n_rows, int n_cols, int n_mats) {
    const long long groups = (long long)n_mats * ((n_rows + 63) / 64);
    long long ks = (long long)n_cols * groups / 2048;
    ks = ((ks + 127) / 128) * 128;
    if (ks < 128) ks = 128;
    if (ks > n_cols) ks = ((n_cols + 31) / 32) * 32;
    return (int)ks;
}

template <bool kF32W>
int mm_launch_mats(const MmMats &M, int n_mats, const float *X, int n_cols, int n_batch, hipStream_t st) {
    int max_rows = 0, max_kg = 0;
    for (int z = 0; z < n_mats; ++z) {
        max_rows = std::max(max_rows, M.n_rows[z]);
        max_kg = std::max(max_kg, (n_cols + 4 * M.ks[z] - 1) / (4 * M.ks[z]));
    }
    const dim3 grid((max_rows + 63) / 64, max_kg, n_mats);
    hipLaunchKernelGGL(mm_stream_kernel<kF32W>, grid, dim3(256), 0, st, M, X, n_cols, n_batch);
    return hip_status(hipGetLastError());
}

template <bool kF32W>
int mm_launch(const void *W, const float *X, float *part, int n_rows, int n_cols, int n_batch,
              hipStream_t st, const void *W2 = nullptr, float *part2 = nullptr) {
    const int n_mats = W2 ? 2 : 1;
    MmMats M = {};
    M.W[0] = W;
    M.Y[0] = part;
    M.n_rows[0] = n_rows;
    M.W[1] = W2;
    M.Y[1] = part2;
    M.n_rows[1] = n_rows;
    M.ks[0] = M.ks[1] = mm_kslice(n_rows, n_cols, n_mats);
    return mm_launch_mats<kF32W>(M, n_mats, X, n_cols, n_batch, st);
}

// Projection into Y through k-group partials in ws (skipped when one k-group
// covers all columns: the kernel then writes Y itself).
template <bool kF32W>
int mm_full(const void *W, const float *X, float *Y, int n_rows, int n_cols, int n_batch,
            void *ws, size_t ws_bytes, hipStream_t st) {
    const int n_kg = ds4hip_mm_k_groups(n_rows, n_cols, 1);
    if (n_kg == 1) return mm_launch<kF32W>(W, X, Y, n_rows, n_cols, n_batch, st);
    const size_t n = (size_t)n_batch * n_rows;
    if (!ws || ws_bytes < (size_t)n_kg * n * sizeof(float)) return kEINVAL;
    float *P = static_cast<float *>(ws);
    int rc = mm_launch<kF32W>(W, X, P, n_rows, n_cols, n_batch, st);
    if (rc) return rc;
    hipLaunchKernelGGL(mm_reduce_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)),
                       dim3(256), 0, st, P, Y, n, n_kg);
    return hip_status(hipGetLastError());
}

}  // namespace

int ds4hip_mm_k_groups(int n_rows, int n_cols, int n_mats) {
    const int ks = mm_kslice(n_rows, n_cols, n_mats);
    return (n_cols + 4 * ks - 1) / (4 * ks);
}

int ds4hip_mm_f32_parts_mats(const float *const *W, float *const *part, const int *n_rows, const int *ks,
                             int n_mats, const float *X, int n_cols, int n_batch, hipStream_t st) {
    if (!W || !part || !n_rows || !ks || n_mats < 1 || n_mats > 4 || !X || n_cols <= 0 || n_cols % 32 ||
        n_batch <= 0 || n_batch > 16)
        return kEINVAL;
    MmMats M = {};
    for (int z = 0; z < n_mats; ++z) {
        if (!W[z] || !part[z] || n_rows[z] <= 0 || ks[z] <= 0 || ks[z] % 32) return kEINVAL;
        M.W[z] = W[z];
        M.Y[z] = part[z];
        M.n_rows[z] = n_rows[z];
        M.ks[z] = ks[z];
    }
    return mm_launch_mats<true>(M, n_mats, X, n_cols, n_batch, st);
}

int ds4hip_mm_kslice(int n_rows, int n_cols, int n_mats) { return mm_kslice(n_rows, n_cols, n_mats); }

int ds4hip_mm_f32_parts(const float *W, const float *X, float *part, int n_rows, int n_cols,
                        int n_batch, hipStream_t st, const float *W2, float *part2) {
    if (!W || !X || !part || n_rows <= 0 || n_cols <= 0 || n_cols % 32 || n_batch <= 0 ||
        n_batch > 16 || (!W2 != !part2))
        return kEINVAL;
    return mm_launch<true>(W, X, part, n_rows, n_cols, n_batch, st, W2, part2);
}

extern "C" size_t ds4hip_mul_mm_workspace_bytes(int n_rows, int n_cols, int n_batch) {
    if (n_rows <= 0 || n_cols <= 0 || n_batch <= 0) return 0;
    const int n_kg = ds4hip_mm_k_groups(n_rows, n_cols, 1);
    return n_kg == 1 ? 0 : (size_t)n_kg * n_batch * n_rows * sizeof(float);
}

extern "C" int ds4hip_mul_mm_f32_f32(const float *W, const float *X, float *Y, int n_rows,
                                     int n_cols, int n_batch, void *workspace,
                                     size_t workspace_bytes, void *stream) {
    if (!W || !X || !Y || n_rows <= 0 || n_cols <= 0 || n_cols % 32 || n_batch <= 0 ||
        n_batch > 16)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(mm_full<true>(W, X, Y, n_rows, n_cols, n_batch, workspace,
                                               workspace_bytes, (hipStream_t)stream));
}

extern "C" int ds4hip_tail_rope_yarn_batch_f32(const float *x_in, float *x_out, int n_seq,
                                               int n_heads, int head_dim, int n_rot,
                                               const int *pos_dev, int il, int inverse,
                                               void *stream) {
    if (n_seq < 0 || !pos_dev) return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(launch_rope(x_in, x_out, n_seq * n_heads, head_dim, n_rot, 0, il,
                                             inverse != 0, (hipStream_t)stream, pos_dev,
                                             n_heads > 0 ? n_heads : 1));
}

extern "C" int ds4hip_tail_rope_yarn_f32(const float *x_in, float *x_out, int n_heads,
                                         int head_dim, int n_rot, int pos, int il, void *stream) {
    return ds4hip_set_last_error(
        launch_rope(x_in, x_out, n_heads, head_dim, n_rot, pos, il, false, (hipStream_t)stream));
}

extern "C" int ds4hip_tail_rope_yarn_inverse_f32(const float *x_in, float *x_out, int n_heads,
                                                 int head_dim, int n_rot, int pos, int il,
                                                 void *stream) {
    return ds4hip_set_last_error(
        launch_rope(x_in, x_out, n_heads, head_dim, n_rot, pos, il, true, (hipStream_t)stream));
}

namespace {
template <int kEpi>
int launch_mv_f16(const uint16_t *w_f16, const float *x_f32, float *y_f32, int out_dim, int in_dim,
                  const MvEpilogue &E, hipStream_t st) {
    if (!w_f16 || !x_f32 || !y_f32 || out_dim < 0 || in_dim <= 0 || in_dim > kMvMaxIn) return kEINVAL;
    if (out_dim == 0) return 0;
    hipLaunchKernelGGL(mv_f16_kernel<kEpi>, dim3((out_dim + 4 * kMvRows - 1) / (4 * kMvRows)), dim3(256),
                       in_dim * sizeof(float), st, w_f16, x_f32, y_f32, out_dim, in_dim, E);
    return hip_status(hipGetLastError());
}
}  // namespace

extern "C" int ds4hip_mul_mv_f16_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32,
                                     int out_dim, int in_dim, void *stream) {
    return ds4hip_set_last_error(
        launch_mv_f16<kMvPlain>(w_f16, x_f32, y_f32, out_dim, in_dim, MvEpilogue{}, (hipStream_t)stream));
}

extern "C" int ds4hip_mul_mv_f16_scaled_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32,
                                            int out_dim, int in_dim, float scale, void *stream) {
    MvEpilogue E;
    E.scale = scale;
    return ds4hip_set_last_error(
        launch_mv_f16<kMvScale>(w_f16, x_f32, y_f32, out_dim, in_dim, E, (hipStream_t)stream));
}

extern "C" int ds4hip_mul_mv_f16_rope_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32,
                                          int n_heads, int head_dim, int n_rot, int pos, int il,
                                          int in_dim, void *stream) {
    // four rows per wave must hold whole pairs of one head's tail
    if (n_heads <= 0 || head_dim <= 0 || head_dim % 4 || n_rot <= 0 || n_rot > 128 || n_rot % 4 ||
        n_rot > head_dim)
        return ds4hip_set_last_error(kEINVAL);
    MvEpilogue E;
    E.head_dim = head_dim;
    E.n_rot = n_rot;
    E.pos = pos;
    E.P = rope_params(n_rot, il, false);
    return ds4hip_set_last_error(launch_mv_f16<kMvRope>(w_f16, x_f32, y_f32, n_heads * head_dim, in_dim, E,
                                                        (hipStream_t)stream));
}

extern "C" int ds4hip_mul_mv_q8_0_q8_0_grouped_f32_prealloc(const void *W, const float *x,
                                                            float *y, int n_groups,
                                                            int group_dim, int rank,
                                                            int8_t *scratch_xq,
                                                            float *scratch_xscale, void *stream) {
    if (!W || !x || !y || !scratch_xq || !scratch_xscale || n_groups <= 0 || rank <= 0 ||
        group_dim <= 0 || group_dim % 32)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(launch_q8(static_cast<const uint8_t *>(W), x, y, n_groups,
                                           group_dim, rank, scratch_xq, scratch_xscale, true,
                                           (hipStream_t)stream));
}

extern "C" int ds4hip_mul_mv_q8_0_q8_0_grouped_f32(const void *W, const float *x, float *y,
                                                   int n_groups, int group_dim, int rank,
                                                   void *stream) {
    if (!W || !x || !y || n_groups <= 0 || rank <= 0 || group_dim <= 0 || group_dim % 32)
        return ds4hip_set_last_error(kEINVAL);
    const hipStream_t st = (hipStream_t)stream;
    // the int8 activations and their scales live in the library's per-stream
    // scratch: the reference's launcher of this name allocates nothing per call
    const size_t n = (size_t)n_groups * group_dim;
    const size_t xs_off = (n + 255) & ~(size_t)255;
    void *buf = nullptr;
    const int e = stream_scratch(st, xs_off + n / 32 * sizeof(float), &buf);
    if (e) return ds4hip_set_last_error(e);
    int8_t *xq = static_cast<int8_t *>(buf);
    float *xs = reinterpret_cast<float *>(static_cast<char *>(buf) + xs_off);
    return ds4hip_set_last_error(launch_q8(static_cast<const uint8_t *>(W), x, y, n_groups,
                                           group_dim, rank, xq, xs, true, st));
}

extern "C" int ds4hip_mul_mv_q8_0_q8_0_f32_prealloc(const void *W, const float *x, float *y,
                                                    int n_rows, int n_cols, int8_t *scratch_xq,
                                                    float *scratch_xscale, void *stream) {
    if (!W || !x || !y || !scratch_xq || !scratch_xscale || n_rows <= 0 || n_cols <= 0 ||
        n_cols % 32)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(launch_q8(static_cast<const uint8_t *>(W), x, y, 1, n_cols,
                                           n_rows, scratch_xq, scratch_xscale, false,
                                           (hipStream_t)stream));
}

// Steps 14-16 of one token (cuda/forward_layer.cu:1172-1210): inverse tail
// RoPE + Q8_0 quantization (one launch), the grouped Q8_0 projection, the
// quantization of its output and the dense Q8_0 projection. The same values as
// ds4hip_tail_rope_yarn_inverse_f32 + the two _prealloc matvecs, one launch
// fewer. Workspace: ds4hip_attn_out_decode_workspace_bytes.
namespace {
struct AttnOutWs {
    int8_t *xq, *xq2;
    float *xs, *low, *xs2;
};
size_t attn_out_ws(int n_head, int head_dim, int n_groups, int rank, char *base, AttnOutWs *w) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t n = (size_t)n_head * head_dim, m = (size_t)n_groups * rank;
    size_t off = 0;
    const size_t o_xq = off; off += al(n);
    const size_t o_xs = off; off += al(n / 32 * sizeof(float));
    const size_t o_low = off; off += al(m * sizeof(float));
    const size_t o_xq2 = off; off += al(m);
    const size_t o_xs2 = off; off += al(m / 32 * sizeof(float));
    if (w) {
        w->xq = reinterpret_cast<int8_t *>(base + o_xq);
        w->xs = reinterpret_cast<float *>(base + o_xs);
        w->low = reinterpret_cast<float *>(base + o_low);
        w->xq2 = reinterpret_cast<int8_t *>(base + o_xq2);
        w->xs2 = reinterpret_cast<float *>(base + o_xs2);
    }
    return off;
}
}  // namespace

extern "C" size_t ds4hip_attn_out_decode_workspace_bytes(int n_head, int head_dim, int n_groups, int rank) {
    if (n_head <= 0 || head_dim <= 0 || n_groups <= 0 || rank <= 0) return 0;
    return attn_out_ws(n_head, head_dim, n_groups, rank, nullptr, nullptr);
}

namespace {
bool attn_out_shape_ok(int n_head, int head_dim, int n_groups, int rank, int out_dim) {
    return n_head > 0 && head_dim > 0 && head_dim % 32 == 0 && head_dim <= 512 && n_groups > 0 &&
           (n_head * head_dim) % n_groups == 0 && ((n_head * head_dim) / n_groups) % 32 == 0 && rank > 0 &&
           rank % 32 == 0 && out_dim > 0;
}
// Steps 15-16 from the quantized attention output: the grouped projection
// with the quantization of its output, then the dense one
void attn_out_projections(const int8_t *xq, const float *xs, const void *w_out_a, const void *w_out_b, float *out,
                          int n_head, int head_dim, int n_groups, int rank, int out_dim, const AttnOutWs &w,
                          hipStream_t st) {
    const int bpg = (n_head * head_dim) / n_groups / 32;
    const int n_low = n_groups * rank;
    hipLaunchKernelGGL(mv_q8_quant_kernel<kQuantRpw>, dim3(n_low / 32), dim3(64 * 32 / kQuantRpw), 0, st,
                       static_cast<const uint8_t *>(w_out_a), xq, xs, w.xq2, w.xs2, bpg, rank, 1);
    hipLaunchKernelGGL(mv_q8_kernel, dim3((out_dim + 3) / 4), dim3(256), 0, st, static_cast<const uint8_t *>(w_out_b),
                       w.xq2, w.xs2, out, out_dim, n_low / 32, out_dim, 0);
}
}  // namespace

extern "C" int ds4hip_attn_out_decode_f32(const float *kqv, const void *w_out_a, const void *w_out_b,
                                          float *out, int n_head, int head_dim, int n_rot, int pos, int il,
                                          int n_groups, int rank, int out_dim, void *workspace,
                                          size_t workspace_bytes, void *stream) {
    if (!kqv || !w_out_a || !w_out_b || !out || !workspace || !attn_out_shape_ok(n_head, head_dim, n_groups, rank, out_dim) ||
        n_rot <= 0 || n_rot > 128 || (n_rot & 1) || n_rot > head_dim ||
        workspace_bytes < attn_out_ws(n_head, head_dim, n_groups, rank, nullptr, nullptr))
        return ds4hip_set_last_error(kEINVAL);
    const hipStream_t st = (hipStream_t)stream;
    AttnOutWs w;
    attn_out_ws(n_head, head_dim, n_groups, rank, static_cast<char *>(workspace), &w);
    const RopeParams P = rope_params(n_rot, il, true);
    hipLaunchKernelGGL(rope_q8_kernel, dim3(n_head), dim3(256), 0, st, kqv, w.xq, w.xs, head_dim, n_rot, pos, P);
    attn_out_projections(w.xq, w.xs, w_out_a, w_out_b, out, n_head, head_dim, n_groups, rank, out_dim, w, st);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_attn_out_decode_q8_f32(const int8_t *xq, const float *xscale, const void *w_out_a,
                                             const void *w_out_b, float *out, int n_head, int head_dim, int n_groups,
                                             int rank, int out_dim, void *workspace, size_t workspace_bytes,
                                             void *stream) {
    if (!xq || !xscale || !w_out_a || !w_out_b || !out || !workspace ||
        !attn_out_shape_ok(n_head, head_dim, n_groups, rank, out_dim) ||
        workspace_bytes < attn_out_ws(n_head, head_dim, n_groups, rank, nullptr, nullptr))
        return ds4hip_set_last_error(kEINVAL);
    const hipStream_t st = (hipStream_t)stream;
    AttnOutWs w;
    attn_out_ws(n_head, head_dim, n_groups, rank, static_cast<char *>(workspace), &w);
    attn_out_projections(xq, xscale, w_out_a, w_out_b, out, n_head, head_dim, n_groups, rank, out_dim, w, st);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

// ---- per-token layer prologue: Steps 11-12c's independent launches as one --------------
//
// The launches of a layer step that depend only on the layer's inputs (the
// FP8 push of the token's KV row, the attention and the indexer compressor
// projections, the indexer query with its RoPE and the scaled head weights)
// run as one launch: its workgroup range is cut into the jobs' own grids, each
// job's workgroups run that job's body (the same device code as its own
// kernel, so the results are bit-identical), on the CUs at the same time
// instead of one launch after another.
namespace {
constexpr int kPrologueRot = 64;   // the model's RoPE tail (the session's row layout)
struct PrologueArgs {
    ds4hip_token_prologue a;
    // first workgroup of each job, in launch order: the query conversion (4
    // workgroups, one per k-step; first, as the longest chains), the push, the
    // head weights (one row per wave: a short chain), the projections, the
    // indexer query (blk_q + n_q = grid)
    int blk_push, blk_hw, blk_comp[2], blk_q;
    int width[2], pos_mod[2];
    MvEpilogue eq, ehw;
};

// xs: the staged input vector, sized by the launch to the longest one (a
// static 8192-float array would leave fewer workgroups per CU than the grid)
__global__ __launch_bounds__(256) void token_prologue_kernel(const PrologueArgs P) {
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const ds4hip_token_prologue &a = P.a;
    const int b = blockIdx.x;
    auto stage = [&](const float *x, int n) {
        stage_to_lds(xs, x, n);
        __syncthreads();
    };
    if (b < P.blk_push) {
        // the decode query, k-step b: producer lane (wave d, lane) of the flat
        // decode kernel; the k-step-3 workgroup also writes the f16 tail
        const int d = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const float *qrow = a.qp_q + (16 * d + (lane & 15)) * 512;
        uint4_t *dst = static_cast<uint4_t *>(a.qp_out);
        uint32_t qf8[3][8];
        int sc[3];
        q_prep_ks<true, true>(qrow, lane >> 4, b, qf8, sc);
        q_prep_store_ks(dst, threadIdx.x, b, qf8, sc);
        if (b == 3) {
            half8_t qt[2], qtl[2];
            q_prep_tail<true>(qrow, lane >> 4, qt, qtl);
            q_prep_store_tail(dst, threadIdx.x, qt, qtl);
        }
        return;
    }
    if (b < P.blk_hw) {   // the FP8 push: one 64-lane row
        if (threadIdx.x < 64)
            fp8_row_body<false>(a.kv, nullptr, a.codes, a.sexp, a.tail, 0, a.head_dim, a.n_rot, a.kv_row,
                                threadIdx.x);
        return;
    }
    if (b < P.blk_comp[0]) {
        stage(a.x, a.in_dim);
        mv_f16_rows<kMvScale, 1, 8>(xs, a.hw_w, a.hw_out, a.hw_rows, a.in_dim, P.ehw, b - P.blk_hw);
        return;
    }
    for (int c = 0; c < 2; ++c) {
        const int end = c == 0 ? P.blk_comp[1] : P.blk_q;
        if (b < end) {
            stage(a.x, a.in_dim);
            comp_project_rows<false>(xs, c ? a.comp1_w_kv : a.comp0_w_kv, c ? a.comp1_w_gate : a.comp0_w_gate,
                                     c ? a.comp1_w_ape : a.comp0_w_ape, a.in_dim, P.width[c],
                                     c ? a.comp1_ratio : a.comp0_ratio, P.pos_mod[c],
                                     c ? a.comp1_state_kv : a.comp0_state_kv,
                                     c ? a.comp1_state_score : a.comp0_state_score, nullptr, nullptr,
                                     b - P.blk_comp[c]);
            return;
        }
    }
    stage(a.q_x, a.q_in);
    mv_f16_rows<kMvRope>(xs, a.q_w, a.q_out, a.q_heads * a.q_head_dim, a.q_in, P.eq, b - P.blk_q);
}
}  // namespace

extern "C" int ds4hip_token_prologue_f32(const ds4hip_token_prologue *a, void *stream) {
    if (!a || !a->kv || !a->codes || !a->sexp || !a->tail || a->kv_row < 0 || a->head_dim != 512 ||
        a->n_rot != kPrologueRot || a->n_comp < 0 || a->n_comp > 2 ||
        ((a->n_comp || a->hw_w) && (!a->x || a->in_dim <= 0 || a->in_dim > kCompMaxIn || a->in_dim % 8)))
        return ds4hip_set_last_error(kEINVAL);
    PrologueArgs P = {};
    P.a = *a;
    int blk = 0;
    if (a->qp_q) {
        if (!a->qp_out || (reinterpret_cast<uintptr_t>(a->qp_q) | reinterpret_cast<uintptr_t>(a->qp_out)) % 16)
            return ds4hip_set_last_error(kEINVAL);
        blk += 4;
    }
    P.blk_push = blk;
    blk += 1;   // one workgroup: the FP8 push
    int xs_floats = 4;   // the longest staged vector
    if (a->n_comp || a->hw_w) xs_floats = std::max(xs_floats, a->in_dim);
    P.blk_hw = blk;
    if (a->hw_w) {
        if (!a->hw_out || a->hw_rows <= 0) return ds4hip_set_last_error(kEINVAL);
        P.ehw.scale = a->hw_scale;
        blk += (a->hw_rows + 3) / 4;   // one row per wave
    }
    const int ratio[2] = {a->comp0_ratio, a->comp1_ratio};
    const int hdo[2] = {a->comp0_head_dim_out, a->comp1_head_dim_out};
    const int pos[2] = {a->comp0_pos, a->comp1_pos};
    for (int c = 0; c < 2; ++c) {
        P.blk_comp[c] = blk;
        if (c >= a->n_comp) continue;
        const void *wk = c ? a->comp1_w_kv : a->comp0_w_kv, *wg = c ? a->comp1_w_gate : a->comp0_w_gate;
        const void *wa = c ? a->comp1_w_ape : a->comp0_w_ape;
        const float *sk = c ? a->comp1_state_kv : a->comp0_state_kv, *ss = c ? a->comp1_state_score : a->comp0_state_score;
        if (!wk || !wg || !wa || !sk || !ss || (ratio[c] != 4 && ratio[c] != 128) || hdo[c] <= 64 ||
            hdo[c] > 512 || hdo[c] % 64 || pos[c] < 0)
            return ds4hip_set_last_error(kEINVAL);
        P.width[c] = (ratio[c] == 4 ? 2 : 1) * hdo[c];
        P.pos_mod[c] = pos[c] % ratio[c];
        blk += (2 * P.width[c] + 4 * kCpRows - 1) / (4 * kCpRows);
    }
    P.blk_q = blk;
    if (a->q_w) {
        if (!a->q_x || !a->q_out || a->q_heads <= 0 || a->q_head_dim <= 0 || a->q_head_dim % 4 || a->q_in <= 0 ||
            a->q_in > kCompMaxIn || a->q_in % 8)
            return ds4hip_set_last_error(kEINVAL);
        P.eq.head_dim = a->q_head_dim;
        P.eq.n_rot = kPrologueRot;
        P.eq.pos = a->q_pos;
        P.eq.P = rope_params(kPrologueRot, a->q_il, false);
        blk += (a->q_heads * a->q_head_dim + 4 * kMvRows - 1) / (4 * kMvRows);
        xs_floats = std::max(xs_floats, a->q_in);
    }
    hipLaunchKernelGGL(token_prologue_kernel, dim3(blk), dim3(256), (size_t)xs_floats * sizeof(float),
                       (hipStream_t)stream, P);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_mul_mm_bf16_f32(const uint16_t *W, const float *X, float *Y, int n_rows,
                                      int n_cols, int n_batch, void *workspace,
                                      size_t workspace_bytes, void *stream) {
    if (!W || !X || !Y || n_rows <= 0 || n_cols <= 0 || n_cols % 32 || n_batch <= 0 ||
        n_batch > 16)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(mm_full<false>(W, X, Y, n_rows, n_cols, n_batch, workspace,
                                                workspace_bytes, (hipStream_t)stream));
}

extern "C" int ds4hip_rms_norm_f32(const float *x, const float *w, float *y, int n, float eps,
                                   void *stream) {
    if (!x || !w || !y || n <= 0) return ds4hip_set_last_error(kEINVAL);
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, x, w, n, y, n,
                       eps);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_rms_norm_batch_f32(const float *x, const float *w, int weight_dim, float *y,
                                         int n_rows, int n_per_row, float eps, void *stream) {
    if (!x || !y || n_rows < 0 || n_per_row <= 0 ||
        !(weight_dim == 0 || weight_dim == n_per_row || (long long)weight_dim == (long long)n_rows * n_per_row) ||
        (weight_dim && !w))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(n_rows), dim3(256), 0, (hipStream_t)stream, x, w,
                       weight_dim, y, n_per_row, eps);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" size_t ds4hip_attn_qkv_decode_workspace_bytes(void) { return qkv_ws(nullptr).bytes; }

extern "C" int ds4hip_attn_qkv_decode_f32(const float *attn_norm, const void *w_q_a,
                                          const float *w_q_a_norm, const void *w_kv_a,
                                          const float *w_kv_a_norm, const void *w_q_b, int pos,
                                          int il, float *q_lora_norm, float *q_cur, float *kv_rope,
                                          void *workspace, size_t workspace_bytes, void *stream) {
    if (!attn_norm || !w_q_a || !w_q_a_norm || !w_kv_a || !w_kv_a_norm || !w_q_b || !q_lora_norm ||
        !q_cur || !kv_rope || !workspace || pos < 0 || il < 0 ||
        workspace_bytes < ds4hip_attn_qkv_decode_workspace_bytes())
        return ds4hip_set_last_error(kEINVAL);
    const hipStream_t st = (hipStream_t)stream;
    const QkvWs W = qkv_ws(workspace);
    const uint8_t *qa = static_cast<const uint8_t *>(w_q_a);
    const uint8_t *kva = static_cast<const uint8_t *>(w_kv_a);
    const uint8_t *qb = static_cast<const uint8_t *>(w_q_b);
    // Steps 3 and 5: q_lora and KVraw from one quantization of attn_norm
    hipLaunchKernelGGL(q8_quant_kernel, dim3(kEmbd / 256), dim3(256), 0, st, attn_norm, W.xq, W.xs,
                       kEmbd / 32);
    hipLaunchKernelGGL(mv_q8_kernel, dim3(kQLora / 4), dim3(256), 0, st, qa, W.xq, W.xs, W.q_lora,
                       kQLora, kEmbd / 32, kQLora, 0);
    hipLaunchKernelGGL(mv_q8_kernel, dim3(kKvDim / 4), dim3(256), 0, st, kva, W.xq, W.xs, W.kv_raw,
                       kKvDim, kEmbd / 32, kKvDim, 0);
    // Step 4 with the quantization of Step 7's input; Steps 6 + 10
    hipLaunchKernelGGL(norm_q8_kernel, dim3(1), dim3(256), 0, st, W.q_lora, w_q_a_norm, q_lora_norm,
                       W.xq2, W.xs2, kQLora, kRmsEps);
    const RopeParams P = rope_params(64, il, false);
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3(1), dim3(64), 0, st, W.kv_raw, w_kv_a_norm,
                       kv_rope, pos, P, kRmsEps);
    // Step 7, then Steps 8 + 9
    hipLaunchKernelGGL(mv_q8_kernel, dim3(kQDim / 4), dim3(256), 0, st, qb, W.xq2, W.xs2, W.q_raw,
                       kQDim, kQLora / 32, kQDim, 0);
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3(64), dim3(64), 0, st, W.q_raw, nullptr, q_cur,
                       pos, P, kRmsEps);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
