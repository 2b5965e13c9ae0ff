// indexer.hip — lightning-indexer scores and exact top-k selection.
//
// Scores (cuda/indexer_allowed.cu:68-171): score[c] = sum_h w[h] relu(q_h . k_c).
// The reference reduces in a warp-shuffle order and accepts ULP drift at the
// top-k boundary (cuda/indexer_allowed.cuh:64-66). Here the order is fixed so
// that the selected set is reproducible bit for bit: dot_h is an fma chain
// over d ascending from +0, then score = fma(w[h], relu(dot_h), score) over h
// ascending from +0. One thread scores one key: the key row (up to 128 dims)
// sits in registers as fp32, the 64 x 128 query in LDS (broadcast reads).
//
// Selection (cuda/indexer_allowed.cu:200-279): top_k rounds of argmax with
// ties to the lowest index select exactly the top_k entries in
// (score desc, index asc) order. This is computed as an exact radix select on
// order-preserving 32-bit keys (11 + 11 + 10 bits; histograms built by all
// workgroups with LDS + global atomics), which yields the threshold key T,
// the number above it and how many ties at T to take; one workgroup then
// walks the candidates in index order and emits the 0/1 mask or the
// ascending position list.

#include "ds4hip_common.h"
#include "../../include/ds4hip.h"

#include <algorithm>
#include <cstdlib>

using namespace ds4hip;

namespace {

constexpr int kMaxHeads = 64;
constexpr int kMaxDim = 128;
constexpr int kQStride = kMaxDim + 4;   // query row stride in LDS for the four-thread form
constexpr int kBins = 2048;

__device__ inline unsigned ord_key(float s) {
    unsigned u = __float_as_uint(s);
    if (u == 0x80000000u) u = 0;                 // -0 ranks as +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int kKind>   // 0 f32, 1 f16, 2 bf16
__device__ inline float key_elem(const void *keys, size_t i) {
    if (kKind == 0) return static_cast<const float *>(keys)[i];
    if (kKind == 1) return f16_bits_to_f32(static_cast<const uint16_t *>(keys)[i]);
    return bf16_to_f32(static_cast<const uint16_t *>(keys)[i]);
}

// Copies the n_head x 128 fp32 query into LDS with all loads issued before
// any store (a plain strided loop waits for each load in turn).
template <int kStride = kMaxDim>
__device__ inline void stage_query(float *qs, const float *q, int n_head) {
    if (reinterpret_cast<uintptr_t>(q) & 15) {   // unaligned caller buffer: plain copy
        for (int i = threadIdx.x; i < n_head * kMaxDim; i += 256)
            qs[(i / kMaxDim) * kStride + i % kMaxDim] = q[i];
        return;
    }
    const int n4 = n_head * kMaxDim / 4;
    float4_t v[kMaxHeads * kMaxDim / 4 / 256];
#pragma unroll
    for (int i = 0; i < kMaxHeads * kMaxDim / 4 / 256; ++i) {
        const int k = (int)threadIdx.x + 256 * i;
        v[i] = k < n4 ? reinterpret_cast<const float4_t *>(q)[k] : float4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < kMaxHeads * kMaxDim / 4 / 256; ++i) {
        const int k = (int)threadIdx.x + 256 * i;
        if (k < n4)
            *reinterpret_cast<float4_t *>(qs + (k / (kMaxDim / 4)) * kStride + 4 * (k % (kMaxDim / 4))) = v[i];
    }
}

// Zero heads of zero weight up to a multiple of 4 (they add +0 * 0 terms
// after the real heads, which leaves every score bit-identical).
__device__ inline void pad_heads(float *qs, float *ws, int n_head) {
    const int n4 = (n_head + 3) & ~3;
    for (int i = threadIdx.x; i < (n4 - n_head) * kMaxDim; i += 256) qs[n_head * kMaxDim + i] = 0.0f;
    if ((int)threadIdx.x < n4 - n_head) ws[n_head + threadIdx.x] = 0.0f;
}

// head_dim 128, one key per thread, the key row in registers as fp32 and the
// query and the weights in LDS: every multiply-add takes its query value from
// a broadcast 16-byte LDS read (in-order returns, so the reads run several
// steps ahead of their use). Two heads at a time: their dot chains are
// independent, and the chains and the head sum keep the canonical order.
template <int kKind>
__device__ __attribute__((always_inline)) inline float score_lds(const float *qs, const float *ws,
                                                                 const void *__restrict__ keys,
                                                                 int c, int n_head) {
    float k[kMaxDim];
    if (kKind == 0) {
        const float4_t *src = reinterpret_cast<const float4_t *>(
            static_cast<const float *>(keys) + (size_t)c * kMaxDim);
#pragma unroll
        for (int v = 0; v < kMaxDim / 4; ++v) {
            const float4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 4; ++e) k[4 * v + e] = u[e];
        }
    } else {
        const uint4_t *src = reinterpret_cast<const uint4_t *>(
            static_cast<const uint16_t *>(keys) + (size_t)c * kMaxDim);
#pragma unroll
        for (int v = 0; v < kMaxDim / 8; ++v) {
            const uint4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t h = (uint16_t)((u[e >> 1] >> (16 * (e & 1))) & 0xFFFF);
                k[8 * v + e] = kKind == 1 ? f16_bits_to_f32(h) : bf16_to_f32(h);
            }
        }
    }
    // four heads at a time: four independent dot chains keep the VALU busy
    // (n_head is padded to a multiple of 4 with zero heads of zero weight)
    float s = 0.0f;
    for (int h = 0; h < n_head; h += 4) {
        const float4_t *q0 = reinterpret_cast<const float4_t *>(qs + h * kMaxDim);
        float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < kMaxDim / 4; ++v) {
            float4_t a[4];
#pragma unroll
            for (int z = 0; z < 4; ++z) a[z] = q0[z * (kMaxDim / 4) + v];
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int z = 0; z < 4; ++z) d[z] = fmaf(a[z][e], k[4 * v + e], d[z]);
        }
#pragma unroll
        for (int z = 0; z < 4; ++z) s = fmaf(ws[h + z], d[z] > 0.0f ? d[z] : 0.0f, s);
    }
    return s;
}

// head_dim 128 with four threads per key (adjacent lanes): thread `part`
// holds dims [32 part, 32 part + 32) of the key and continues the dot chain of
// part - 1 (handed over by a lane shift), so every head's dot is still one fma
// chain over d ascending from +0, and part 3 runs the head sum in head order:
// bit-identical to the one-thread form, with a quarter of the key registers
// (several waves per SIMD hide the LDS latency of the query reads). In
// iteration i, part p works on head i - p. The query rows sit kQStride floats
// apart in LDS: with stride 128 the four parts' reads (offsets 32 p - 128 p)
// would fall on the same banks; 132 spreads them over four bank groups.
// load_key32 reads one part's dims.
template <int kKind>
__device__ inline void load_key32(const void *__restrict__ keys, int c, int part, float *k) {
    if (kKind == 0) {
        const float4_t *src = reinterpret_cast<const float4_t *>(
            static_cast<const float *>(keys) + (size_t)c * kMaxDim + 32 * part);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 4; ++e) k[4 * v + e] = u[e];
        }
    } else {
        const uint4_t *src = reinterpret_cast<const uint4_t *>(
            static_cast<const uint16_t *>(keys) + (size_t)c * kMaxDim + 32 * part);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t h = (uint16_t)((u[e >> 1] >> (16 * (e & 1))) & 0xFFFF);
                k[8 * v + e] = kKind == 1 ? f16_bits_to_f32(h) : bf16_to_f32(h);
            }
        }
    }
}

// Two keys (c0, c1) per group of four lanes: their chains are independent,
// which gives the VALU two dependency chains to interleave. Scores are valid
// in part 3.
template <int kKind>
__device__ __attribute__((always_inline)) inline void score_chain4x2(const float *qs, const float *ws,
                                                                     const void *__restrict__ keys,
                                                                     int c0, int c1, int n_head, int part,
                                                                     float &s0, float &s1) {
    float k0[32], k1[32];
    load_key32<kKind>(keys, c0, part, k0);
    load_key32<kKind>(keys, c1, part, k1);
    float carry0 = 0.0f, carry1 = 0.0f;
    s0 = 0.0f;
    s1 = 0.0f;
    for (int i = 0; i < n_head + 3; ++i) {
        const int h = i - part;
        const bool act = h >= 0 && h < n_head;
        const float4_t *qv = reinterpret_cast<const float4_t *>(qs + (act ? h : 0) * kQStride + 32 * part);
        float d0 = part == 0 ? 0.0f : carry0;
        float d1 = part == 0 ? 0.0f : carry1;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4_t a = qv[v];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                d0 = fmaf(a[e], k0[4 * v + e], d0);
                d1 = fmaf(a[e], k1[4 * v + e], d1);
            }
        }
        // lane l takes lane l-1's chains (row_shr:1; part 0 ignores them)
        carry0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d0), 0x111, 0xF, 0xF, false));
        carry1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d1), 0x111, 0xF, 0xF, false));
        if (part == 3 && act) {
            s0 = fmaf(ws[h], d0 > 0.0f ? d0 : 0.0f, s0);
            s1 = fmaf(ws[h], d1 > 0.0f ? d1 : 0.0f, s1);
        }
    }
}

// Any head_dim <= 128: the key row is zero-padded to 128 in registers and
// the query is read with the same padding from LDS.
template <int kKind>
__device__ inline float score_any(const float *qs, const float *ws, const void *keys, int c,
                                  int n_head, int head_dim) {
    float k[kMaxDim];
#pragma unroll
    for (int d = 0; d < kMaxDim; ++d)
        k[d] = d < head_dim ? key_elem<kKind>(keys, (size_t)c * head_dim + d) : 0.0f;
    float s = 0.0f;
    for (int h = 0; h < n_head; ++h) {
        const float *qh = qs + h * head_dim;
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < kMaxDim; ++d)
            if (d < head_dim) dot = fmaf(qh[d], k[d], dot);
        s = fmaf(ws[h], dot > 0.0f ? dot : 0.0f, s);
    }
    return s;
}

// kFull: head_dim == 128 (the scalar-load path); otherwise the LDS path. Two
// instantiations so that neither path's registers limit the other's occupancy.
template <int kKind, bool kFull>
__global__ __launch_bounds__(256) void score_kernel(const float *__restrict__ q,
                                                    const float *__restrict__ w,
                                                    const void *__restrict__ keys, int n_comp,
                                                    int n_head, int head_dim,
                                                    float *__restrict__ scores,
                                                    unsigned *__restrict__ hist, int n_cand) {
    __shared__ unsigned lh[kBins];
    if (hist)
        for (int i = threadIdx.x; i < kBins; i += 256) lh[i] = 0;
    __shared__ __attribute__((aligned(16))) float qs[kMaxHeads * kQStride];
    __shared__ float ws[kMaxHeads];
    if (kFull) {
        // one thread per key: the query staged once per 256 keys (the four-lane
        // chained form measures slower here, where a launch has many keys)
        const int c = blockIdx.x * 256 + threadIdx.x;
        float s = 0.0f;
        stage_query(qs, q, n_head);
        for (int i = threadIdx.x; i < n_head; i += 256) ws[i] = w[i];
        pad_heads(qs, ws, n_head);
        __syncthreads();
        if (c < n_comp) s = score_lds<kKind>(qs, ws, keys, c, n_head);
        if (c < n_comp) scores[c] = s;
        if (hist) {
            __syncthreads();
            if (c < n_cand) atomicAdd(&lh[ord_key(s) >> 21], 1u);
            __syncthreads();
            for (int i = threadIdx.x; i < kBins; i += 256)
                if (lh[i]) atomicAdd(&hist[i], lh[i]);
        }
        return;
    }
    const int c = blockIdx.x * 256 + threadIdx.x;
    float s = 0.0f;
    {
        for (int i = threadIdx.x; i < n_head * head_dim; i += 256) qs[i] = q[i];
        for (int i = threadIdx.x; i < n_head; i += 256) ws[i] = w[i];
        __syncthreads();
        if (c < n_comp) s = score_any<kKind>(qs, ws, keys, c, n_head, head_dim);
    }
    if (c < n_comp) scores[c] = s;
    if (hist) {
        __syncthreads();
        if (c < n_cand) atomicAdd(&lh[ord_key(s) >> 21], 1u);
        __syncthreads();
        for (int i = threadIdx.x; i < kBins; i += 256)
            if (lh[i]) atomicAdd(&hist[i], lh[i]);
    }
}

// The same scores (head_dim 128, n_head a multiple of 4) with the query and
// the weights read from global memory at wave-uniform addresses, so they come
// through scalar loads into SGPRs and every fma takes its query value as a
// scalar operand: no LDS staging and no LDS reads. The key row, the four
// independent head chains and the head sum keep score_lds' order, so the
// scores are bit-identical to it.
template <int kKind>
__global__ __launch_bounds__(256) void score_sgpr_kernel(const float *__restrict__ q,
                                                         const float *__restrict__ w,
                                                         const void *__restrict__ keys, int n_comp,
                                                         int n_head, float *__restrict__ scores,
                                                         unsigned *__restrict__ hist, int n_cand) {
    __shared__ unsigned lh[kBins];
    if (hist)
        for (int i = threadIdx.x; i < kBins; i += 256) lh[i] = 0;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int cc = c < n_comp ? c : n_comp - 1;   // the last block's spare lanes score a real key
    float k[kMaxDim];
    if (kKind == 0) {
        const float4_t *src = reinterpret_cast<const float4_t *>(
            static_cast<const float *>(keys) + (size_t)cc * kMaxDim);
#pragma unroll
        for (int v = 0; v < kMaxDim / 4; ++v) {
            const float4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 4; ++e) k[4 * v + e] = u[e];
        }
    } else {
        const uint4_t *src = reinterpret_cast<const uint4_t *>(
            static_cast<const uint16_t *>(keys) + (size_t)cc * kMaxDim);
#pragma unroll
        for (int v = 0; v < kMaxDim / 8; ++v) {
            const uint4_t u = src[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t h = (uint16_t)((u[e >> 1] >> (16 * (e & 1))) & 0xFFFF);
                k[8 * v + e] = kKind == 1 ? f16_bits_to_f32(h) : bf16_to_f32(h);
            }
        }
    }
    float s = 0.0f;
    for (int h = 0; h < n_head; h += 4) {
        const float *q0 = q + (size_t)h * kMaxDim;
        float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < kMaxDim / 4; ++v) {
            float4_t a[4];
#pragma unroll
            for (int z = 0; z < 4; ++z) a[z] = *reinterpret_cast<const float4_t *>(q0 + z * kMaxDim + 4 * v);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int z = 0; z < 4; ++z) d[z] = fmaf(a[z][e], k[4 * v + e], d[z]);
            // at most 4 x 64 query values in SGPRs at a time (the other waves
            // of the SIMD cover the scalar loads' latency)
            if ((v & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int z = 0; z < 4; ++z) s = fmaf(w[h + z], d[z] > 0.0f ? d[z] : 0.0f, s);
    }
    if (c < n_comp) scores[c] = s;
    if (hist) {
        __syncthreads();
        if (c < n_cand) atomicAdd(&lh[ord_key(s) >> 21], 1u);
        __syncthreads();
        for (int i = threadIdx.x; i < kBins; i += 256)
            if (lh[i]) atomicAdd(&hist[i], lh[i]);
    }
}

// DS4HIP_INDEXER_SGPR_SCORES=1 scores with score_sgpr_kernel (read at every
// launch; off by default until it has run on the GPU).
bool sgpr_scores_enabled() {
    const char *e = getenv("DS4HIP_INDEXER_SGPR_SCORES");
    return e && e[0] == '1';
}

__global__ void zero_u32_kernel(unsigned *p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// Inclusive prefix sum over the 256 threads of a workgroup (4 waves).
__device__ inline unsigned block_incl_scan(unsigned v, unsigned *wsum) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned u = __shfl_up(v, off);
        if (lane >= off) v += u;
    }
    if (lane == 63) wsum[wv] = v;
    __syncthreads();
    unsigned before = 0;
    for (int i = 0; i < wv; ++i) before += wsum[i];
    __syncthreads();
    return v + before;
}

// Finds, in histogram h (nb bins, high bin = larger keys), the bin holding the
// need-th largest key and the count strictly above that bin (need == 0:
// the top bin, nothing above).
// Called by every thread of a 256-thread workgroup: thread t sums bins
// [nb-1-t*per, nb-1-(t+1)*per), a block scan finds the thread whose range
// crosses need, and that thread walks its <= 8 bins.
__device__ void find_bin(const unsigned *h, int nb, unsigned need, unsigned *s_bin,
                         unsigned *s_above, unsigned *scratch) {
    const int t = threadIdx.x;
    const int per = nb / 256;
    unsigned local = 0;
    for (int i = 0; i < per; ++i) local += h[nb - 1 - (t * per + i)];
    const unsigned incl = block_incl_scan(local, scratch);
    const unsigned excl = incl - local;
    if (need == 0) {
        if (t == 0) {
            *s_bin = (unsigned)(nb - 1);
            *s_above = 0;
        }
    } else if (excl < need && incl >= need) {
        unsigned run = excl;
        int bin = nb - 1 - t * per;
        for (int i = 0; i < per - 1; ++i, --bin) {
            if (run + h[bin] >= need) break;
            run += h[bin];
        }
        *s_bin = (unsigned)bin;
        *s_above = run;
    }
    __syncthreads();
}

// Threshold key T (the need0-th largest candidate key) and the number of
// candidates equal to T that are taken (lowest indices first).
__device__ void threshold(const unsigned *hists, unsigned need0, unsigned *T, unsigned *need_eq,
                          unsigned *scratch, unsigned *s_bin, unsigned *s_above) {
    unsigned need = need0;
    find_bin(hists, kBins, need, s_bin, s_above, scratch);
    unsigned t = *s_bin << 21;
    need -= *s_above;
    __syncthreads();
    find_bin(hists + kBins, kBins, need, s_bin, s_above, scratch);
    t |= *s_bin << 10;
    need -= *s_above;
    __syncthreads();
    find_bin(hists + 2 * kBins, 1024, need, s_bin, s_above, scratch);
    t |= *s_bin;
    need -= *s_above;
    *T = t;
    *need_eq = need;
}

// Stage 2 / 3 histogram: recompute the selection state from the previous
// histograms, then histogram the next bit field of keys matching the prefix.
template <int kStage>
__global__ __launch_bounds__(256) void hist_next_kernel(const float *__restrict__ scores,
                                                        int n_cand, unsigned need0,
                                                        unsigned *__restrict__ hists) {
    __shared__ unsigned lh[kBins];
    __shared__ unsigned scratch[256];
    __shared__ unsigned s_bin, s_above;
    unsigned *h1 = hists, *h2 = hists + kBins, *h3 = hists + 2 * kBins;
    find_bin(h1, kBins, need0, &s_bin, &s_above, scratch);
    unsigned prefix = s_bin << 21, need = need0 - s_above;
    int shift = 10, nb = kBins;
    if (kStage == 3) {
        __syncthreads();
        find_bin(h2, kBins, need, &s_bin, &s_above, scratch);
        prefix |= s_bin << 10;
        shift = 0;
        nb = 1024;
    }
    for (int i = threadIdx.x; i < nb; i += 256) lh[i] = 0;
    __syncthreads();
    const unsigned mask_hi = kStage == 2 ? 0xFFE00000u : 0xFFFFFC00u;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < n_cand; c += gridDim.x * 256) {
        const unsigned k = ord_key(scores[c]);
        if ((k & mask_hi) == prefix) atomicAdd(&lh[(k >> shift) & (nb - 1)], 1u);
    }
    __syncthreads();
    unsigned *dst = kStage == 2 ? h2 : h3;
    for (int i = threadIdx.x; i < nb; i += 256)
        if (lh[i]) atomicAdd(&dst[i], lh[i]);
}

constexpr int kChunk = 1024;   // positions per emit workgroup (256 threads x 4)

// Per chunk: candidates strictly above T and equal to T.
__global__ __launch_bounds__(256) void count_kernel(const float *__restrict__ scores, int n_cand,
                                                    unsigned need0,
                                                    const unsigned *__restrict__ hists,
                                                    unsigned *__restrict__ chunk_gt,
                                                    unsigned *__restrict__ chunk_eq) {
    __shared__ unsigned scratch[256];
    __shared__ unsigned s_bin, s_above, red[2][4];
    unsigned T, need_eq;
    threshold(hists, need0, &T, &need_eq, scratch, &s_bin, &s_above);
    unsigned gt = 0, eq = 0;
    for (int i = 0; i < 4; ++i) {
        const int c = blockIdx.x * kChunk + i * 256 + threadIdx.x;
        if (c < n_cand) {
            const unsigned k = ord_key(scores[c]);
            gt += k > T;
            eq += k == T;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        gt += __shfl_xor(gt, off);
        eq += __shfl_xor(eq, off);
    }
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = gt;
        red[1][threadIdx.x >> 6] = eq;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        chunk_gt[blockIdx.x] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
        chunk_eq[blockIdx.x] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    }
}

// Block-wide exclusive scan of 256 values (one per thread); returns the total.
__device__ unsigned block_excl_scan(unsigned v, unsigned *buf, unsigned *excl) {
    const int t = threadIdx.x;
    buf[t] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const unsigned u = t >= off ? buf[t - off] : 0;
        __syncthreads();
        buf[t] += u;
        __syncthreads();
    }
    *excl = buf[t] - v;
    const unsigned total = buf[255];
    __syncthreads();
    return total;
}

// Per chunk: every candidate above T, ties at T in index order while the
// global tie rank < need_eq, and every position >= n_cand (the forced recent
// window). Writes the 0/1 mask and/or the ascending position list.
__global__ __launch_bounds__(256) void emit_kernel(const float *__restrict__ scores, int n_comp,
                                                   int n_cand, unsigned need0,
                                                   const unsigned *__restrict__ hists,
                                                   const unsigned *__restrict__ chunk_gt,
                                                   const unsigned *__restrict__ chunk_eq,
                                                   int32_t *__restrict__ mask,
                                                   int32_t *__restrict__ pos_out) {
    __shared__ unsigned scratch[256], buf[256];
    __shared__ unsigned s_bin, s_above;
    unsigned T, need_eq;
    threshold(hists, need0, &T, &need_eq, scratch, &s_bin, &s_above);
    // selections and ties of the earlier chunks
    unsigned sel_b = 0, eq_b = 0;
    for (int c2 = threadIdx.x; c2 < (int)blockIdx.x; c2 += 256) {
        eq_b += chunk_eq[c2];
        sel_b += chunk_gt[c2];
    }
    unsigned ex;
    const unsigned eq_before = block_excl_scan(eq_b, buf, &ex);
    const unsigned gt_before = block_excl_scan(sel_b, buf, &ex);
    // ties taken by earlier chunks = min(need_eq, ties before)
    const unsigned ties_taken_before = eq_before < need_eq ? eq_before : need_eq;
    const unsigned sel_before = gt_before + ties_taken_before;
    // this thread's 4 consecutive positions
    const int base = blockIdx.x * kChunk + threadIdx.x * 4;
    unsigned k4[4];
    unsigned my_eq = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = base + i;
        k4[i] = (c < n_cand) ? ord_key(scores[c]) : 0;
        my_eq += (c < n_cand) && k4[i] == T;
    }
    unsigned eq_ex;
    block_excl_scan(my_eq, buf, &eq_ex);
    unsigned rank = eq_before + eq_ex;
    bool take[4];
    unsigned my_sel = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = base + i;
        bool t = false;
        if (c < n_cand) {
            if (k4[i] > T) t = true;
            else if (k4[i] == T) { t = rank < need_eq; ++rank; }
        } else if (c < n_comp) {
            t = true;
        }
        take[i] = t;
        my_sel += t;
    }
    unsigned sel_ex;
    block_excl_scan(my_sel, buf, &sel_ex);
    unsigned o = sel_before + sel_ex;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = base + i;
        if (c >= n_comp) break;
        if (mask) mask[c] = take[i] ? 1 : 0;
        if (take[i] && pos_out) pos_out[o] = c;
        o += take[i];
    }
}

__global__ void fill_kernel(int32_t *out, int n, int32_t v, int iota) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = iota ? i : v;
}

__global__ void scale_kernel(float *y, int n, float s) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] *= s;
}

// ---- prefiltered selection (bf16 keys, 64 heads x 128) -------------------------------------
//
// The exact scores cost 8192 dependent fp32 fma per key. Only the keys whose
// score could fall on either side of the selection threshold need them:
//
//  1. prefilter_kernel: approximate scores a_c on the bf16 MFMA (the query
//     split into bf16 hi + lo, the key bf16 exact; fp32 accumulation), with a
//     per-key bound b_c >= |a_c - s_c| on the distance to the exact score s_c
//     (derivation below), the level-1 histogram of a and max_c b_c.
//  2. hist_next_kernel<2>: the level-2 histogram of a. The need-th largest a
//     then lies in a 22-bit key bucket [lo, hi].
//  3. band_kernel: with B = max b, the need-th largest exact score lies in
//     [lo - B, hi + B]; a key with a - b > hi + B is certainly selected, one
//     with a + b < lo - B certainly not; the rest (the band) is rescored with
//     the exact fixed-order chains. The last workgroup to finish selects the
//     need - (certainly selected) best band keys by (exact score desc, index
//     asc), marks every candidate's score slot +inf (selected) or -inf, and
//     writes each chunk's output offset.
//  4. emit_marked_kernel: the positions (and/or mask) in index order.
//
// Bound: with u = 2^-24, the reference's chains give |s - s*| <= (128 + 64) u
// sum_h |w_h| A_h, A_h = sum_d |q_hd k_d| (s* the exact real score; relu is
// 1-Lipschitz). The MFMA form differs from s* by at most (2 * 128 + 64) u
// sum_h |w_h| A_h for its two accumulation passes and head sum, plus 2^-18
// sum_h |w_h| A_h for the part of q that hi + lo drops. So |a - s| <= 3.5e-5
// sum_h |w_h| A_h <= 3.5e-5 ||k|| sum_h |w_h| ||q_h|| (Cauchy-Schwarz); b
// uses the constant 1e-4 for margin.
constexpr float kBoundC = 1.0e-4f;
constexpr int kPfMaxChunks = 1024;   // candidates <= kPfMaxChunks * kChunk
constexpr int kPfMinCand = 8192;      // fewer candidates: the exact scorer outright
// DS4HIP_INDEXER_PREFILTER=0 keeps the exact scorer for every key.
// Off by default: two GPU runs of a timing variant of this path (a fake
// level-1 histogram, not part of this code) left most of the position list
// unwritten, and the gathered decode then read rows at garbage indices. The
// emit kernel now writes valid positions whenever the counts disagree; the
// prefilter stays opt-in (DS4HIP_INDEXER_PREFILTER=1 or
// ds4hip_set_indexer_prefilter(1)) until it has run again.
int g_prefilter = -1;
bool prefilter_enabled() {
    if (g_prefilter < 0) {
        const char *e = getenv("DS4HIP_INDEXER_PREFILTER");
        g_prefilter = (e && e[0] == '1') ? 1 : 0;
    }
    return g_prefilter == 1;
}
typedef short pf_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 pf_bf16x2_t __attribute__((ext_vector_type(2)));
typedef short pf_short2_t __attribute__((ext_vector_type(2)));

// A load that sees other workgroups' completed writes (device-coherent).
template <typename T>
__device__ inline T ld_agent(const T *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline float key_to_float(unsigned k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Selection scratch of the prefiltered path, after the three histograms.
struct PfScratch {
    unsigned *bmax;        // max bound (float bits; bounds are >= 0)
    unsigned *done;        // band workgroups finished
    unsigned *chunk_in;    // [n_chunks] certainly selected candidates per chunk
    unsigned *chunk_off;   // [n_chunks] output offset of each chunk
    unsigned *band_n;      // [n_chunks] band keys per chunk
    float *bound;          // [n_chunks * kChunk]
    float *band_val;       // [n_chunks * kChunk] exact scores of band keys, per chunk
    int *band_idx;         // [n_chunks * kChunk]
    float *cval;           // [n_chunks * kChunk] the band entries compacted
    int *cidx;             // [n_chunks * kChunk]
};

__host__ __device__ inline size_t pf_align(size_t n) { return (n + 63) & ~size_t(63); }

__host__ __device__ inline PfScratch pf_scratch(unsigned *base, int n_comp) {
    const size_t chunks = (size_t)(n_comp > 0 ? n_comp : 1) / kChunk + 1;
    const size_t rows = chunks * kChunk;
    unsigned *p = base + 3 * kBins;
    PfScratch S;
    S.bmax = p;
    S.done = p + 1;
    p += 64;
    S.chunk_in = p;
    p += pf_align(chunks);
    S.chunk_off = p;
    p += pf_align(chunks);
    S.band_n = p;
    p += pf_align(chunks);
    S.bound = reinterpret_cast<float *>(p);
    p += rows;
    S.band_val = reinterpret_cast<float *>(p);
    p += rows;
    S.band_idx = reinterpret_cast<int *>(p);
    p += rows;
    S.cval = reinterpret_cast<float *>(p);
    p += rows;
    S.cidx = reinterpret_cast<int *>(p);
    return S;
}

size_t pf_scratch_words(int n_comp) {
    const size_t chunks = (size_t)(n_comp > 0 ? n_comp : 1) / kChunk + 1;
    return 3 * kBins + 64 + 3 * pf_align(chunks) + 5 * chunks * kChunk;
}

// sum over lanes l, l^16, l^32, l^48 with VALU lane swaps (no LDS)
__device__ inline float pf_xsum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One wave scores 16 keys per step: D = Q . K^T per head tile with A = 16
// query heads x 32 dims (lane (j, g): head 16 ht + j, dims 8 g .. 8 g + 7 of
// the k-step; hi and lo parts) and B = 32 dims x 16 keys (lane (j, g): key j,
// the same dims). Lane (j, g) then holds heads 16 ht + 4 g + r of key j, so
// the weighted head sum is 16 fmas in the lane and two lane swaps, and the
// key's norm reduces the same way: no LDS round trips.
__global__ __launch_bounds__(256) void prefilter_kernel(const float *__restrict__ q,
                                                        const float *__restrict__ w,
                                                        const uint16_t *__restrict__ keys,
                                                        int n_cand, float *__restrict__ a_out,
                                                        unsigned *__restrict__ hist1, PfScratch S) {
    __shared__ unsigned lh[kBins];
    __shared__ unsigned s_bmax;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kBins; i += 256) lh[i] = 0;
    if (tid == 0) s_bmax = 0;
    const int j = lane & 15, g = lane >> 4;
    pf_bf16x8_t qh[4][4], ql[4][4];   // [head tile][k-step]
    float qn2[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // ||q_h||^2 of head 16 ht + j (this lane's 32 dims)
#pragma unroll
    for (int ht = 0; ht < 4; ++ht)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const float *src = q + (16 * ht + j) * kMaxDim + 32 * ks + 8 * g;
            const float4_t x0 = *reinterpret_cast<const float4_t *>(src);
            const float4_t x1 = *reinterpret_cast<const float4_t *>(src + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) qn2[ht] = fmaf(x0[e], x0[e], fmaf(x1[e], x1[e], qn2[ht]));
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float v0 = e < 4 ? x0[e] : x1[e - 4], v1 = e < 4 ? x0[e + 1] : x1[e - 3];
                const pf_bf16x2_t h = pf_bf16x2_t{(__bf16)v0, (__bf16)v1};
                const pf_bf16x2_t l = pf_bf16x2_t{(__bf16)(v0 - (float)h[0]), (__bf16)(v1 - (float)h[1])};
                const pf_short2_t hs = __builtin_bit_cast(pf_short2_t, h), ls = __builtin_bit_cast(pf_short2_t, l);
                qh[ht][ks][e] = hs[0];
                qh[ht][ks][e + 1] = hs[1];
                ql[ht][ks][e] = ls[0];
                ql[ht][ks][e + 1] = ls[1];
            }
        }
    // Wq = sum_h |w_h| ||q_h|| (lane (j, g) holds a quarter of head 16 ht + j's norm)
    float wq = 0.0f;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) wq += fabsf(w[16 * ht + j]) * sqrtf(pf_xsum(qn2[ht]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) wq += __shfl_xor(wq, off, 16);
    // the head weights of the D rows this lane holds: head 16 ht + 4 g + r
    float wr[4][4];
#pragma unroll
    for (int ht = 0; ht < 4; ++ht)
#pragma unroll
        for (int r = 0; r < 4; ++r) wr[ht][r] = w[16 * ht + 4 * g + r];
    __syncthreads();
    float bmax = 0.0f;
    const int n_tiles = (n_cand + 15) / 16;
    // the next tile's key fragments are loaded before this tile's MFMAs
    auto load_tile = [&](int tile, uint4_t (&u)[4]) {
        const int row = 16 * tile + j;
        const int rr = row < n_cand ? row : n_cand - 1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            u[ks] = *reinterpret_cast<const uint4_t *>(keys + (size_t)rr * kMaxDim + 32 * ks + 8 * g);
    };
    const int stride = gridDim.x * 4;
    // two fragment buffers in turn, so the next tile's loads need no copy; a
    // load past the last tile re-reads the last tile (unused)
    auto process = [&](int tile, const uint4_t (&uc)[4]) {
        pf_bf16x8_t a[4];
        float n2 = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint4_t u = uc[ks];
            a[ks] = __builtin_bit_cast(pf_bf16x8_t, u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const pf_bf16x2_t kp = __builtin_bit_cast(pf_bf16x2_t, u[e]);
                n2 = __builtin_amdgcn_fdot2_f32_bf16(kp, kp, n2, false);
            }
        }
        float4_t c[4];
#pragma unroll
        for (int ht = 0; ht < 4; ++ht) {
            c[ht] = float4_t{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                c[ht] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh[ht][ks], a[ks], c[ht], 0, 0, 0);
                c[ht] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql[ht][ks], a[ks], c[ht], 0, 0, 0);
            }
        }
        // lane (j, g): heads 16 ht + 4 g + r of key j
        float v = 0.0f;
#pragma unroll
        for (int ht = 0; ht < 4; ++ht)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float rl;   // relu without the quieting that fmaxf adds
                asm("v_max_f32 %0, 0, %1" : "=v"(rl) : "v"(c[ht][r]));
                v = fmaf(wr[ht][r], rl, v);
            }
        v = pf_xsum(v);
        const float kn2 = pf_xsum(n2);   // ||k_j||^2
        const int kr = 16 * tile + j;
        if (g == 0 && kr < n_cand) {
            const float b = kBoundC * sqrtf(kn2) * wq;
            a_out[kr] = v;
            S.bound[kr] = b;
            bmax = fmaxf(bmax, b);
            atomicAdd(&lh[ord_key(v) >> 21], 1u);
        }
    };
    const int first = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(wave);
    uint4_t ub0[4], ub1[4];
    if (first < n_tiles) load_tile(first, ub0);
    for (int tile = first; tile < n_tiles; tile += 2 * stride) {
        load_tile(min(tile + stride, n_tiles - 1), ub1);
        process(tile, ub0);
        if (tile + stride >= n_tiles) break;
        load_tile(min(tile + 2 * stride, n_tiles - 1), ub0);
        process(tile + stride, ub1);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bmax = fmaxf(bmax, __shfl_xor(bmax, off));
    if (lane == 0) atomicMax(&s_bmax, __float_as_uint(bmax));
    __syncthreads();
    for (int i = tid; i < kBins; i += 256)
        if (lh[i]) atomicAdd(&hist1[i], lh[i]);
    if (tid == 0) atomicMax(S.bmax, s_bmax);
}

// Exact score of key c (the canonical chains): lane h forms dot_h over d
// ascending, then the head chain runs over h ascending in lane 0.
__device__ inline float exact_score_wave(const float *qs, const float *ws, const uint16_t *keys, int c) {
    const int h = threadIdx.x & 63;
    const uint16_t *kr = keys + (size_t)c * kMaxDim;
    uint4_t kk[kMaxDim / 8];   // the whole key first: one memory round trip
#pragma unroll
    for (int v = 0; v < kMaxDim / 8; ++v) kk[v] = *reinterpret_cast<const uint4_t *>(kr + 8 * v);
    float dot = 0.0f;
#pragma unroll
    for (int v = 0; v < kMaxDim / 8; ++v) {
        const uint4_t u = kk[v];
        const float4_t q0 = *reinterpret_cast<const float4_t *>(qs + h * kQStride + 8 * v);
        const float4_t q1 = *reinterpret_cast<const float4_t *>(qs + h * kQStride + 8 * v + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t b = (uint16_t)((u[e >> 1] >> (16 * (e & 1))) & 0xFFFF);
            dot = fmaf(e < 4 ? q0[e] : q1[e - 4], bf16_to_f32(b), dot);
        }
    }
    const float r = dot > 0.0f ? dot : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int hh = 0; hh < kMaxHeads; ++hh)
        s = fmaf(ws[hh], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), hh)), s);
    return s;
}

// Threshold of the need-th largest of n 32-bit keys key_of(i) (need >= 1):
// returns T and how many entries equal to T are taken. One workgroup.
template <typename KeyOf>
__device__ void wg_select(int n, unsigned need, KeyOf key_of, unsigned *lh, unsigned *scratch,
                          unsigned *s_bin, unsigned *s_above, unsigned *T_out, unsigned *eq_out) {
    unsigned prefix = 0, mask = 0;
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    for (int lvl = 0; lvl < 3; ++lvl) {
        const int nb = 1 << widths[lvl];
        for (int i = threadIdx.x; i < kBins; i += 256) lh[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += 256) {
            const unsigned k = key_of(i);
            if ((k & mask) == prefix) atomicAdd(&lh[(k >> shifts[lvl]) & (nb - 1)], 1u);
        }
        __syncthreads();
        find_bin(lh, nb, need, s_bin, s_above, scratch);
        prefix |= *s_bin << shifts[lvl];
        mask |= (unsigned)(nb - 1) << shifts[lvl];
        need -= *s_above;
        __syncthreads();
    }
    *T_out = prefix;
    *eq_out = need;
}

__global__ __launch_bounds__(256) void band_kernel(const float *__restrict__ q,
                                                   const float *__restrict__ w,
                                                   const uint16_t *__restrict__ keys, int n_cand,
                                                   int n_comp, unsigned need0, int n_chunks,
                                                   float *__restrict__ a_io,
                                                   const unsigned *__restrict__ hists, PfScratch S) {
    __shared__ __attribute__((aligned(16))) float qs[kMaxHeads * kQStride];
    __shared__ float ws[kMaxHeads];
    __shared__ unsigned lh[kBins];
    __shared__ unsigned scratch[256];
    __shared__ unsigned s_bin, s_above, s_ticket, s_cnt[4];
    __shared__ int band_l[kChunk];
    __shared__ unsigned s_nband;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the bucket of the need0-th largest approximate score
    find_bin(hists, kBins, need0, &s_bin, &s_above, scratch);
    unsigned prefix = s_bin << 21;
    const unsigned need1 = need0 - s_above;
    __syncthreads();
    find_bin(hists + kBins, kBins, need1, &s_bin, &s_above, scratch);
    prefix |= s_bin << 10;
    const float lo = key_to_float(prefix), hi = key_to_float(prefix | 0x3FFu);
    const float B = __uint_as_float(*S.bmax);
    if (tid == 0) s_nband = 0;
    stage_query<kQStride>(qs, q, kMaxHeads);
    if (tid < kMaxHeads) ws[tid] = w[tid];
    __syncthreads();
    unsigned cin = 0;
    for (int i = 0; i < 4; ++i) {
        const int c = blockIdx.x * kChunk + i * 256 + tid;
        if (c >= n_cand) continue;
        const float a = a_io[c], b = S.bound[c];
        if (a - b > hi + B) {
            a_io[c] = INFINITY;
            ++cin;
        } else if (a + b < lo - B) {
            a_io[c] = -INFINITY;
        } else {
            band_l[atomicAdd(&s_nband, 1u)] = c;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cin += __shfl_xor(cin, off);
    if (lane == 0) s_cnt[wave] = cin;
    __syncthreads();
    const unsigned nband = s_nband;
    // exact rescoring: one wave per band key, into this chunk's band slots
    const size_t base = (size_t)blockIdx.x * kChunk;
    for (unsigned e = wave; e < nband; e += 4) {
        const int c = band_l[e];
        const float s = exact_score_wave(qs, ws, keys, c);
        if (lane == 0) {
            S.band_val[base + e] = s;
            S.band_idx[base + e] = c;
        }
    }
    if (tid == 0) {
        S.chunk_in[blockIdx.x] = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
        S.band_n[blockIdx.x] = nband;
    }
    // the last workgroup to finish selects within the band
    __threadfence();
    __syncthreads();
    if (tid == 0) s_ticket = atomicAdd(S.done, 1u);
    __syncthreads();
    if (s_ticket != gridDim.x - 1) return;
    __threadfence();
    // compact the chunks' band entries (4 chunks per thread; <= 1024 chunks)
    int nb;
    {
        unsigned v[4], tot = 0;
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * tid + k;
            // (bounded: a chunk holds at most kChunk band keys)
            v[k] = i < (int)gridDim.x ? min(ld_agent(&S.band_n[i]), (unsigned)kChunk) : 0u;
            tot += v[k];
        }
        unsigned ex;
        nb = (int)block_excl_scan(tot, scratch, &ex);
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * tid + k;
            for (unsigned e = 0; e < v[k]; ++e) {
                S.cval[ex + e] = ld_agent(&S.band_val[(size_t)i * kChunk + e]);
                S.cidx[ex + e] = ld_agent(&S.band_idx[(size_t)i * kChunk + e]);
            }
            ex += v[k];
        }
        __threadfence_block();
        __syncthreads();
    }
    unsigned c_in = 0;
    for (int i = tid; i < (int)gridDim.x; i += 256) c_in += ld_agent(&S.chunk_in[i]);
    for (int off = 32; off > 0; off >>= 1) c_in += __shfl_xor(c_in, off);
    if (lane == 0) s_cnt[wave] = c_in;
    __syncthreads();
    c_in = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    const unsigned m = need0 - c_in;   // band keys to take (1 <= m <= nb)
    unsigned T, eq;
    wg_select(nb, m, [&](int i) { return ord_key(S.cval[i]); }, lh, scratch, &s_bin, &s_above, &T, &eq);
    // ties at T: the eq lowest indices (the largest ~index)
    unsigned Ti = 0, eqi = 0;
    if (eq > 0) {
        wg_select(nb, eq, [&](int i) { return ord_key(S.cval[i]) == T ? ~(unsigned)S.cidx[i] : 0u; },
                  lh, scratch, &s_bin, &s_above, &Ti, &eqi);
    }
    // chunk counts: certainly selected + selected band keys + forced recent positions
    unsigned *cnt = lh;   // reuse: n_chunks <= kPfMaxChunks <= kBins
    for (int i = tid; i < n_chunks; i += 256) cnt[i] = i < (int)gridDim.x ? ld_agent(&S.chunk_in[i]) : 0u;
    __syncthreads();
    for (int i = tid; i < nb; i += 256) {
        const unsigned k = ord_key(S.cval[i]);
        const int c = S.cidx[i];
        if ((unsigned)c >= (unsigned)n_cand) continue;   // (never: every entry is a candidate)
        const bool sel = k > T || (k == T && eq > 0 && ~(unsigned)c >= Ti);
        a_io[c] = sel ? INFINITY : -INFINITY;
        if (sel) atomicAdd(&cnt[c / kChunk], 1u);
    }
    __syncthreads();
    for (int i = tid; i < n_chunks; i += 256) {
        const int c0 = i * kChunk, c1 = min(c0 + kChunk, n_comp);
        const int r0 = max(c0, n_cand);
        cnt[i] += r0 < c1 ? (unsigned)(c1 - r0) : 0u;
    }
    __syncthreads();
    // exclusive prefix over the chunks (n_chunks <= 1024: 4 per thread)
    unsigned v[4], tot = 0;
    for (int k = 0; k < 4; ++k) {
        const int i = 4 * tid + k;
        v[k] = i < n_chunks ? cnt[i] : 0u;
        tot += v[k];
    }
    unsigned ex;
    const unsigned total = block_excl_scan(tot, scratch, &ex);
    for (int k = 0; k < 4; ++k) {
        const int i = 4 * tid + k;
        if (i < n_chunks) S.chunk_off[i] = ex;
        ex += v[k];
    }
    if (tid == 0) {
        *S.done = 0;
        // the counts add up to the output size by construction; if they ever
        // did not, the emit kernel writes positions 0.. instead of a list with
        // holes (every output slot stays a valid row index)
        S.bmax[2] = total == need0 + (unsigned)(n_comp - n_cand) ? 0u : 1u;
    }
}

// Per chunk: positions of the marked (+inf) candidates and of the forced
// recent window, in index order, from the chunk's offset.
__global__ __launch_bounds__(256) void emit_marked_kernel(const float *__restrict__ marks, int n_comp,
                                                          int n_cand, int n_out, PfScratch S,
                                                          int32_t *__restrict__ mask,
                                                          int32_t *__restrict__ pos_out) {
    __shared__ unsigned buf[256];
    if (S.bmax[2]) {
        for (int i = blockIdx.x * 256 + threadIdx.x; i < n_out; i += gridDim.x * 256) {
            if (pos_out) pos_out[i] = i < n_comp ? i : n_comp - 1;
            if (mask && i < n_comp) mask[i] = 1;
        }
        return;
    }
    const int base = blockIdx.x * kChunk + threadIdx.x * 4;
    bool take[4];
    unsigned my = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = base + i;
        take[i] = c < n_cand ? marks[c] == INFINITY : c < n_comp;
        my += take[i];
    }
    unsigned ex;
    block_excl_scan(my, buf, &ex);
    unsigned o = S.chunk_off[blockIdx.x] + ex;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = base + i;
        if (c >= n_comp) break;
        if (mask) mask[c] = take[i] ? 1 : 0;
        if (take[i] && pos_out && o < (unsigned)n_out) pos_out[o] = c;
        o += take[i];
    }
}

int pf_grid() {
    static const int v = [] {
        const char *e = getenv("DS4HIP_PF_GRID");
        return e ? atoi(e) : 256;
    }();
    return v;
}

int score_select_prefilter(const float *q, const float *w, const uint16_t *keys, int n_comp,
                           int n_cand, unsigned need0, float *scores, unsigned *scratch, int32_t *mask,
                           int32_t *pos_out, hipStream_t st) {
    const PfScratch S = pf_scratch(scratch, n_comp);
    const int n_chunks = (n_comp + kChunk - 1) / kChunk;
    const int n_band_wg = (n_cand + kChunk - 1) / kChunk;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(24), dim3(256), 0, st, scratch, 3 * kBins + 64);
    hipLaunchKernelGGL(prefilter_kernel, dim3(std::min(pf_grid(), (n_cand + 63) / 64)), dim3(256), 0, st, q, w,
                       keys, n_cand, scores, scratch, S);
    const int g = (n_cand + 256 * 8 - 1) / (256 * 8) + 1;
    hipLaunchKernelGGL(hist_next_kernel<2>, dim3(g), dim3(256), 0, st, scores, n_cand, need0, scratch);
    hipLaunchKernelGGL(band_kernel, dim3(n_band_wg), dim3(256), 0, st, q, w, keys, n_cand, n_comp, need0,
                       n_chunks, scores, scratch, S);
    hipLaunchKernelGGL(emit_marked_kernel, dim3(n_chunks), dim3(256), 0, st, scores, n_comp, n_cand,
                       (int)need0 + (n_comp - n_cand), S, mask, pos_out);
    return hip_status(hipGetLastError());
}

int launch_scores(const float *q, const float *w, const void *keys, int kind, int n_comp,
                  int n_head, int head_dim, float *scores, unsigned *hist, int n_cand,
                  hipStream_t st) {
    const bool full = head_dim == kMaxDim;
    const dim3 grid((n_comp + 255) / 256);
    if (full && n_head % 4 == 0 && n_comp > 0 && sgpr_scores_enabled()) {
        switch (kind) {
        case 0: hipLaunchKernelGGL(score_sgpr_kernel<0>, grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, scores, hist, n_cand); break;
        case 1: hipLaunchKernelGGL(score_sgpr_kernel<1>, grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, scores, hist, n_cand); break;
        default: hipLaunchKernelGGL(score_sgpr_kernel<2>, grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, scores, hist, n_cand); break;
        }
        return hip_status(hipGetLastError());
    }
    switch (kind) {
    case 0:
        if (full) hipLaunchKernelGGL((score_kernel<0, true>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        else hipLaunchKernelGGL((score_kernel<0, false>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        break;
    case 1:
        if (full) hipLaunchKernelGGL((score_kernel<1, true>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        else hipLaunchKernelGGL((score_kernel<1, false>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        break;
    default:
        if (full) hipLaunchKernelGGL((score_kernel<2, true>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        else hipLaunchKernelGGL((score_kernel<2, false>), grid, dim3(256), 0, st, q, w, keys, n_comp, n_head, head_dim, scores, hist, n_cand);
        break;
    }
    return hip_status(hipGetLastError());
}

// scores + selection. mask and/or pos_out; n_recent trailing positions are
// always selected and take part in no comparison.
size_t select_scratch_bytes(int n_comp) {
    const size_t chunks = (size_t)(n_comp > 0 ? n_comp : 1) / kChunk + 1;
    return std::max((3 * kBins + 2 * chunks), pf_scratch_words(n_comp)) * sizeof(unsigned);
}

int score_select(const float *q, const float *w, const void *keys, int kind, int n_comp,
                 int n_head, int head_dim, int top_k, int n_recent, float *scores,
                 unsigned *scratch, int32_t *mask, int32_t *pos_out, hipStream_t st) {
    if (!q || !w || !keys || !scores || !scratch || n_head <= 0 || n_head > kMaxHeads ||
        head_dim <= 0 || head_dim > kMaxDim || n_recent < 0 || (!mask && !pos_out))
        return kEINVAL;
    if (n_comp <= 0) return 0;
    if (top_k <= 0) {
        if (mask) hipLaunchKernelGGL(fill_kernel, dim3((n_comp + 255) / 256), dim3(256), 0, st, mask, n_comp, 0, 0);
        return hip_status(hipGetLastError());
    }
    if (n_comp <= top_k) {
        int rc = launch_scores(q, w, keys, kind, n_comp, n_head, head_dim, scores, nullptr, 0, st);
        if (rc) return rc;
        if (mask) hipLaunchKernelGGL(fill_kernel, dim3((n_comp + 255) / 256), dim3(256), 0, st, mask, n_comp, 1, 0);
        if (pos_out) hipLaunchKernelGGL(fill_kernel, dim3((n_comp + 255) / 256), dim3(256), 0, st, pos_out, n_comp, 0, 1);
        return hip_status(hipGetLastError());
    }
    const int recent = n_recent < top_k ? n_recent : top_k;
    const int n_cand = n_comp - recent;
    const unsigned need0 = (unsigned)(top_k - recent);
    const int n_chunks = (n_comp + kChunk - 1) / kChunk;
    // bf16 keys of the model's indexer shape: the MFMA prefilter with exact
    // rescoring near the threshold (the same selection, a fraction of the work)
    if (kind == 2 && n_head == kMaxHeads && head_dim == kMaxDim && n_cand >= kPfMinCand &&
        (n_cand + kChunk - 1) / kChunk <= kPfMaxChunks && n_chunks <= kPfMaxChunks &&
        !(reinterpret_cast<uintptr_t>(keys) & 15) && !(reinterpret_cast<uintptr_t>(q) & 15) &&
        prefilter_enabled())
        return score_select_prefilter(q, w, static_cast<const uint16_t *>(keys), n_comp, n_cand, need0,
                                      scores, scratch, mask, pos_out, st);
    unsigned *hists = scratch;
    unsigned *chunk_gt = scratch + 3 * kBins;
    unsigned *chunk_eq = chunk_gt + n_chunks;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(24), dim3(256), 0, st, hists, 3 * kBins);
    int rc = launch_scores(q, w, keys, kind, n_comp, n_head, head_dim, scores, hists, n_cand, st);
    if (rc) return rc;
    const int g = (n_cand + 256 * 8 - 1) / (256 * 8) + 1;
    hipLaunchKernelGGL(hist_next_kernel<2>, dim3(g), dim3(256), 0, st, scores, n_cand, need0, hists);
    hipLaunchKernelGGL(hist_next_kernel<3>, dim3(g), dim3(256), 0, st, scores, n_cand, need0, hists);
    hipLaunchKernelGGL(count_kernel, dim3(n_chunks), dim3(256), 0, st, scores, n_cand, need0, hists,
                       chunk_gt, chunk_eq);
    hipLaunchKernelGGL(emit_kernel, dim3(n_chunks), dim3(256), 0, st, scores, n_comp, n_cand, need0,
                       hists, chunk_gt, chunk_eq, mask, pos_out);
    return hip_status(hipGetLastError());
}

}  // namespace

extern "C" int ds4hip_indexer_allowed_short_circuit_i32(int32_t *out_i32, int n_comp, int top_k,
                                                        void *stream) {
    // cuda/indexer_allowed.cu:283-305: n_comp <= 0 -> nothing; n_comp > top_k
    // is a caller error (the reference aborts; here it is reported).
    if (n_comp <= 0) return 0;
    if (!out_i32 || n_comp > top_k) return ds4hip_set_last_error(kEINVAL);
    hipLaunchKernelGGL(fill_kernel, dim3((n_comp + 127) / 128), dim3(128), 0, (hipStream_t)stream,
                       out_i32, n_comp, 1, 0);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_scale_inplace_f32(float *y, int n, float scale, void *stream) {
    if (n <= 0) return 0;
    if (!y) return ds4hip_set_last_error(kEINVAL);
    hipLaunchKernelGGL(scale_kernel, dim3((n + 63) / 64), dim3(64), 0, (hipStream_t)stream, y, n, scale);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" size_t ds4hip_indexer_select_scratch_bytes(int n_comp) { return select_scratch_bytes(n_comp); }

extern "C" int ds4hip_set_indexer_prefilter(int enable) {
    if (enable != 0 && enable != 1) return ds4hip_set_last_error(kEINVAL);
    const int prev = prefilter_enabled() ? 1 : 0;
    g_prefilter = enable;
    return prev;
}

// The reference launchers take only a score scratch; the selection
// histograms are stream-ordered allocations here.
static int with_hists(int (*fn)(unsigned *, void *), void *ctx, int n_comp, hipStream_t st) {
    void *h = nullptr;
    hipError_t e = hipMallocAsync(&h, select_scratch_bytes(n_comp), st);
    if (e != hipSuccess) return hip_status(e);
    int rc = fn(static_cast<unsigned *>(h), ctx);
    e = hipFreeAsync(h, st);
    return rc ? rc : hip_status(e);
}

struct TopkCall {
    const float *q, *w;
    const void *keys;
    int kind, n_comp, n_head, head_dim, top_k;
    int32_t *allowed;
    float *scores;
    hipStream_t st;
};

extern "C" int ds4hip_indexer_score_topk_i32(const float *q, const float *weights,
                                             const uint16_t *index_comp, int n_comp, int n_head,
                                             int head_dim, int top_k, int32_t *allowed_out,
                                             float *scratch_scores, void *stream) {
    if (n_comp <= 0 || n_head <= 0 || head_dim <= 0) return 0;   // cuda/indexer_allowed.cu:330-331
    TopkCall c{q, weights, index_comp, 1, n_comp, n_head, head_dim, top_k, allowed_out,
               scratch_scores, (hipStream_t)stream};
    return ds4hip_set_last_error(with_hists(
        [](unsigned *h, void *p) {
            auto *c = static_cast<TopkCall *>(p);
            return score_select(c->q, c->w, c->keys, c->kind, c->n_comp, c->n_head, c->head_dim,
                                c->top_k, 0, c->scores, h, c->allowed, nullptr, c->st);
        },
        &c, n_comp, (hipStream_t)stream));
}

extern "C" int ds4hip_indexer_score_topk_f32_i32(const float *q, const float *weights,
                                                 const float *index_comp_f32, int n_comp,
                                                 int n_head, int head_dim, int top_k,
                                                 int32_t *allowed_out, float *scratch_scores,
                                                 void *stream) {
    if (n_comp <= 0 || n_head <= 0 || head_dim <= 0) return 0;
    TopkCall c{q, weights, index_comp_f32, 0, n_comp, n_head, head_dim, top_k, allowed_out,
               scratch_scores, (hipStream_t)stream};
    return ds4hip_set_last_error(with_hists(
        [](unsigned *h, void *p) {
            auto *c = static_cast<TopkCall *>(p);
            return score_select(c->q, c->w, c->keys, c->kind, c->n_comp, c->n_head, c->head_dim,
                                c->top_k, 0, c->scores, h, c->allowed, nullptr, c->st);
        },
        &c, n_comp, (hipStream_t)stream));
}

extern "C" int ds4hip_indexer_topk_positions(const float *q, const float *weights,
                                             const void *keys, int key_kind, int n_comp,
                                             int n_head, int head_dim, int top_k, int n_recent,
                                             float *scratch_scores, void *scratch_select,
                                             int32_t *allowed_mask, int32_t *positions_out,
                                             void *stream) {
    if (key_kind < 0 || key_kind > 2) return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(score_select(
        q, weights, keys, key_kind, n_comp, n_head, head_dim, top_k, n_recent, scratch_scores,
        static_cast<unsigned *>(scratch_select), allowed_mask, positions_out, (hipStream_t)stream));
}

// ---- batched selection (several sequences, one launch per phase) -------------------------
//
// Scores: the key rows of all sequences are concatenated; block ranges per
// sequence come from a prefix table in the kernel arguments, so each block
// scores keys of one sequence with that sequence's query and weights.
// Selection: one 1024-thread workgroup per sequence holds the ordered keys of
// its candidates in LDS (up to kSelMax) and runs a 4 x 8-bit radix select,
// then emits the positions in ascending order (same rule as above: the top
// (score desc, index asc) plus the forced recent window).

namespace {

constexpr int kMaxSeq = 16;
constexpr int kSelMax = 16384;

struct BatchArgs {
    const float *q;            // [n_seq][n_head][128]
    const float *w;            // [n_seq][n_head]
    const void *keys;          // key rows, sequence s at row key0[s]
    float *scores;             // same indexing as the key rows
    int32_t *pos_out;          // [n_seq][pos_stride]
    int n_seq, n_head, top_k, n_recent, pos_stride;
    long long key0[kMaxSeq];
    int n_comp[kMaxSeq];
    int blk0[kMaxSeq + 1];     // first score block of each sequence
};

// kSplit threads per key (1 or 4); blocks of 256 threads cover 256 / kSplit keys.
template <int kKind, int kSplit>
__global__ __launch_bounds__(256) void score_batch_kernel(const BatchArgs A) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeq; ++i)
        if (i < A.n_seq && (int)blockIdx.x >= A.blk0[i]) s = i;
    int n = 0;
    long long k0 = 0;
#pragma unroll
    for (int i = 0; i < kMaxSeq; ++i)
        if (i == s) {
            n = A.n_comp[i];
            k0 = A.key0[i];
        }
    int first = 0;
#pragma unroll
    for (int i = 0; i < kMaxSeq; ++i)
        if (i == s) first = A.blk0[i];
    const int c = ((int)blockIdx.x - first) * (kSplit == 1 ? 256 : 128) + (int)threadIdx.x / kSplit;
    __shared__ __attribute__((aligned(16))) float qs[kMaxHeads * kQStride];
    __shared__ float ws[kMaxHeads];
    const float *qg = A.q + (size_t)s * A.n_head * kMaxDim;
    const float *wg = A.w + (size_t)s * A.n_head;
    if (kSplit == 1)
        stage_query(qs, qg, A.n_head);
    else
        stage_query<kQStride>(qs, qg, A.n_head);
    for (int i = threadIdx.x; i < A.n_head; i += 256) ws[i] = wg[i];
    if (kSplit == 1) pad_heads(qs, ws, A.n_head);
    __syncthreads();
    if (c >= n) return;   // the kSplit lanes of a key leave together
    if (kSplit == 1) {
        A.scores[k0 + c] = score_lds<kKind>(qs, ws, A.keys, (int)(k0 + c), A.n_head);
    } else {
        // keys c and c + 64 of this block's 128
        const int c1 = c + 64;
        float s0, s1;
        score_chain4x2<kKind>(qs, ws, A.keys, (int)(k0 + c), (int)(k0 + (c1 < n ? c1 : c)), A.n_head,
                              (int)threadIdx.x % kSplit, s0, s1);
        if (threadIdx.x % kSplit == kSplit - 1) {
            A.scores[k0 + c] = s0;
            if (c1 < n) A.scores[k0 + c1] = s1;
        }
    }
}

__device__ inline unsigned scan1024_excl(unsigned v, unsigned *wsum, unsigned *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    unsigned x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned u = __shfl_up(x, off);
        if (lane >= off) x += u;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    unsigned before = 0, tot = 0;
    for (int i = 0; i < 16; ++i) {
        const unsigned t = wsum[i];
        before += i < wv ? t : 0;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return before + x - v;
}

__global__ __launch_bounds__(1024) void select_batch_kernel(const BatchArgs A) {
    __shared__ unsigned keys[kSelMax];
    __shared__ unsigned hist[256];
    __shared__ unsigned wsum[16];
    __shared__ unsigned s_bin, s_above;
    const int s = blockIdx.x;
    int n = 0;
    long long k0 = 0;
#pragma unroll
    for (int i = 0; i < kMaxSeq; ++i)
        if (i == s) {
            n = A.n_comp[i];
            k0 = A.key0[i];
        }
    int32_t *out = A.pos_out + (size_t)s * A.pos_stride;
    const int t = threadIdx.x;
    if (n <= A.top_k) {
        for (int i = t; i < n; i += 1024) out[i] = i;
        return;
    }
    const int recent = A.n_recent < A.top_k ? A.n_recent : A.top_k;
    const int n_cand = n - recent;
    const unsigned need0 = (unsigned)(A.top_k - recent);
    for (int i = t; i < n_cand; i += 1024) keys[i] = ord_key(A.scores[k0 + i]);
    // radix select of the need0-th largest key, 8 bits at a time
    unsigned prefix = 0, pmask = 0, need = need0;
    for (int shift = 24; shift >= 0 && need > 0; shift -= 8) {
        if (t < 256) hist[t] = 0;
        __syncthreads();
        for (int i = t; i < n_cand; i += 1024) {
            const unsigned k = keys[i];
            if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255], 1u);
        }
        __syncthreads();
        // bins from the top: thread b < 256 owns bin 255 - b
        const unsigned v = t < 256 ? hist[255 - t] : 0;
        unsigned tot;
        const unsigned ex = scan1024_excl(v, wsum, &tot);
        if (t < 256 && ex < need && ex + v >= need) {
            s_bin = 255 - t;
            s_above = ex;
        }
        __syncthreads();
        prefix |= s_bin << shift;
        pmask |= 255u << shift;
        need -= s_above;
        __syncthreads();
    }
    // need0 == 0 leaves T above every key
    const unsigned T = need0 ? prefix : 0xFFFFFFFFu;
    const unsigned need_eq = need0 ? need : 0;
    // emit in index order: thread t owns a contiguous range
    const int per = (n_cand + 1023) / 1024;
    const int b0 = t * per, b1 = min(b0 + per, n_cand);
    unsigned n_eq = 0;
    for (int i = b0; i < b1; ++i) n_eq += keys[i] == T;
    unsigned tot_eq;
    unsigned eq_rank = scan1024_excl(n_eq, wsum, &tot_eq);
    unsigned n_sel = 0;
    {
        unsigned r = eq_rank;
        for (int i = b0; i < b1; ++i) {
            const unsigned k = keys[i];
            if (k > T) ++n_sel;
            else if (k == T) { n_sel += r < need_eq; ++r; }
        }
    }
    unsigned tot_sel;
    unsigned o = scan1024_excl(n_sel, wsum, &tot_sel);
    {
        unsigned r = eq_rank;
        for (int i = b0; i < b1; ++i) {
            const unsigned k = keys[i];
            bool take = k > T;
            if (k == T) { take = r < need_eq; ++r; }
            if (take) out[o++] = i;
        }
    }
    for (int i = t; i < recent; i += 1024) out[tot_sel + i] = n_cand + i;
}

}  // namespace

extern "C" int ds4hip_indexer_topk_positions_batch(
        const float *q, const float *weights, const void *keys, int key_kind,
        const long long *key_row0_host, const int *n_comp_host, int n_seq, int n_head,
        int head_dim, int top_k, int n_recent, float *scratch_scores, int32_t *positions_out,
        int pos_stride, void *stream) {
    if (!q || !weights || !keys || !key_row0_host || !n_comp_host || !scratch_scores ||
        !positions_out || key_kind < 0 || key_kind > 2 || n_seq <= 0 || n_seq > kMaxSeq ||
        n_head <= 0 || n_head > kMaxHeads || head_dim != kMaxDim || top_k <= 0 || n_recent < 0 ||
        pos_stride < top_k)
        return ds4hip_set_last_error(kEINVAL);
    BatchArgs A;
    A.q = q;
    A.w = weights;
    A.keys = keys;
    A.scores = scratch_scores;
    A.pos_out = positions_out;
    A.n_seq = n_seq;
    A.n_head = n_head;
    A.top_k = top_k;
    A.n_recent = n_recent;
    A.pos_stride = pos_stride;
    // four threads per key, two keys per thread group (128 keys per block)
    const bool split = true;   // the chained four-thread form works for any n_head
    const int keys_per_blk = split ? 128 : 256;
    int blk = 0;
    for (int s = 0; s < kMaxSeq; ++s) {
        const int n = s < n_seq ? n_comp_host[s] : 0;
        if (n < 0 || (n > top_k && n - (n_recent < top_k ? n_recent : top_k) > kSelMax))
            return ds4hip_set_last_error(kEINVAL);
        A.n_comp[s] = n;
        A.key0[s] = s < n_seq ? key_row0_host[s] : 0;
        A.blk0[s] = blk;
        // only sequences that need a selection are scored
        if (s < n_seq && n > top_k) blk += (n + keys_per_blk - 1) / keys_per_blk;
    }
    A.blk0[kMaxSeq] = blk;
    const hipStream_t st = (hipStream_t)stream;
    if (blk > 0) {
        const dim3 g(blk), b(256);
        switch (key_kind) {
        case 0:
            if (split) hipLaunchKernelGGL((score_batch_kernel<0, 4>), g, b, 0, st, A);
            else hipLaunchKernelGGL((score_batch_kernel<0, 1>), g, b, 0, st, A);
            break;
        case 1:
            if (split) hipLaunchKernelGGL((score_batch_kernel<1, 4>), g, b, 0, st, A);
            else hipLaunchKernelGGL((score_batch_kernel<1, 1>), g, b, 0, st, A);
            break;
        default:
            if (split) hipLaunchKernelGGL((score_batch_kernel<2, 4>), g, b, 0, st, A);
            else hipLaunchKernelGGL((score_batch_kernel<2, 1>), g, b, 0, st, A);
            break;
        }
    }
    hipLaunchKernelGGL(select_batch_kernel, dim3(n_seq), dim3(1024), 0, st, A);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
