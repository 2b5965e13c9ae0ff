// indexer.hip — lightning-indexer scores and exact top-k selection.
//
// Scores (cuda/indexer_allowed.cu:68-171): score[c] = sum_h w[h] relu(q_h . k_c),
// computed with the reference kernel's own operations so that scores and the
// selected positions are bit-identical to it. The reference runs one block per
// key, thread h = head h:
//   dot_h = fma chain over d ascending from 0.0f (`dot += q * k`, contracted);
//   relu `dot < 0 ? 0 : dot`; partial_h = dot_h * w[h] (a rounded product);
//   each 32-head warp adds its partials with an xor butterfly (16, 8, 4, 2, 1),
//   warp 0 combines the warp sums with an xor butterfly over 8 lanes (4, 2, 1;
//   lanes past the last warp hold 0.0f).
// Here one thread scores one key (the key row in registers, the query in LDS)
// and evaluates the same tree: a butterfly's lane-0 result is a balanced
// binary tree whose leaves, left to right, are the heads in bit-reversed
// order (h, h + 16, h + 8, h + 24, ...), so feeding the products in that
// order to a five-level carry chain (HeadTree) adds exactly the reference's
// pairs. Floating-point contraction is off in this file: every product and
// sum rounds where the reference's does; the dot chains call fmaf.
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

#pragma clang fp contract(off)

namespace {

constexpr int kMaxHeads = 64;
constexpr int kMaxDim = 128;
constexpr int kQStride = kMaxDim + 4;   // query row stride in LDS for the four-thread form
constexpr int kBins = 2048;
constexpr int kBatchKeys = 128;   // keys per workgroup of the four-lane scorer
constexpr int kSmallSelect = 16384;   // candidates one workgroup selects in LDS (the batched select's limit)

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
        v[i] = reinterpret_cast<const float4_t *>(q)[min(k, n4 - 1)];   // clamped: no branch between the loads
    }
#pragma unroll
    for (int i = 0; i < kMaxHeads * kMaxDim / 4 / 256; ++i) {
        const int k = (int)threadIdx.x + 256 * i;
        if (k < n4)
            *reinterpret_cast<float4_t *>(qs + (k / (kMaxDim / 4)) * kStride + 4 * (k % (kMaxDim / 4))) = v[i];
    }
}

// Zero query rows and weights for the heads past n_head up to the next
// multiple of 32 (a whole warp of the reference's block). Their products are
// replaced by 0.0f anyway, as the reference's idle threads contribute.
__device__ inline void pad_heads(float *qs, float *ws, int n_head, int stride = kMaxDim) {
    const int n32 = (n_head + 31) & ~31;
    for (int i = threadIdx.x; i < (n32 - n_head) * kMaxDim; i += 256)
        qs[(n_head + i / kMaxDim) * stride + i % kMaxDim] = 0.0f;
    if ((int)threadIdx.x < n32 - n_head) ws[n_head + threadIdx.x] = 0.0f;
}

// The reference's head sum (see the top of the file), fed one leaf at a time
// in leaf order: leaf t of warp t >> kLevels. A leaf is one head's product
// (kLevels = 5) or the sum of a group of four heads h, h + 16, h + 8, h + 24
// (kLevels = 3, the butterfly's first two levels already added). An odd leaf
// index closes a pair with the level below, like a binary counter's carry.
template <int kLevels>
struct HeadTree {
    float l[kLevels];
    float w0 = 0.0f, w1 = 0.0f;
    // branch-free (t is uniform, but branches here cost the caller's
    // registers): every level's sum is formed and selects keep the right ones
    __device__ inline void push(int t, float v) {
        bool carry = true;   // v still travels up
#pragma unroll
        for (int k = 0; k < kLevels; ++k) {
            const bool odd = (t >> k) & 1;
            const float up = l[k] + v;
            l[k] = (carry && !odd) ? v : l[k];
            carry = carry && odd;
            v = up;
        }
        const bool w_is_1 = (t >> kLevels) & 1;
        w0 = (carry && !w_is_1) ? v : w0;
        w1 = (carry && w_is_1) ? v : w1;
    }
    // warp 0's 8-lane butterfly over (w0, w1, 0, ..., 0): lane 0 gets
    // ((w0 + 0) + 0) + ((w1 + 0) + 0); x + 0 + 0 == x + 0
    __device__ inline float result() const { return (w0 + 0.0f) + (w1 + 0.0f); }
};

// Head of leaf t in the 5-level order: bits 0..4 reversed within the warp.
__device__ inline int head_of_leaf(int t) {
    return (t & ~31) | (int)(__builtin_bitreverse32((unsigned)(t & 31)) >> 27);
}
// First head of four-head group g: the 3 low bits of g reversed.
__device__ inline int head_of_group(int g) {
    return (g & ~7) * 4 + (int)(__builtin_bitreverse32((unsigned)(g & 7)) >> 29);
}

// relu and the rounded product of one head (cuda/indexer_allowed.cu:89-90)
__device__ inline float head_partial(float dot, float w) {
    if (dot < 0.0f) dot = 0.0f;
    return dot * w;
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
    // four heads at a time (four independent dot chains keep the VALU busy):
    // group g = heads h, h + 16, h + 8, h + 24 of one warp, whose products
    // the butterfly's first two levels add as ((p_h + p_h+16) + (p_h+8 + p_h+24))
    HeadTree<3> tree;
    const int n_groups = ((n_head + 31) & ~31) / 4;
    for (int g = 0; g < n_groups; ++g) {
        const int h = head_of_group(g);
        float v = 0.0f;
        if (h < n_head) {   // else all four heads are idle threads of the reference
            const float4_t *q0 = reinterpret_cast<const float4_t *>(qs + h * kMaxDim);
            constexpr int kOff[4] = {0, 16, 8, 24};
            float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            // the query reads run kAhead steps ahead of their use (LDS returns
            // in order; with two waves per SIMD nothing else hides the latency)
            constexpr int kAhead = 3;
            float4_t a[kAhead][4];
#pragma unroll
            for (int v4 = 0; v4 < kAhead; ++v4)
#pragma unroll
                for (int z = 0; z < 4; ++z) a[v4][z] = q0[kOff[z] * (kMaxDim / 4) + v4];
#pragma unroll
            for (int v4 = 0; v4 < kMaxDim / 4; ++v4) {
                float4_t cur[4];
#pragma unroll
                for (int z = 0; z < 4; ++z) cur[z] = a[v4 % kAhead][z];
                if (v4 + kAhead < kMaxDim / 4) {
#pragma unroll
                    for (int z = 0; z < 4; ++z) a[v4 % kAhead][z] = q0[kOff[z] * (kMaxDim / 4) + v4 + kAhead];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int z = 0; z < 4; ++z) d[z] = fmaf(cur[z][e], k[4 * v4 + e], d[z]);
            }
            float p[4];
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                // heads past n_head give +0.0f (the reference's idle threads);
                // their query rows and weights are zero-padded, so the loads
                // stay in bounds, and a bit mask replaces the product
                const float pz = head_partial(d[z], ws[h + kOff[z]]);
                p[z] = __int_as_float(__float_as_int(pz) & (h + kOff[z] < n_head ? ~0 : 0));
            }
            v = (p[0] + p[1]) + (p[2] + p[3]);
        }
        tree.push(g, v);
    }
    return tree.result();
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
// which gives the VALU two dependency chains to interleave. The group runs
// kLeaves consecutive leaves (heads, in bit-reversed order within their
// warp), from leaf0, of the reference's block (a whole warp: 32), and part 3
// returns their subtree of the warp's butterfly for both keys.
template <int kKind, int kLeaves>
__device__ __attribute__((always_inline)) inline void score_chain4x2(const float *qs, const float *ws,
                                                                     const void *__restrict__ keys,
                                                                     int c0, int c1, int n_head, int part,
                                                                     float *pbuf, int kl0, int kl1, int leaf0,
                                                                     float &w0, float &w1) {
    float k0[32], k1[32];
    load_key32<kKind>(keys, c0, part, k0);
    load_key32<kKind>(keys, c1, part, k1);
    float carry0 = 0.0f, carry1 = 0.0f;
    for (int i = 0; i < kLeaves + 3; ++i) {
        const int leaf = leaf0 + i - part;
        const bool in = i - part >= 0 && i - part < kLeaves;
        const int h = in ? head_of_leaf(leaf) : 0;
        const bool act = in && h < n_head;
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
        // the head's product, in leaf order, for the tree below
        if (part == 3 && in) {
            pbuf[leaf * kBatchKeys + kl0] = act ? head_partial(d0, ws[h]) : 0.0f;
            pbuf[leaf * kBatchKeys + kl1] = act ? head_partial(d1, ws[h]) : 0.0f;
        }
    }
    // In leaf order the butterfly of a warp of heads is a balanced tree of
    // adjacent pairs.
    if (part == 3) {
#pragma unroll
        for (int z = 0; z < 2; ++z) {
            const int kl = z ? kl1 : kl0;
            float v[kLeaves];
#pragma unroll
            for (int t = 0; t < kLeaves; ++t) v[t] = pbuf[(leaf0 + t) * kBatchKeys + kl];
#pragma unroll
            for (int n = kLeaves / 2; n >= 1; n >>= 1)
#pragma unroll
                for (int t = 0; t < n; ++t) v[t] = v[2 * t] + v[2 * t + 1];
            (z ? w1 : w0) = v[0];
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
    HeadTree<5> tree;
    const int n_leaves = (n_head + 31) & ~31;
    for (int t = 0; t < n_leaves; ++t) {
        const int h = head_of_leaf(t);
        float p = 0.0f;
        if (h < n_head) {
            const float *qh = qs + h * head_dim;
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < kMaxDim; ++d)
                if (d < head_dim) dot = fmaf(qh[d], k[d], dot);
            p = head_partial(dot, ws[h]);
        }
        tree.push(t, p);
    }
    return tree.result();
}

// kFull: head_dim == 128 (the scalar-load path); otherwise the LDS path. Two
// instantiations so that neither path's registers limit the other's occupancy.
// One key per thread: 131072 keys make two waves per SIMD, so the register
// budget is that of two waves per SIMD, which holds the query reads several
// steps ahead (measured 67 -> 61 us for the indexer over 131072 keys).
template <int kKind, bool kFull>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void score_kernel(const float *__restrict__ q,
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
        stage_to_lds(qs, q, n_head * head_dim);
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

int launch_scores(const float *q, const float *w, const void *keys, int kind, int n_comp,
                  int n_head, int head_dim, float *scores, unsigned *hist, int n_cand,
                  hipStream_t st) {
    const bool full = head_dim == kMaxDim;
    const dim3 grid((n_comp + 255) / 256);
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
size_t select_large_scratch_words(int n_comp);
size_t select_scratch_bytes(int n_comp) {
    const size_t chunks = (size_t)(n_comp > 0 ? n_comp : 1) / kChunk + 1;
    return std::max((3 * kBins + 2 * chunks), select_large_scratch_words(n_comp)) * sizeof(unsigned);
}

int launch_select_large(const float *scores, int n_comp, int n_cand, unsigned need0, unsigned *scratch,
                        int32_t *mask, int32_t *pos_out, hipStream_t st);
size_t select_large_scratch_words(int n_comp);
constexpr int kLargeSelectMax = 262144;   // candidates of the two-launch select (its LDS bitmaps)

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
    // Few candidates and positions only (the model's decode: a few thousand
    // compressed rows): the batched pair with one sequence, four lanes per
    // key and one workgroup's LDS radix select, two launches instead of six;
    // the same scores and the same selection rule.
    if (!mask && head_dim == kMaxDim && n_cand <= kSmallSelect) {
        const long long row0 = 0;
        return ds4hip_indexer_topk_positions_batch(q, w, keys, kind, &row0, &n_comp, 1, n_head, head_dim, top_k,
                                                   n_recent, scores, pos_out, top_k, st);
    }
    const unsigned need0 = (unsigned)(top_k - recent);
    const int n_chunks = (n_comp + kChunk - 1) / kChunk;
    unsigned *hists = scratch;
    unsigned *chunk_gt = scratch + 3 * kBins;
    unsigned *chunk_eq = chunk_gt + n_chunks;
    // up to kLargeSelectMax candidates (16-byte aligned scores): the level-1
    // histogram in the score kernel, then the two-launch select
    if (n_cand <= kLargeSelectMax && (reinterpret_cast<uintptr_t>(scores) & 15) == 0) {
        // level-1 histogram, list counter and bitmap start at zero
        const int nz = kBins + 1 + (n_cand + 31) / 32;
        hipLaunchKernelGGL(zero_u32_kernel, dim3((nz + 255) / 256), dim3(256), 0, st, scratch, nz);
        int rc = launch_scores(q, w, keys, kind, n_comp, n_head, head_dim, scores, scratch, n_cand, st);
        if (rc) return rc;
        return launch_select_large(scores, n_comp, n_cand, need0, scratch, mask, pos_out, st);
    }
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

// The reference launchers take only a score scratch; the selection
// histograms live in the library's per-stream scratch (no allocation once it
// has grown to the size a stream needs).
static int with_hists(int (*fn)(unsigned *, void *), void *ctx, int n_comp, hipStream_t st) {
    void *h = nullptr;
    const int e = stream_scratch(st, select_scratch_bytes(n_comp), &h);
    if (e) return e;
    return fn(static_cast<unsigned *>(h), ctx);
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
// Four chained lanes per key, two keys per lane group, 128 keys per
// workgroup of 2 x 256 threads: thread group g runs the leaves of warp g of
// the reference's block (heads 32 g .. 32 g + 31) for the same keys, so a
// wave's chain is half as long and the launch has twice the waves (cfg-5
// layer-step 195.5 -> 187.2 us; four groups of 16 leaves measured the same);
// the two warp sums meet in LDS for warp 0's combine.
constexpr int kGroups = 2;
constexpr int kHalf = kBatchKeys / 2;            // a lane group's second key: kl + kHalf
constexpr int kGroupThreads = 4 * kHalf;         // threads of one leaf group
template <int kKind>
__global__ __launch_bounds__(kGroupThreads * kGroups) void score_batch_kernel(const BatchArgs A) {
    constexpr int kLeaves = kMaxHeads / kGroups;
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
    const int grp = (int)threadIdx.x / kGroupThreads, tl = (int)threadIdx.x % kGroupThreads;
    const int c = ((int)blockIdx.x - first) * kBatchKeys + tl / 4;
    __shared__ __attribute__((aligned(16))) float qs[kMaxHeads * kQStride];
    __shared__ float ws[kMaxHeads];
    __shared__ float pbuf[kMaxHeads * kBatchKeys];   // [leaf][key of the block]
    __shared__ float sub[kGroups][kBatchKeys];       // subtree sums per key of the block
    const float *qg = A.q + (size_t)s * A.n_head * kMaxDim;
    const float *wg = A.w + (size_t)s * A.n_head;
    if (threadIdx.x < 256) stage_query<kQStride>(qs, qg, A.n_head);
    for (int i = threadIdx.x; i < A.n_head; i += kGroupThreads * kGroups) ws[i] = wg[i];
    __syncthreads();
    const int part = tl % 4;
    const int kl = tl / 4;   // the group's first key within the block; the second is kl + kHalf
    const int c1 = c + kHalf;
    const int n_leaves = (A.n_head + 31) & ~31;   // an absent warp 1 adds +0.0f
    const int leaf0 = grp * kLeaves;
    float s0 = 0.0f, s1 = 0.0f;
    if (c < n && leaf0 < n_leaves)
        score_chain4x2<kKind, kLeaves>(qs, ws, A.keys, (int)(k0 + c), (int)(k0 + (c1 < n ? c1 : c)), A.n_head,
                                       part, pbuf, kl, kl + kHalf, leaf0, s0, s1);
    if (part == 3) {
        sub[grp][kl] = s0;
        sub[grp][kl + kHalf] = s1;
    }
    __syncthreads();
    if (grp == 0 && part == 3 && c < n) {
#pragma unroll
        for (int z = 0; z < 2; ++z) {
            const int k = kl + kHalf * z;
            const float w0 = sub[0][k], w1 = sub[1][k];
            // warp 0's 8-lane butterfly over (w0, w1, 0, ..., 0)
            if (z == 0 || c1 < n) A.scores[k0 + c + kHalf * z] = (w0 + 0.0f) + (w1 + 0.0f);
        }
    }
}

// Lane-per-head scorer (the reference's own layout, cuda/indexer_allowed.cu:
// 68-171: one thread per head): lane h of a wave holds q_h in registers, the
// block's keys sit in LDS as fp32 and are read by broadcast, and a wave scores
// kHeadsKpw keys, two dot chains at a time. The head sum is the reference's
// tree literally: an xor butterfly over each 32-lane half (offsets 16 .. 1),
// then lane 0's and lane 32's warp sums combined as warp 0 combines them.
// Many keys per launch need few registers per key; this form suits a few
// thousand keys, where one thread per key would leave most CUs idle.
// Two keys per wave (one pair of chains) gives the most workgroups; eight
// measured 135 us slower per token over 43 layers at context 4096.
constexpr int kHeadsKpw = 2;                    // keys per wave
constexpr int kHeadsKpb = 4 * kHeadsKpw;        // keys per workgroup
// Up to this many keys per launch. Measured (one sequence, 64 heads, fp32
// keys): this form 5.2 / 8.6 / 12.4 / 22.0 us at 1500 / 3000 / 6000 / 12000
// keys, the four-lane form 19.3 / 19.6 / 20.0 us at 3000 / 6000 / 12000.
constexpr long long kHeadsMaxKeys = 10240;
template <int kKind>
__global__ __launch_bounds__(256) void score_heads_kernel(const BatchArgs A) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeq; ++i)
        if (i < A.n_seq && (int)blockIdx.x >= A.blk0[i]) s = i;
    int n = 0, first = 0;
    long long k0 = 0;
#pragma unroll
    for (int i = 0; i < kMaxSeq; ++i)
        if (i == s) {
            n = A.n_comp[i];
            k0 = A.key0[i];
            first = A.blk0[i];
        }
    const int c0 = ((int)blockIdx.x - first) * kHeadsKpb;
    __shared__ __attribute__((aligned(16))) float qs[kMaxHeads * kQStride];
    __shared__ __attribute__((aligned(16))) float ks[kHeadsKpb * kMaxDim];
    const float *qg = A.q + (size_t)s * A.n_head * kMaxDim;
    stage_query<kQStride>(qs, qg, A.n_head);
    // the block's keys, widened to fp32 (rows past n are zeros, never stored):
    // 16-byte loads, all issued before any is used (rows past n load row
    // n - 1, so there is no branch between them)
    constexpr int kEsz = kKind == 0 ? 4 : 2;
    constexpr int kPer = 16 / kEsz;                    // elements per load
    constexpr int kRowVecs = kMaxDim / kPer;
    constexpr int kLoads = (kHeadsKpb * kRowVecs + 255) / 256;
    const int rows_here = min(n - c0, kHeadsKpb);
    const char *kbase = static_cast<const char *>(A.keys) + (size_t)(k0 + c0) * kMaxDim * kEsz;
    if (rows_here > 0 && (reinterpret_cast<uintptr_t>(kbase) & 15) == 0) {
        uint4_t kv[kLoads];
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int vi = (int)threadIdx.x + 256 * u;
            const int kr = min(vi / kRowVecs, rows_here - 1);
            kv[u] = reinterpret_cast<const uint4_t *>(kbase)[kr * kRowVecs + vi % kRowVecs];
        }
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int vi = (int)threadIdx.x + 256 * u;
            if (vi >= kHeadsKpb * kRowVecs) break;   // a block of few bf16 rows: fewer vectors than threads
            const bool in = vi / kRowVecs < rows_here;
            float f[kPer];
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const uint32_t w = kv[u][e * kEsz / 4];
                const uint16_t h = (uint16_t)(e & 1 ? w >> 16 : w & 0xFFFF);
                f[e] = kKind == 0 ? __uint_as_float(kv[u][e]) : (kKind == 1 ? f16_bits_to_f32(h) : bf16_to_f32(h));
                f[e] = in ? f[e] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < kPer; e += 4)
                *reinterpret_cast<float4_t *>(ks + vi * kPer + e) = float4_t{f[e], f[e + 1], f[e + 2], f[e + 3]};
        }
    } else {
        for (int i = threadIdx.x; i < kHeadsKpb * kMaxDim; i += 256) {
            const int kr = i / kMaxDim, d = i % kMaxDim;
            ks[i] = c0 + kr < n ? key_elem<kKind>(A.keys, (size_t)(k0 + c0 + kr) * kMaxDim + d) : 0.0f;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane;
    const bool live = h < A.n_head;
    float q[kMaxDim];
#pragma unroll
    for (int v = 0; v < kMaxDim / 4; ++v) {
        const float4_t t = *reinterpret_cast<const float4_t *>(qs + (live ? h : 0) * kQStride + 4 * v);
#pragma unroll
        for (int e = 0; e < 4; ++e) q[4 * v + e] = t[e];
    }
    const float wh = live ? A.w[(size_t)s * A.n_head + h] : 0.0f;
#pragma unroll 1
    for (int kk = wave * kHeadsKpw; kk < (wave + 1) * kHeadsKpw; kk += 2) {
        if (c0 + kk >= n) break;
        float dot[2] = {0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < kMaxDim / 4; ++v) {
            float4_t kv[2];
#pragma unroll
            for (int z = 0; z < 2; ++z) kv[z] = *reinterpret_cast<const float4_t *>(ks + (kk + z) * kMaxDim + 4 * v);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int z = 0; z < 2; ++z) dot[z] = fmaf(q[4 * v + e], kv[z][e], dot[z]);
        }
#pragma unroll
        for (int z = 0; z < 2; ++z) {
            // idle heads (the reference's threads h >= n_head) add +0.0f
            float v = __int_as_float(__float_as_int(head_partial(dot[z], wh)) & (live ? ~0 : 0));
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) v = v + __shfl_xor(v, off);
            const float w0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
            const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
            // warp 0's 8-lane butterfly over (w0, w1, 0, ...): lanes of an
            // absent warp hold +0.0f, which (w1 + 0) reproduces
            const float score = (w0 + 0.0f) + (w1 + 0.0f);
            const int c = c0 + kk + z;
            if (lane == 0 && c < n) A.scores[k0 + c] = score;
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

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ inline unsigned wave_scan_incl(unsigned x) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned y = __shfl_up(x, off);
        x += lane >= off ? y : 0u;
    }
    return x;
}

// Exclusive prefix sum over a 1024-thread workgroup of small per-thread
// values (below 32): within a wave from ballots of the values' bit planes (no
// lane shuffles), then the 16 wave totals through LDS with one barrier. ws is
// this scan's own 16 words (not reused by another scan of the launch).
__device__ inline unsigned scan1024_small(unsigned v, unsigned *ws, unsigned *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    unsigned below = 0, wtot = 0;
#pragma unroll
    for (int b = 0; b < 5; ++b) {
        const unsigned long long m = __ballot((v >> b) & 1u);
        below += __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u)) << b;
        wtot += (unsigned)__popcll(m) << b;
    }
    if (lane == 0) ws[wv] = wtot;
    __syncthreads();
    unsigned before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const unsigned x = ws[i];
        before += i < wv ? x : 0u;
        tot += x;
    }
    *total = tot;
    return before + below;
}

__global__ __launch_bounds__(1024) void select_batch_kernel(const BatchArgs A) {
    __shared__ unsigned keys[kSelMax];
    __shared__ __attribute__((aligned(16))) unsigned hist[2][256];
    __shared__ unsigned wemit[2][16];
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
    // four loads in flight per thread (clamped, not branched): a strided copy
    // loop would wait for each load in turn
    for (int b = 0; b < n_cand; b += 4096) {
        unsigned v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = ord_key(A.scores[k0 + min(b + 1024 * u + t, n_cand - 1)]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (b + 1024 * u + t < n_cand) keys[b + 1024 * u + t] = v[u];
    }
    // radix select of the need0-th largest key, 8 bits at a time. Two
    // histograms alternate by pass, so a pass is two barriers: every wave
    // reads the whole histogram (4 bins per lane) and finds the threshold
    // bin itself with a lane scan; the next pass's histogram is cleared
    // meanwhile (its last reads were before this pass's first barrier).
    if (t < 256) hist[0][t] = 0;
    unsigned prefix = 0, pmask = 0, need = need0;
    for (int shift = 24, p = 0; shift >= 0 && need > 0; shift -= 8, ++p) {
        unsigned *h = hist[p & 1];
        __syncthreads();
        for (int i = t; i < n_cand; i += 1024) {
            const unsigned k = keys[i];
            if ((k & pmask) == prefix) atomicAdd(&h[(k >> shift) & 255], 1u);
        }
        __syncthreads();
        if (t < 256) hist[(p + 1) & 1][t] = 0;
        const int lane = t & 63;
        // lane l: bins 255 - 4l down to 252 - 4l
        const uint4_t c4 = *reinterpret_cast<const uint4_t *>(h + 252 - 4 * lane);
        const unsigned ls = c4[0] + c4[1] + c4[2] + c4[3];
        const unsigned cum = wave_scan_incl(ls);
        const int L = __builtin_ctzll(__ballot(cum >= need));
        unsigned acc = cum - ls, bin = 0, above = 0;
        bool found = false;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const unsigned v = c4[i];
            if (!found && acc + v >= need) {
                found = true;
                bin = (unsigned)(252 - 4 * lane + i);
                above = acc;
            }
            acc += v;
        }
        prefix |= (unsigned)__builtin_amdgcn_readlane((int)bin, L) << shift;
        pmask |= 255u << shift;
        need -= (unsigned)__builtin_amdgcn_readlane((int)above, L);
    }
    if (need0 == 0) __syncthreads();   // the keys' stores, otherwise ordered by the passes' barriers
    // need0 == 0 leaves T above every key
    const unsigned T = need0 ? prefix : 0xFFFFFFFFu;
    const unsigned need_eq = need0 ? need : 0;
    // emit in index order: thread t owns a contiguous range
    const int per = (n_cand + 1023) / 1024;
    const int b0 = t * per, b1 = min(b0 + per, n_cand);
    unsigned n_eq = 0;
    for (int i = b0; i < b1; ++i) n_eq += keys[i] == T;
    unsigned tot_eq;
    // per <= 16 keys per thread: the counts are small
    unsigned eq_rank = scan1024_small(n_eq, wemit[0], &tot_eq);
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
    unsigned o = scan1024_small(n_sel, wemit[1], &tot_sel);
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

// ---- two-launch selection of a long candidate list ----------------------------------------
//
// After the score kernel's level-1 histogram (key bits 31..21):
//  compact (one workgroup per 1024 candidates, coalesced): keys above the
//    level-1 threshold bin set their bit in a global bitmap; keys in the bin
//    are appended, unordered, to a global list of (key, index) pairs (one
//    counter add per wave);
//  finish (one 1024-thread workgroup): levels 2 (bits 20..10) and 3 (bits
//    9..0) of the radix select over the listed keys give the exact threshold
//    key T and the number of ties at T to take; listed keys above T join the
//    bitmap (copied to LDS), keys equal to T go to a tie bitmap whose
//    popcount scan ranks them by index, and the need_eq lowest join too; a
//    popcount scan of the bitmap writes the positions in ascending order (and
//    / or the 0/1 mask), then the forced recent window.
// Two launches instead of four, and the full score list is read once more
// instead of three times. The list has room for every candidate, so a
// threshold bin of any size is handled (a large one only costs list reads).
constexpr int kLargeBits = 262144;   // candidates the finishing workgroup's LDS bitmaps cover
constexpr int kFinishPairs = 8192;   // listed keys it copies to LDS (a longer list is read from memory)

__global__ __launch_bounds__(256) void compact_kernel(const float *__restrict__ scores, int n_cand,
                                                      unsigned need0, const unsigned *__restrict__ hist1,
                                                      unsigned *__restrict__ bitmap,
                                                      unsigned *__restrict__ list_n,
                                                      unsigned *__restrict__ list_key,
                                                      int *__restrict__ list_idx) {
    __shared__ unsigned scratch[256];
    __shared__ unsigned s_bin, s_above;
    if (need0 == 0) return;
    find_bin(hist1, kBins, need0, &s_bin, &s_above, scratch);
    const unsigned b1 = s_bin;
    const int c = blockIdx.x * kChunk + 4 * threadIdx.x;
    unsigned k[4];
    if (c + 3 < n_cand) {
        const float4_t v = *reinterpret_cast<const float4_t *>(scores + c);
#pragma unroll
        for (int j = 0; j < 4; ++j) k[j] = ord_key(v[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) k[j] = c + j < n_cand ? ord_key(scores[c + j]) : 0;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // in-bin keys: per-wave ballots, one counter add per workgroup (a counter
    // add per wave would serialize ~1000 same-address atomics)
    __shared__ unsigned s_wcnt[4][4], s_base;
    unsigned long long bal[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool live = c + j < n_cand;
        const unsigned hb = k[j] >> 21;
        if (live && hb > b1) atomicOr(&bitmap[(c + j) >> 5], 1u << ((c + j) & 31));
        bal[j] = __ballot(live && hb == b1);
        if (lane == 0) s_wcnt[wv][j] = (unsigned)__popcll(bal[j]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned tot = 0;
        for (int w = 0; w < 4; ++w)
            for (int j = 0; j < 4; ++j) {
                const unsigned n = s_wcnt[w][j];
                s_wcnt[w][j] = tot;   // exclusive prefix in (wave, j) order
                tot += n;
            }
        s_base = tot ? atomicAdd(list_n, tot) : 0;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if ((bal[j] >> lane) & 1) {
            const unsigned o = s_base + s_wcnt[wv][j] + (unsigned)__popcll(bal[j] & ((1ULL << lane) - 1));
            list_key[o] = k[j];
            list_idx[o] = c + j;
        }
}

__global__ __launch_bounds__(1024) void finish_kernel(int n_comp, int n_cand, unsigned need0,
                                                      const unsigned *__restrict__ hist1,
                                                      const unsigned *__restrict__ bitmap,
                                                      const unsigned *__restrict__ list_n,
                                                      const unsigned *__restrict__ list_key,
                                                      const int *__restrict__ list_idx,
                                                      int32_t *__restrict__ mask,
                                                      int32_t *__restrict__ pos_out) {
    __shared__ unsigned sel[kLargeBits / 32];
    __shared__ unsigned tie[kLargeBits / 32];
    __shared__ unsigned hist[kBins];
    __shared__ unsigned lkey[kFinishPairs];
    __shared__ int lidx[kFinishPairs];
    __shared__ unsigned wsum[16];
    __shared__ unsigned s_bin, s_above;
    const int t = threadIdx.x;
    const int n_words = (n_cand + 31) / 32;
    // the independent loads first (bitmap, level-1 histogram, list length),
    // so their latencies overlap; then the list, once
    const unsigned np = need0 ? *list_n : 0;
    if (need0)
        for (int i = t; i < kBins; i += 1024) hist[i] = hist1[i];
    for (int i = t; i < n_words; i += 1024) {
        sel[i] = need0 ? bitmap[i] : 0;
        tie[i] = 0;
    }
    const bool in_lds = np <= (unsigned)kFinishPairs;
    if (in_lds)
        for (unsigned i = t; i < np; i += 1024) {
            lkey[i] = list_key[i];
            lidx[i] = list_idx[i];
        }
    __syncthreads();
    const unsigned *keys_l = in_lds ? lkey : list_key;
    const int *idx_l = in_lds ? lidx : list_idx;
    // the bin of histogram h (nb bins, high bin = larger keys) that holds the
    // need-th largest key, and the count above it (thread t owns nb / 1024
    // bins from the top)
    auto find = [&](const unsigned *h, int nb, unsigned need) {
        const int per = nb / 1024;
        unsigned v = 0;
        for (int i = 0; i < per; ++i) v += h[nb - 1 - t * per - i];
        unsigned tot;
        const unsigned ex = scan1024_excl(v, wsum, &tot);
        if (ex < need && ex + v >= need) {
            unsigned run = ex;
            int b = nb - 1 - t * per;
            for (int i = 0; i < per - 1; ++i, --b) {
                if (run + h[b] >= need) break;
                run += h[b];
            }
            s_bin = (unsigned)b;
            s_above = run;
        }
        __syncthreads();
    };
    const int wpt = (n_words + 1023) / 1024;   // thread t owns words [t * wpt, (t + 1) * wpt)
    const int w0 = t * wpt, w1 = min(w0 + wpt, n_words);
    if (need0 > 0) {
        find(hist, kBins, need0);
        const unsigned b1 = s_bin;
        unsigned need = need0 - s_above;
        unsigned pref = b1 << 21, pmask = 0xFFE00000u;
        for (int lvl = 0; lvl < 2; ++lvl) {
            const int shift = lvl == 0 ? 10 : 0, nb = lvl == 0 ? kBins : 1024;
            __syncthreads();   // the previous level's readers of s_bin are done
            for (int i = t; i < nb; i += 1024) hist[i] = 0;
            __syncthreads();
            for (unsigned i = t; i < np; i += 1024) {
                const unsigned k = keys_l[i];
                if ((k & pmask) == pref) atomicAdd(&hist[(k >> shift) & (nb - 1)], 1u);
            }
            __syncthreads();
            find(hist, nb, need);
            pref |= s_bin << shift;
            pmask |= (unsigned)(nb - 1) << shift;
            need -= s_above;
        }
        const unsigned T = pref, need_eq = need;
        for (unsigned i = t; i < np; i += 1024) {
            const unsigned k = keys_l[i];
            const int c = idx_l[i];
            if (k > T) atomicOr(&sel[c >> 5], 1u << (c & 31));
            else if (k == T) atomicOr(&tie[c >> 5], 1u << (c & 31));
        }
        __syncthreads();
        // the need_eq ties of lowest index
        unsigned nt = 0;
        for (int w = w0; w < w1; ++w) nt += __popc(tie[w]);
        unsigned tot;
        unsigned rank = scan1024_excl(nt, wsum, &tot);
        for (int w = w0; w < w1; ++w) {
            unsigned bits = tie[w], add = 0;
            while (bits && rank < need_eq) {
                const unsigned low = bits & (0u - bits);
                add |= low;
                bits ^= low;
                ++rank;
            }
            sel[w] |= add;   // this thread's words only
        }
        __syncthreads();
    }
    unsigned ns = 0;
    for (int w = w0; w < w1; ++w) ns += __popc(sel[w]);
    unsigned tot;
    unsigned o = scan1024_excl(ns, wsum, &tot);
    for (int w = w0; w < w1; ++w) {
        unsigned bits = sel[w];
        if (mask)
            for (int b = 0; b < 32 && w * 32 + b < n_cand; ++b) mask[w * 32 + b] = (bits >> b) & 1u;
        if (pos_out)
            while (bits) {
                const int b = __builtin_ctz(bits);
                bits &= bits - 1;
                pos_out[o++] = w * 32 + b;
            }
    }
    for (int i = t; i < n_comp - n_cand; i += 1024) {
        if (pos_out) pos_out[need0 + i] = n_cand + i;
        if (mask) mask[n_cand + i] = 1;
    }
}

// scratch: [hist1 kBins][list_n 1][bitmap words][list keys n_cand][list idx n_cand] (u32)
size_t select_large_scratch_words(int n_comp) {
    const size_t n = (size_t)(n_comp > 0 ? n_comp : 1);
    return kBins + 1 + (n + 31) / 32 + 2 * n;
}

int launch_select_large(const float *scores, int n_comp, int n_cand, unsigned need0, unsigned *scratch,
                        int32_t *mask, int32_t *pos_out, hipStream_t st) {
    unsigned *hist1 = scratch, *list_n = scratch + kBins, *bitmap = list_n + 1;
    const int n_words = (n_cand + 31) / 32;
    unsigned *list_key = bitmap + n_words;
    int *list_idx = reinterpret_cast<int *>(list_key + n_cand);
    hipLaunchKernelGGL(compact_kernel, dim3((n_cand + kChunk - 1) / kChunk), dim3(256), 0, st, scores, n_cand,
                       need0, hist1, bitmap, list_n, list_key, list_idx);
    hipLaunchKernelGGL(finish_kernel, dim3(1), dim3(1024), 0, st, n_comp, n_cand, need0, hist1, bitmap, list_n,
                       list_key, list_idx, mask, pos_out);
    return hip_status(hipGetLastError());
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
    // Few keys in all: one wave per kHeadsKpw keys, lane = head
    // (score_heads_kernel), which fills the chip where one group of lanes per
    // key would not. Many keys: four chained lanes per key (score_batch_kernel).
    long long n_scored = 0;
    for (int s = 0; s < n_seq; ++s)
        if (n_comp_host[s] > top_k) n_scored += n_comp_host[s];
    const bool heads = n_scored <= kHeadsMaxKeys;
    const int keys_per_blk = heads ? kHeadsKpb : kBatchKeys;
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
            if (heads) hipLaunchKernelGGL(score_heads_kernel<0>, g, b, 0, st, A);
            else hipLaunchKernelGGL(score_batch_kernel<0>, g, dim3(kGroupThreads * kGroups), 0, st, A);
            break;
        case 1:
            if (heads) hipLaunchKernelGGL(score_heads_kernel<1>, g, b, 0, st, A);
            else hipLaunchKernelGGL(score_batch_kernel<1>, g, dim3(kGroupThreads * kGroups), 0, st, A);
            break;
        default:
            if (heads) hipLaunchKernelGGL(score_heads_kernel<2>, g, b, 0, st, A);
            else hipLaunchKernelGGL(score_batch_kernel<2>, g, dim3(kGroupThreads * kGroups), 0, st, A);
            break;
        }
    }
    hipLaunchKernelGGL(select_batch_kernel, dim3(n_seq), dim3(1024), 0, st, A);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
