// flash_attn.hip — single-query (decode) attention with attention sinks on
// gfx950 MFMA, for the FP8 E4M3FN KV cache and for the reference's fp32 rows.
//
// Math (cuda/flash_attn.cuh:9-26,90-117): per head h,
//   out_h = sum_k exp(s_k - M) V_k / (exp(sink_h - M) + sum_k exp(s_k - M)),
//   s_k = (q_h . K_k) / sqrt(head_dim), K == V (one latent KV head, MLA),
// K/V elements f16-rounded on read, masked rows contribute nothing.
//
// Work split. The rows of all problems (layers or sequences) are concatenated
// and cut into equal chunks, one per 256-thread workgroup (stream-K): a
// workgroup whose chunk crosses a problem boundary emits one partial
// (m, l, O) per problem it touched. A second kernel merges the partials of
// each problem with the sink. Each workgroup covers all 64 heads: wave w owns
// heads [16w, 16w+16), so every KV row is dequantized and used by 4 waves.
//
// Per 32-row tile, per wave:
//   S^T[32 rows x 16 heads] = K[32 x 512] . Q^T  — v_mfma_f32_16x16x32_f16,
//     A = K fragments loaded straight from HBM into registers (lane = row,
//     16 consecutive dims), dequantized with v_cvt_scalef32_pk_f16_fp8;
//     B = Q^T held in registers for the whole chunk;
//   online softmax in the exp2 domain, P kept in registers: the S^T output
//     layout (lane = head, 4+4 rows) is already the A layout of P . V;
//   O[16 heads x 512] += P[16 x 32] . V[32 x 512] — B = V^T fragments read
//     from LDS as 16-byte vectors. The V^T tile is written once per workgroup:
//     wave w transposes dims [128w, 128w+128) from the registers it already
//     holds.
// Rows inside a V^T line are stored in the order the P fragment uses
// (row 4a+c of half-tile t at position 8a+4t+c), so each B fragment is one
// contiguous 16-byte LDS read.

#include "ds4hip_common.h"
#include "../../include/ds4hip.h"

#include <algorithm>
#include <cstddef>
#include <vector>

using namespace ds4hip;

namespace {

constexpr int kH = 64;           // query heads
constexpr int kD = 512;          // head dim
constexpr int kRot = 64;         // RoPE tail dims (stored f16 in the FP8 cache)
constexpr int kNope = kD - kRot; // 448 FP8-coded dims, 7 scale blocks
constexpr int kTile = 32;        // rows per tile
constexpr int kVtStride = 40;    // halves per V^T line (32 rows + 8 pad)
constexpr int kMaxProb = 128;
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeArgs {
    const void *q;
    long long q_stride;
    const float *sinks;
    long long sinks_stride;
    float *out;
    long long out_stride;
    // FP8 cache (codes [row][448], sexp [row][8], tail f16 [row][64])
    const uint8_t *codes;
    const int8_t *sexp;
    const uint16_t *tail;
    // fp32 rows of the reference launchers: rows < f32_n_raw come from f32_raw,
    // the rest from f32_comp, gated by f32_allowed (may be null)
    const float *f32_raw;
    const float *f32_comp;
    const int32_t *f32_allowed;
    int f32_n_raw;
    // logical row -> physical cache row
    const long long *row_base;       // per problem, or null -> p * row_base_stride
    long long row_base_stride;
    const int32_t *row_idx;          // per problem position lists, or null
    long long row_idx_stride;
    const int32_t *page_table;       // per problem page lists, or null
    int page_table_stride;
    int page_shift;
    // schedule
    int n_prob;
    int chunk;
    int s_max;
    float kq_log2;                   // log2(e) / sqrt(head_dim)
    long long total;
    long long start[kMaxProb + 1];
    // workspace
    float *ws_o;                     // [slot][64][512]
    float *ws_ml;                    // [slot][2][64]
    int *ws_prob;                    // [slot]
};

// bytes [0,1] (kHi = false) or [2,3] (kHi = true) of w, times scale, to f16
template <bool kHi>
__device__ inline half2_t cvt_fp8x2(uint32_t w, float scale) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, scale, kHi);
}

__device__ inline float pow2f(int e) {
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

__device__ inline half8_t make_half8(half2_t a, half2_t b, half2_t c, half2_t d) {
    return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ inline half8_t f32x8_to_half8(float4_t a, float4_t b) {
    return half8_t{(half_t)a[0], (half_t)a[1], (half_t)a[2], (half_t)a[3],
                   (half_t)b[0], (half_t)b[1], (half_t)b[2], (half_t)b[3]};
}

__device__ inline long long phys_row(const DecodeArgs &A, int p, long long r) {
    long long pos = A.row_idx ? (long long)A.row_idx[(long long)p * A.row_idx_stride + r] : r;
    if (A.page_table) {
        const long long page = A.page_table[(long long)p * A.page_table_stride + (pos >> A.page_shift)];
        return (page << A.page_shift) | (pos & ((1LL << A.page_shift) - 1));
    }
    return (A.row_base ? A.row_base[p] : (long long)p * A.row_base_stride) + pos;
}

// Raw registers of one half-tile (16 rows) for one lane: its row's 16-dim
// slice of each of the 7 code blocks, the matching 16 tail dims, and the
// row's 8 scale exponents.
struct Fp8Frag {
    uint4_t c[7];
    uint4_t t0, t1;
    uint2_t e;
};

__device__ inline void load_fp8_frag(const DecodeArgs &A, long long phys, int q, bool valid,
                                     Fp8Frag &f) {
    if (valid) {
        const uint4_t *cp = reinterpret_cast<const uint4_t *>(A.codes + phys * kNope + 16 * q);
#pragma unroll
        for (int b = 0; b < 7; ++b) f.c[b] = __builtin_nontemporal_load(cp + 4 * b);
        const uint4_t *tp = reinterpret_cast<const uint4_t *>(A.tail + phys * kRot + 16 * q);
        f.t0 = __builtin_nontemporal_load(tp);
        f.t1 = __builtin_nontemporal_load(tp + 1);
        f.e = *reinterpret_cast<const uint2_t *>(A.sexp + phys * 8);
    } else {
#pragma unroll
        for (int b = 0; b < 7; ++b) f.c[b] = uint4_t{0, 0, 0, 0};
        f.t0 = f.t1 = uint4_t{0, 0, 0, 0};
        f.e = uint2_t{0, 0};
    }
}

// Dequantized A fragments for block b (dims 64b+16q+[0,8) and +[8,16)).
__device__ inline void dequant_fp8(const Fp8Frag &f, int b, half8_t &a0, half8_t &a1) {
    if (b < 7) {
        const uint32_t ew = b < 4 ? f.e[0] : f.e[1];
        const int e = (int)(int8_t)((ew >> (8 * (b & 3))) & 0xFF);
        const float s = pow2f(e);
        const uint4_t c = f.c[b];
        a0 = make_half8(cvt_fp8x2<false>(c[0], s), cvt_fp8x2<true>(c[0], s),
                        cvt_fp8x2<false>(c[1], s), cvt_fp8x2<true>(c[1], s));
        a1 = make_half8(cvt_fp8x2<false>(c[2], s), cvt_fp8x2<true>(c[2], s),
                        cvt_fp8x2<false>(c[3], s), cvt_fp8x2<true>(c[3], s));
    } else {
        a0 = __builtin_bit_cast(half8_t, f.t0);
        a1 = __builtin_bit_cast(half8_t, f.t1);
    }
}

// fp32 rows (reference launchers): the lane's 16-dim slice of block b,
// f16-rounded exactly like f16_round (cuda/flash_attn.cu:113-115).
__device__ inline void load_f32_block(const float *row, int b, int q, bool valid,
                                      half8_t &a0, half8_t &a1) {
    if (!valid) {
        a0 = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        a1 = a0;
        return;
    }
    const float4_t *p = reinterpret_cast<const float4_t *>(row + 64 * b + 16 * q);
    a0 = f32x8_to_half8(p[0], p[1]);
    a1 = f32x8_to_half8(p[2], p[3]);
}

// Q^T B fragments of one problem: k-step 2b+s covers dims 64b+16q+8s+[0,8).
template <bool kQf32>
__device__ inline void load_q(const DecodeArgs &A, int p, int head, int q, half8_t *qh,
                              half8_t *ql) {
    if (kQf32) {
        const float *src = static_cast<const float *>(A.q) + (long long)p * A.q_stride +
                           (long long)head * kD + 16 * q;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const float4_t x0 = *reinterpret_cast<const float4_t *>(src + 64 * b + 8 * s);
                const float4_t x1 = *reinterpret_cast<const float4_t *>(src + 64 * b + 8 * s + 4);
                half8_t hi, lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    hi[i] = (half_t)x0[i];
                    lo[i] = (half_t)(x0[i] - (float)hi[i]);
                    hi[4 + i] = (half_t)x1[i];
                    lo[4 + i] = (half_t)(x1[i] - (float)hi[4 + i]);
                }
                qh[2 * b + s] = hi;
                ql[2 * b + s] = lo;
            }
        }
    } else {
        const uint16_t *src = static_cast<const uint16_t *>(A.q) + (long long)p * A.q_stride +
                              (long long)head * kD + 16 * q;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint4_t v = *reinterpret_cast<const uint4_t *>(src + 64 * b + 8 * s);
                half8_t h;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    h[2 * i] = (half_t)bf16_to_f32((uint16_t)(v[i] & 0xFFFF));
                    h[2 * i + 1] = (half_t)bf16_to_f32((uint16_t)(v[i] >> 16));
                }
                qh[2 * b + s] = h;
            }
        }
    }
}

// LDS position of row r (0..31) of a tile inside a V^T line.
__device__ inline int vt_pos(int r) {
    const int t = r >> 4, i = r & 15;
    return 8 * (i >> 2) + 4 * t + (i & 3);
}

// Copies the problem prefix table from the kernel arguments into LDS. The
// table is read with constant indices only: a dynamically indexed array inside
// a by-value kernel argument would be copied to scratch.
__device__ inline void stage_start(const DecodeArgs &A, long long *s_start) {
    (void)A;
    // DecodeArgs is the only kernel argument, so it sits at offset 0 of the
    // kernarg segment and the table can be read through a plain pointer.
    const long long *tab = reinterpret_cast<const long long *>(
        (const char *)__builtin_amdgcn_kernarg_segment_ptr() +
        offsetof(DecodeArgs, start));
    for (int i = threadIdx.x; i <= kMaxProb; i += blockDim.x) s_start[i] = tab[i];
    __syncthreads();
}

template <bool kFp8, bool kQf32>
__global__ __launch_bounds__(256) void decode_partial_kernel(const DecodeArgs A) {
    __shared__ half_t vt[kD * kVtStride];
    __shared__ long long s_start[kMaxProb + 1];
    stage_start(A, s_start);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15;          // row (A/K loads) or head / dim column (outputs)
    const int q = lane >> 4;          // k-group
    const int head = wave * 16 + j;   // head owned by this lane in S^T / Q layout

    long long g0 = (long long)blockIdx.x * A.chunk;
    const long long g1 = min(g0 + (long long)A.chunk, A.total);
    int p = 0;
    int slot_s = 0;
    const int wg = blockIdx.x;

    while (g0 < g1) {
        while (s_start[p + 1] <= g0) ++p;
        const long long seg_end = min(g1, s_start[p + 1]);
        const long long r0 = g0 - s_start[p];
        const long long r1 = seg_end - s_start[p];

        half8_t qh[16], ql[kQf32 ? 16 : 1];
        load_q<kQf32>(A, p, head, q, qh, ql);

        float m_run = -INFINITY;
        float l_run = 0.0f;
        float4_t o[32];
#pragma unroll
        for (int n = 0; n < 32; ++n) o[n] = float4_t{0, 0, 0, 0};

        for (long long rb = r0; rb < r1; rb += kTile) {
            // ---- issue this tile's loads -------------------------------------
            Fp8Frag fr[2];
            const float *frow[2] = {nullptr, nullptr};
            bool lvalid[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const long long r = rb + 16 * t + j;
                lvalid[t] = r < r1;
                if (kFp8) {
                    const long long ph = lvalid[t] ? phys_row(A, p, r) : 0;
                    load_fp8_frag(A, ph, q, lvalid[t], fr[t]);
                } else if (lvalid[t]) {
                    if (r < A.f32_n_raw) {
                        frow[t] = A.f32_raw + r * kD;
                    } else {
                        const long long rc = r - A.f32_n_raw;
                        if (A.f32_allowed && A.f32_allowed[rc] == 0) lvalid[t] = false;
                        frow[t] = A.f32_comp + rc * kD;
                    }
                }
            }

            __syncthreads();   // previous tile's P.V reads of vt are done

            // ---- S^T = K . Q^T, and this wave's quarter of V^T -------------------
            float4_t acc[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                acc[t] = float4_t{0, 0, 0, 0};
                const int prow = vt_pos(16 * t + j);
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    half8_t a0, a1;
                    if (kFp8) dequant_fp8(fr[t], b, a0, a1);
                    else load_f32_block(frow[t], b, q, lvalid[t], a0, a1);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[2 * b], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[2 * b + 1], acc[t], 0, 0, 0);
                    if (kQf32) {
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[2 * b], acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[2 * b + 1], acc[t], 0, 0, 0);
                    }
                    if ((b >> 1) == wave) {
                        const int d0 = 64 * b + 16 * q;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            vt[(d0 + i) * kVtStride + prow] = a0[i];
                            vt[(d0 + 8 + i) * kVtStride + prow] = a1[i];
                        }
                    }
                }
            }

            // ---- online softmax (exp2 domain) ------------------------------------
            float s[2][4];
            float tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const long long row = rb + 16 * t + 4 * q + r;
                    bool ok = row < r1;
                    if (!kFp8 && ok && row >= A.f32_n_raw && A.f32_allowed)
                        ok = A.f32_allowed[row - A.f32_n_raw] != 0;
                    s[t][r] = ok ? acc[t][r] * A.kq_log2 : -INFINITY;
                    tmax = fmaxf(tmax, s[t][r]);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m_run, tmax);
            const bool none = m_new == -INFINITY;
            const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            half8_t pf;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = none ? 0.0f : __builtin_amdgcn_exp2f(s[t][r] - m_new);
                    psum += pv;
                    pf[4 * t + r] = (half_t)pv;
                }
            }
            l_run = l_run * alpha + psum;
            m_run = m_new;
            if (__any(alpha != 1.0f)) {
                // O rows are heads 16w+4q+r; their alpha sits in lanes 4q+r
                float ar[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * q + r);
#pragma unroll
                for (int n = 0; n < 32; ++n)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[n][r] *= ar[r];
            }

            __syncthreads();   // V^T tile complete

            // ---- O += P . V -----------------------------------------------------
#pragma unroll
            for (int n = 0; n < 32; ++n) {
                const half8_t vb =
                    *reinterpret_cast<const half8_t *>(&vt[(16 * n + j) * kVtStride + 8 * q]);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf, vb, o[n], 0, 0, 0);
            }
        }

        // ---- emit this segment's partial ------------------------------------------
        l_run += __shfl_xor(l_run, 16);
        l_run += __shfl_xor(l_run, 32);
        const long long slot = (long long)wg * A.s_max + slot_s;
        float *wo = A.ws_o + slot * (kH * kD) + (wave * 16 + 4 * q) * kD + j;
        // keep the 128 store addresses from being hoisted out of the tile loop
        asm volatile("" : "+v"(wo));
#pragma unroll
        for (int n = 0; n < 32; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) wo[r * kD + 16 * n] = o[n][r];
        if (q == 0) {
            A.ws_ml[slot * 2 * kH + head] = m_run;
            A.ws_ml[slot * 2 * kH + kH + head] = l_run;
        }
        if (threadIdx.x == 0) A.ws_prob[slot] = p;
        ++slot_s;
        g0 = seg_end;
    }
    if (threadIdx.x == 0)
        for (int s2 = slot_s; s2 < A.s_max; ++s2) A.ws_prob[(long long)wg * A.s_max + s2] = -1;
}

// One block per (problem, head): combine the partials with the sink.
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeArgs A) {
    __shared__ long long s_start[kMaxProb + 1];
    stage_start(A, s_start);
    if (threadIdx.x >= 128) return;
    const int p = blockIdx.x;
    const int h = blockIdx.y;
    const int d = threadIdx.x * 4;
    const float sink = A.sinks[(long long)p * A.sinks_stride + h] * kLog2e;
    float mx = sink;
    const long long b0 = s_start[p], b1 = s_start[p + 1];
    long long w0 = 0, w1 = -1;
    if (b1 > b0) {
        w0 = b0 / A.chunk;
        w1 = (b1 - 1) / A.chunk;
    }
    for (long long w = w0; w <= w1; ++w)
        for (int s = 0; s < A.s_max; ++s) {
            const long long slot = w * A.s_max + s;
            if (A.ws_prob[slot] == p) mx = fmaxf(mx, A.ws_ml[slot * 2 * kH + h]);
        }
    float denom = __builtin_amdgcn_exp2f(sink - mx);
    float4_t acc = float4_t{0, 0, 0, 0};
    for (long long w = w0; w <= w1; ++w)
        for (int s = 0; s < A.s_max; ++s) {
            const long long slot = w * A.s_max + s;
            if (A.ws_prob[slot] != p) continue;
            const float m = A.ws_ml[slot * 2 * kH + h];
            if (m == -INFINITY) continue;
            const float sc = __builtin_amdgcn_exp2f(m - mx);
            denom += A.ws_ml[slot * 2 * kH + kH + h] * sc;
            const float4_t v =
                *reinterpret_cast<const float4_t *>(A.ws_o + slot * (kH * kD) + h * kD + d);
            acc += v * sc;
        }
    const float inv = 1.0f / denom;
    *reinterpret_cast<float4_t *>(A.out + (long long)p * A.out_stride + h * kD + d) = acc * inv;
}

// ---- host-side planning -----------------------------------------------------------

int g_num_cus = 0;

int num_cus() {
    if (g_num_cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
            return 256;
        g_num_cus = prop.multiProcessorCount;
    }
    return g_num_cus;
}

struct Plan {
    int n_wg = 0;
    int chunk = 0;
    int s_max = 0;
    size_t ws_bytes = 0;
};

size_t slot_bytes() { return (size_t)kH * kD * 4 + 2 * kH * 4 + 4; }

// Chunk the concatenated rows so that ~2 workgroups run per CU, each chunk a
// whole number of tiles; s_max bounds the problems one chunk can touch.
Plan make_plan(const long long *start, int n_prob, int wg_per_cu) {
    Plan pl;
    const long long total = start[n_prob];
    const long long target = (long long)num_cus() * wg_per_cu;
    long long chunk = total > 0 ? (total + target - 1) / target : kTile;
    chunk = ((chunk + kTile - 1) / kTile) * kTile;
    if (chunk < kTile) chunk = kTile;
    pl.chunk = (int)chunk;
    pl.n_wg = total > 0 ? (int)((total + chunk - 1) / chunk) : 0;
    int smax = 1;
    for (int w = 0; w < pl.n_wg; ++w) {
        const long long a = (long long)w * chunk, b = std::min(a + chunk, total);
        int cnt = 0;
        for (int p = 0; p < n_prob; ++p)
            if (start[p + 1] > a && start[p] < b) ++cnt;
        smax = std::max(smax, cnt);
    }
    pl.s_max = smax;
    const size_t slots = (size_t)std::max(pl.n_wg, 1) * smax;
    pl.ws_bytes = slots * ((size_t)kH * kD * 4 + 2 * kH * 4) + slots * 4 + 256 * 3;
    return pl;
}

void carve(DecodeArgs &A, void *ws, const Plan &pl) {
    const size_t slots = (size_t)std::max(pl.n_wg, 1) * pl.s_max;
    char *c = static_cast<char *>(ws);
    auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
    A.ws_o = reinterpret_cast<float *>(c);
    c += align(slots * (size_t)kH * kD * 4);
    A.ws_ml = reinterpret_cast<float *>(c);
    c += align(slots * 2 * kH * 4);
    A.ws_prob = reinterpret_cast<int *>(c);
}

template <bool kFp8, bool kQf32>
int launch(DecodeArgs &A, const Plan &pl, hipStream_t st, int phases = 3) {
    A.chunk = pl.chunk;
    A.s_max = pl.s_max;
    A.kq_log2 = kLog2e / sqrtf((float)kD);
    if ((phases & 1) && pl.n_wg > 0) {
        hipLaunchKernelGGL((decode_partial_kernel<kFp8, kQf32>), dim3(pl.n_wg), dim3(256), 0, st, A);
        const int e = hip_status(hipGetLastError());
        if (e) return e;
    }
    if (phases & 2)
        hipLaunchKernelGGL(decode_merge_kernel, dim3(A.n_prob, kH), dim3(256), 0, st, A);
    return hip_status(hipGetLastError());
}

}  // namespace

extern "C" int ds4hip_flash_attn_decode_fp8_workspace_size(const long long *n_rows_per_prob,
                                                           int n_prob, size_t *bytes) {
    if (!bytes || n_prob <= 0 || n_prob > kMaxProb || !n_rows_per_prob) return kEINVAL;
    long long start[kMaxProb + 1];
    start[0] = 0;
    for (int p = 0; p < n_prob; ++p) {
        if (n_rows_per_prob[p] < 0) return kEINVAL;
        start[p + 1] = start[p] + n_rows_per_prob[p];
    }
    *bytes = make_plan(start, n_prob, 2).ws_bytes;
    return 0;
}

extern "C" int ds4hip_flash_attn_decode_fp8(
        const void *q, int q_is_f32, long long q_stride, const float *sinks,
        long long sinks_stride, float *out, long long out_stride, const uint8_t *codes,
        const int8_t *sexp, const uint16_t *tail, const long long *n_rows_per_prob,
        int n_prob, const long long *row_base, long long row_base_stride,
        const int32_t *row_idx, long long row_idx_stride, const int32_t *page_table,
        int page_table_stride, int page_rows, int n_head, int head_dim, int n_rot,
        void *workspace, size_t workspace_bytes, int phases, void *stream) {
    if (phases < 1 || phases > 3 || n_head != kH || head_dim != kD || n_rot != kRot || n_prob <= 0 || n_prob > kMaxProb ||
        !n_rows_per_prob || !q || !sinks || !out || !codes || !sexp || !tail || !workspace)
        return ds4hip_set_last_error(kEINVAL);
    int page_shift = 0;
    if (page_table) {
        if (page_rows <= 0 || (page_rows & (page_rows - 1))) return ds4hip_set_last_error(kEINVAL);
        while ((1 << page_shift) < page_rows) ++page_shift;
    }
    DecodeArgs A = {};
    A.start[0] = 0;
    for (int p = 0; p < n_prob; ++p) {
        if (n_rows_per_prob[p] < 0) return ds4hip_set_last_error(kEINVAL);
        A.start[p + 1] = A.start[p] + n_rows_per_prob[p];
    }
    const Plan pl = make_plan(A.start, n_prob, 2);
    if (workspace_bytes < pl.ws_bytes) return ds4hip_set_last_error(kEINVAL);
    A.q = q;
    A.q_stride = q_stride;
    A.sinks = sinks;
    A.sinks_stride = sinks_stride;
    A.out = out;
    A.out_stride = out_stride;
    A.codes = codes;
    A.sexp = sexp;
    A.tail = tail;
    A.row_base = row_base;
    A.row_base_stride = row_base_stride;
    A.row_idx = row_idx;
    A.row_idx_stride = row_idx_stride;
    A.page_table = page_table;
    A.page_table_stride = page_table_stride;
    A.page_shift = page_shift;
    A.n_prob = n_prob;
    A.total = A.start[n_prob];
    carve(A, workspace, pl);
    const hipStream_t st = (hipStream_t)stream;
    const int rc = q_is_f32 ? launch<true, true>(A, pl, st, phases)
                            : launch<true, false>(A, pl, st, phases);
    return ds4hip_set_last_error(rc);
}

// fp32 launchers of the reference (cuda/flash_attn.cuh:73,142). The workspace
// for the split partials is stream-ordered (hipMallocAsync/hipFreeAsync), as
// the reference's non-prealloc launchers do for their scratch.
namespace {
int run_f32(const float *Q, const float *raw, int n_raw, const float *comp, int n_comp,
            const int32_t *allowed, const float *sinks, float *out, hipStream_t st) {
    DecodeArgs A = {};
    A.start[0] = 0;
    A.start[1] = (long long)n_raw + n_comp;
    const Plan pl = make_plan(A.start, 1, 2);
    void *ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, pl.ws_bytes, st);
    if (e != hipSuccess) return hip_status(e);
    A.q = Q;
    A.q_stride = 0;
    A.sinks = sinks;
    A.out = out;
    A.f32_raw = raw;
    A.f32_comp = comp;
    A.f32_allowed = allowed;
    A.f32_n_raw = n_raw;
    A.n_prob = 1;
    A.total = A.start[1];
    carve(A, ws, pl);
    int rc = launch<false, true>(A, pl, st);
    e = hipFreeAsync(ws, st);
    if (!rc) rc = hip_status(e);
    return rc;
}
}  // namespace

extern "C" int ds4hip_flash_attn_decode_raw_f32(const float *Q, const float *K, const float *V,
                                                const float *sinks, float *out, int n_head,
                                                int n_kv, int head_dim, void *stream) {
    // cuda/flash_attn.cu:259-269 drops the launch on a bad shape; the 128-row
    // cap of the reference kernel is lifted. K and V must be the same buffer
    // (MLA layout, cuda/flash_attn.cu:30-33).
    if (head_dim != kD || n_head != kH || n_kv < 0 || K != V || !Q || !sinks || !out ||
        (n_kv > 0 && !K))
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(
        run_f32(Q, K, n_kv, nullptr, 0, nullptr, sinks, out, (hipStream_t)stream));
}

extern "C" int ds4hip_flash_attn_decode_mixed_f32(const float *Q, const float *raw_kv,
                                                  const float *comp_kv,
                                                  const int32_t *comp_allowed,
                                                  const float *sinks, float *out, int n_head,
                                                  int n_raw, int n_comp, int head_dim,
                                                  void *stream) {
    if (head_dim != kD || n_head != kH || n_raw < 0 || n_comp < 0 || !Q || !sinks || !out ||
        (n_raw > 0 && !raw_kv) || (n_comp > 0 && !comp_kv))
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(run_f32(Q, raw_kv, n_raw, comp_kv, n_comp, comp_allowed, sinks,
                                         out, (hipStream_t)stream));
}
