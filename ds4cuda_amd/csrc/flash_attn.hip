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
// FP8 kernel, per 32-row tile:
//   * the tile's raw bytes (codes, f16 tail, exponents: 584 B/row) are copied
//     HBM -> LDS by global_load_lds_dwordx4, three tiles ahead of use (4-stage
//     ring), so HBM latency is covered without holding registers;
//   * S^T[32 rows x 16 heads] = K[32 x 512] . Q^T per wave with
//     v_mfma_f32_16x16x32_f16: A = K fragments read from the stage (lane = row,
//     16 dims = one 16-byte chunk) and dequantized with
//     v_cvt_scalef32_pk_f16_fp8; B = Q^T held in registers for the segment;
//   * online softmax in the exp2 domain; P stays in registers: the S^T output
//     layout (lane = head, 4+4 rows) is already the A layout of P . V;
//   * O[16 heads x 512] += P[16 x 32] . V[32 x 512] with B = V^T fragments
//     read from LDS as 16-byte vectors. Wave w writes V^T for dims
//     [128w, 128w+128) from the registers it already holds.
// Rows inside a V^T line are stored in the order the P fragment uses
// (row 4a+c of half-tile t at position 8a+4t+c), so each B fragment is one
// contiguous 16-byte LDS read.

#include "ds4hip_common.h"
#include "q_prep.h"
#include "rope.h"
#include "../../include/ds4hip.h"

#include <algorithm>
#include <mutex>
#include <cstddef>
#include <type_traits>
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
constexpr int kMinChunk = 2 * kTile;       // the register-load kernels run tiles in pairs
constexpr int kMinChunkFlat = kTile;       // the flat-stage kernel: one tile is a whole chunk
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyLog2 = 8.0f;   // decode softmax: reference point slack (log2 units)
constexpr int kFp8WgPerCu = 1;   // the FP8 kernel's LDS ring allows one workgroup per CU

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
    const float *f32_v_raw;          // V rows of the raw launcher when V != K, else null
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
    // gathered rows (row_idx or page_table): physical row of every logical
    // row, resolved by phys_kernel before the partial kernel
    long long *phys;
    // rows addressable from codes / sexp / tail: a row outside [0, n_cache_rows)
    // is never read; its problem is marked bad and its output set to NaN
    long long n_cache_rows;
    // schedule
    int n_prob;
    int chunk;
    int s_max;
    float kq_log2;                   // log2(e) / sqrt(head_dim)
    long long total;
    long long start[kMaxProb + 1];   // row offset of each problem in the chunked row space
    long long count[kMaxProb];       // rows of each problem (the space may pad between problems)
    // workspace
    float *ws_o;                     // [slot][64][512]
    float *ws_ml;                    // [slot][2][64]
    int *ws_prob;                    // [slot]
    // merge output form (DS4HIP_DECODE_OUT_*): 0 fp32 rows, 1 rotated Q8_0,
    // 2 rotated fp32; rotation position rope_pos_dev[p] or rope_pos
    int out_form;
    int rope_pos;
    const int *rope_pos_dev;
    RopeParams rope;
    int8_t *q8_out;
    float *q8_scale;
};

// The rotation coefficients of dims dim0 .. dim0 + 3 of problem p for
// merge_store (rotated forms and tail dims only), computed at the merge's
// start, under its loads.
struct MergeRope {
    float c[2], s[2];
};
__device__ inline MergeRope merge_rope(const DecodeArgs &A, int p, int dim0) {
    MergeRope r = {{1.0f, 1.0f}, {0.0f, 0.0f}};
    constexpr int kNope = kD - kRot;
    if (A.out_form && dim0 >= kNope) {
        const int pos = A.rope_pos_dev ? A.rope_pos_dev[p] : A.rope_pos;
        rope_cs((dim0 - kNope) / 2, pos, A.rope, r.c[0], r.s[0]);
        rope_cs((dim0 + 2 - kNope) / 2, pos, A.rope, r.c[1], r.s[1]);
    }
    // here, not sunk next to their use at the end
    asm volatile("" : "+v"(r.c[0]), "+v"(r.c[1]), "+v"(r.s[0]), "+v"(r.s[1]));
    return r;
}

// The merge's result for dims dim0 .. dim0 + 3 of head h of problem p: into
// out, or rotated by the inverse tail RoPE (rope_tail_kernel's arithmetic)
// into out (out_form 2) or quantized as Q8_0 with the arithmetic of
// rope_q8_kernel (out_form 1). The 8 lanes of a 32-dim block are consecutive
// lanes of one wave, all present.
__device__ inline void merge_store(const DecodeArgs &A, int p, int h, int dim0, float4_t res, const MergeRope &R) {
    const long long o = (long long)p * (kH * kD) + h * kD + dim0;
    float4_t *dst = reinterpret_cast<float4_t *>(A.out + (long long)p * A.out_stride + h * kD + dim0);
    if (!A.out_form) {
        *dst = res;
        return;
    }
    float v[4] = {res[0], res[1], res[2], res[3]};
    constexpr int kNope = kD - kRot;
    if (dim0 >= kNope) {
        rope_apply(v[0], v[1], R.c[0], R.s[0], v[0], v[1]);
        rope_apply(v[2], v[3], R.c[1], R.s[1], v[2], v[3]);
    }
    if (A.out_form == 2) {
        *dst = float4_t{v[0], v[1], v[2], v[3]};
        return;
    }
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int off = 4; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
    const float dq = a / 127.0f;
    const float id = dq != 0.0f ? 1.0f / dq : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int q = (int)__builtin_rintf(v[i] * id);
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        packed |= (uint32_t)(q & 0xFF) << (8 * i);
    }
    *reinterpret_cast<uint32_t *>(A.q8_out + o) = packed;
    if ((dim0 & 31) == 0) A.q8_scale[o / 32] = dq;
}

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

// (-1 for a position past the problem's page list: no table entry is read
// outside [0, page_table_stride))
__device__ inline long long phys_row(const DecodeArgs &A, int p, long long r) {
    long long pos = A.row_idx ? (long long)A.row_idx[(long long)p * A.row_idx_stride + r] : r;
    if (A.page_table) {
        if (pos < 0 || (pos >> A.page_shift) >= A.page_table_stride) return -1;
        const long long page = A.page_table[(long long)p * A.page_table_stride + (pos >> A.page_shift)];
        return (page << A.page_shift) | (pos & ((1LL << A.page_shift) - 1));
    }
    return (A.row_base ? A.row_base[p] : (long long)p * A.row_base_stride) + pos;
}

// Out-of-range rows. phys_kernel stores kBadRow for a gathered row outside
// the cache. A partial kernel scans its segment's rows once before the tile
// loop (scan_segment_rows) and marks its slot with kBadSlot in ws_prob; the
// merge then writes NaN for every head of that problem. Inside the tile loop
// a bad row only becomes row 0 (unmark_row / clamp_row: two or three VALU
// instructions, no carried flag, no branch), so nothing outside the cache is
// ever read.
constexpr long long kBadRow = (long long)(1ULL << 63);
constexpr int kBadSlot = 1 << 30;
__device__ inline long long unmark_row(long long r) { return r & ~(r >> 63); }
__device__ inline long long clamp_row(long long r, long long n_rows) {
    return min(max(r, 0LL), n_rows - 1);
}
// Row bases of the problems into LDS (so the tile loops issue no row loads).
// A direct-row problem (no row_idx, no pages) whose rows [base, base + count)
// leave the cache reads from base 0 instead and is marked bad.
__device__ inline void stage_rowbase(const DecodeArgs &A, long long *s_rowbase, int *s_badp) {
    const bool direct = !A.row_idx && !A.page_table;
    for (int i = threadIdx.x; i < A.n_prob; i += blockDim.x) {
        const long long rb = A.row_base ? A.row_base[i] : (long long)i * A.row_base_stride;
        const bool bad = direct && (rb < 0 || rb + A.count[i] > A.n_cache_rows);
        s_rowbase[i] = bad ? 0 : rb;
        s_badp[i] = bad ? 1 : 0;
    }
}
// Called by every thread at the start of a segment of problem p (logical
// rows [r0, r1), global rows [g0, g1)): sets s_bad[slot_s & 1] when a
// gathered row of the segment lies outside the cache. use_phys: the rows come
// from the phys array this launch's phys pass wrote; otherwise from row_idx
// (the array the workspace reserves for phys then holds nothing of this launch).
__device__ inline void scan_segment_rows(const DecodeArgs &A, bool use_phys, int p, long long g0, long long g1,
                                         long long r0, long long r1, long long seg_base, int slot_s, int *s_bad) {
    bool bad = false;
    if (use_phys) {
        for (long long g = g0 + threadIdx.x; g < g1; g += blockDim.x) bad |= A.phys[g] < 0;
    } else if (A.row_idx) {
        for (long long r = r0 + threadIdx.x; r < r1; r += blockDim.x) {
            const long long v = seg_base + A.row_idx[(long long)p * A.row_idx_stride + r];
            bad |= v < 0 || v >= A.n_cache_rows;
        }
    }
    if (bad) atomicOr(&s_bad[slot_s & 1], 1);
}

// Slot mark of a finished segment: the problem id, plus kBadSlot when a lane
// of the workgroup met a bad row (s_bad, one word per segment parity, so the
// next segment's marks cannot mix in) or the problem's rows were refused.
// Called by every thread; ends with a barrier.
__device__ inline void mark_slot(const DecodeArgs &A, long long slot, int p, int slot_s, int *s_bad,
                                 const int *s_badp) {
    __syncthreads();
    if (threadIdx.x == 0) {
        A.ws_prob[slot] = p | ((s_bad[slot_s & 1] | s_badp[p]) ? kBadSlot : 0);
        s_bad[slot_s & 1] = 0;
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

// max / sum over lanes l, l^16, l^32, l^48 with VALU lane swaps (no LDS).
__device__ inline float xmax_16_32(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float xsum_16_32(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Barrier for this kernel's LDS pipeline: waits for this wave's LDS
// operations, then s_barrier. Unlike __syncthreads() it does not wait for
// outstanding global->LDS copies (vmcnt), which keeps the prefetch in flight.
__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct SegState {
    float m_run;
    float l_run;
    float4_t o[32];
};

// Online softmax of one 32-row tile (S^T accumulators acc[t][r] = row
// 16t+4q+r, head j) and the P fragment for P . V. row_ok(t, r) says whether
// that row takes part.
template <typename RowOk>
__device__ inline half8_t softmax_tile(const float4_t *acc, float kq_log2, int q, SegState &S,
                                       RowOk row_ok) {
    float s[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[t][r] = row_ok(t, r) ? acc[t][r] * kq_log2 : -INFINITY;
            tmax = fmaxf(tmax, s[t][r]);
        }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(S.m_run, tmax);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(S.m_run - m_new);
    half8_t pf;
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = none ? 0.0f : __builtin_amdgcn_exp2f(s[t][r] - m_new);
            psum += pv;
            pf[4 * t + r] = (half_t)pv;
        }
    S.l_run = S.l_run * alpha + psum;
    S.m_run = m_new;
    if (__any(alpha != 1.0f)) {
        // O rows are heads 16w+4q+r; their alpha sits in lanes 4q+r
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * q + r);
#pragma unroll
        for (int n = 0; n < 32; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) S.o[n][r] *= ar[r];
    }
    return pf;
}

__device__ inline void pv_tile(const half_t *vt, half8_t pf, int j, int q, SegState &S) {
#pragma unroll
    for (int n = 0; n < 32; ++n) {
        const half8_t vb = *reinterpret_cast<const half8_t *>(&vt[(16 * n + j) * kVtStride + 8 * q]);
        S.o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf, vb, S.o[n], 0, 0, 0);
    }
}

// Writes this wave's V^T slice (dims 64b+16q .. +15 of row `prow`).
__device__ inline void vt_write(half_t *vt, int b, int q, int prow, half8_t a0, half8_t a1) {
    const int d0 = 64 * b + 16 * q;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        vt[(d0 + i) * kVtStride + prow] = a0[i];
        vt[(d0 + 8 + i) * kVtStride + prow] = a1[i];
    }
}

__device__ inline void emit_partial(const DecodeArgs &A, long long slot, int wave, int j, int q,
                                    int head, int p, SegState &S) {
    float l = S.l_run;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    float *wo = A.ws_o + slot * (kH * kD) + (wave * 16 + 4 * q) * kD + j;
    // keep the 128 store addresses from being hoisted out of the tile loop
    asm volatile("" : "+v"(wo));
#pragma unroll
    for (int n = 0; n < 32; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) wo[r * kD + 16 * n] = S.o[n][r];
    if (q == 0) {
        A.ws_ml[slot * 2 * kH + head] = S.m_run;
        A.ws_ml[slot * 2 * kH + kH + head] = l;
    }
    if (threadIdx.x == 0) A.ws_prob[slot] = p;
}

__device__ inline void seg_init(SegState &S) {
    S.m_run = -INFINITY;
    S.l_run = 0.0f;
#pragma unroll
    for (int n = 0; n < 32; ++n) S.o[n] = float4_t{0, 0, 0, 0};
}

// ---- FP8 cache kernel ------------------------------------------------------------------
//
// Copy ring. Each 32-row tile is copied HBM -> LDS by global_load_lds three
// tiles ahead of use (4-stage ring). Copy instruction i < 18 moves 64-dim
// block i>>1 (blocks 0..6 = codes, 7..8 = the f16 tail) of the 16 rows of
// half-tile i&1: lane L fetches 16-byte chunk (L&3) ^ ((L>>4)&3)... of row
// L>>2, so every row contributes one whole 64-byte segment per instruction
// and the chunk order inside the LDS segment is XOR-swizzled by the row,
// which makes the fragment reads below bank-conflict free. Instruction 18
// copies the 32 rows' scale exponents; instruction 19 is a filler that
// keeps every wave at 5 copies per stage.
//
// Work split inside a workgroup (4 waves): wave w owns head dims
// [128w, 128w+128) — code blocks 2w, 2w+1 (wave 3: block 6 and the tail) —
// and heads [16w, 16w+16) for the softmax. Per tile:
//   1. partial scores over the wave's dims for all 64 heads,
//      S_w^T[32 rows x 64 heads] (v_mfma_f32_16x16x32_f16, A = the wave's own
//      dequantized K fragments, B = Q^T slice in registers);
//   2. reduce-scatter through LDS: wave w sums the four partials of its 16
//      heads, runs the online softmax and publishes P (f16) and the rescale
//      factors of its heads;
//   3. O_w[64 heads x 128 dims] += P . V_w with V_w the wave's own f16 slice,
//      kept row-major in LDS and read as MFMA B fragments with
//      ds_read_b64_tr_b16 (transposing 16-bit load).
// Every KV element is dequantized once and read from HBM once.

constexpr int kStages = 4;
constexpr int kStageBytes = 18 * 1024 + 256 + 256;
constexpr int kSexpOff = 18 * 1024;
constexpr int kPhysOff = kSexpOff + 256;         // 32 x int64 physical rows (gathered modes)
constexpr int kCopiesPerWave = 5;
constexpr int kVRowBytes = 288;                  // 128 dims f16 + 32 B pad (bank spread)
constexpr int kVTileBytes = kTile * kVRowBytes;  // per wave

__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// LDS byte offset of 16-byte chunk c (0..3) of row k (0..15) in copy region
// `region` (= 2*block + half) of a stage.
__device__ inline int stage_off(int region, int k, int c) {
    return region * 1024 + 64 * k + 16 * (c ^ ((k >> 1) & 3));
}

// Issues the 5 copies of this wave for one tile. ph_h0 / ph_h1: physical rows
// of tile rows lane>>2 and 16 + (lane>>2); ph_e: tile row lane>>1 (exponent
// copy). The wave-3 spare copy carries, when phys_src != null, the physical
// rows of the tile kStages ahead of this one (32 x int64 from phys_src,
// lanes 0..15) into the stage's phys slot; otherwise it repeats the exponent
// copy so every wave issues the same number of copies.
__device__ inline void issue_stage(const DecodeArgs &A, uint8_t *stage, long long ph_h0,
                                   long long ph_h1, long long ph_e, const long long *phys_src,
                                   int lane, int wave) {
    const int k = lane >> 2;
    const int c = (lane & 3) ^ ((k >> 1) & 3);
#pragma unroll
    for (int kk = 0; kk < kCopiesPerWave; ++kk) {
        const int i = wave * kCopiesPerWave + kk;
        if (i < 18) {
            const int blk = i >> 1;
            const long long row = (i & 1) ? ph_h1 : ph_h0;
            const uint8_t *g = blk < 7
                ? A.codes + row * kNope + blk * 64 + c * 16
                : reinterpret_cast<const uint8_t *>(A.tail) + row * (2 * kRot) + (blk - 7) * 64 + c * 16;
            __builtin_amdgcn_global_load_lds(g, stage + i * 1024, 16, 0, 0);
        } else if (i == 18 || !phys_src) {
            const uint8_t *g = reinterpret_cast<const uint8_t *>(A.sexp) + ph_e * 8 + (lane & 1) * 4;
            __builtin_amdgcn_global_load_lds(g, stage + kSexpOff, 4, 0, 0);
        } else if (lane < 16) {
            // 16 lanes x 16 bytes = the 32 int64 rows (one copy, partial exec)
            __builtin_amdgcn_global_load_lds(phys_src + 2 * lane, stage + kPhysOff, 16, 0, 0);
        }
    }
}

// Waits until at most `pending_stages` stages of this wave's copies are in flight.
__device__ inline void wait_copies(int pending_stages) {
    switch (pending_stages) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    }
}

// LDS accessors used inside the copy-ring loop. They are inline assembly so
// that the compiler does not make them wait for the outstanding global->LDS
// copies (it cannot tell the ring apart from the other LDS buffers and would
// insert vmcnt(0), draining the ring every tile). Reads return without
// waiting; lds_wait() completes them and ties the results to the wait.
template <typename T>
__device__ inline void lds_st128(uint32_t a, T v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}
// Eight 16-byte stores of MFMA results at a + off[i]. The compiler does not
// insert the wait states that a read of an MFMA destination register needs
// when the read is inside inline assembly, so the statement starts with them
// (16, more than the 16x16x32 f16 MFMA needs) and ends with two for the
// store-data hazard of a following write of those registers.
template <int O0, int O1, int O2, int O3, int O4, int O5, int O6, int O7>
__device__ inline void lds_st128x8_mfma(uint32_t a, const float4_t *v) {
    asm volatile(
        "s_nop 7\n\ts_nop 7\n\t"
        "ds_write_b128 %0, %1 offset:%9\n\tds_write_b128 %0, %2 offset:%10\n\t"
        "ds_write_b128 %0, %3 offset:%11\n\tds_write_b128 %0, %4 offset:%12\n\t"
        "ds_write_b128 %0, %5 offset:%13\n\tds_write_b128 %0, %6 offset:%14\n\t"
        "ds_write_b128 %0, %7 offset:%15\n\tds_write_b128 %0, %8 offset:%16\n\t"
        "s_nop 1"
        :: "v"(a), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]),
           "v"(v[7]), "n"(O0), "n"(O1), "n"(O2), "n"(O3), "n"(O4), "n"(O5), "n"(O6), "n"(O7)
        : "memory");
}
__device__ inline void lds_st32(uint32_t a, float v) {
    asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}
// Eight 16-byte LDS reads at a + off[i] completed by one lgkmcnt wait in the
// same statement (a separate wait would let the compiler copy a destination
// register before its load has landed).
template <int O0, int O1, int O2, int O3, int O4, int O5, int O6, int O7, typename T>
__device__ inline void lds_ld128x8(uint32_t a, T *v) {
    asm volatile(
        "ds_read_b128 %0, %8 offset:%9\n\tds_read_b128 %1, %8 offset:%10\n\t"
        "ds_read_b128 %2, %8 offset:%11\n\tds_read_b128 %3, %8 offset:%12\n\t"
        "ds_read_b128 %4, %8 offset:%13\n\tds_read_b128 %5, %8 offset:%14\n\t"
        "ds_read_b128 %6, %8 offset:%15\n\tds_read_b128 %7, %8 offset:%16\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7])
        : "v"(a), "n"(O0), "n"(O1), "n"(O2), "n"(O3), "n"(O4), "n"(O5), "n"(O6), "n"(O7));
}

// Four 16-byte reads at a + 64*i and four at b + 1024*i, one wait.
// Four 16-byte reads at a + 1024*i, one wait.
__device__ inline void lds_ld128x4(uint32_t a, half8_t *v) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
        : "v"(a));
}
__device__ inline void lds_ld_alpha_p(uint32_t a, uint32_t b, float4_t *ar, half8_t *pa) {
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:64\n\t"
        "ds_read_b128 %2, %8 offset:128\n\tds_read_b128 %3, %8 offset:192\n\t"
        "ds_read_b128 %4, %9\n\tds_read_b128 %5, %9 offset:1024\n\t"
        "ds_read_b128 %6, %9 offset:2048\n\tds_read_b128 %7, %9 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(ar[0]), "=&v"(ar[1]), "=&v"(ar[2]), "=&v"(ar[3]), "=&v"(pa[0]), "=&v"(pa[1]),
          "=&v"(pa[2]), "=&v"(pa[3])
        : "v"(a), "v"(b));
}

// The three physical rows a lane needs from a phys slot (rows a, 16 + a and b).
__device__ inline void lds_ld_phys3(uint32_t slot, int a, int b, long long &h0, long long &h1,
                                    long long &e) {
    uint2_t x, y, z;
    asm volatile("ds_read_b64 %0, %3\n\tds_read_b64 %1, %3 offset:128\n\tds_read_b64 %2, %4\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(x), "=&v"(y), "=&v"(z)
                 : "v"(slot + 8 * a), "v"(slot + 8 * b));
    h0 = (long long)(((unsigned long long)x[1] << 32) | x[0]);
    h1 = (long long)(((unsigned long long)y[1] << 32) | y[0]);
    e = (long long)(((unsigned long long)z[1] << 32) | z[0]);
}

// The wave's raw fragments of both half-tile rows at once (one LDS round
// trip): two 16-byte chunks (its two 64-dim blocks, 16 dims each) in
// c[h2][0..1] and the row's exponents in e[h2]; for wave 3, th[h2] is the
// second tail chunk (f16 chunk 2q+1), otherwise untouched. Issued from inline
// assembly because the compiler would otherwise make each read wait for all
// outstanding global->LDS copies; the trailing lgkmcnt wait makes the outputs
// valid when the statement completes.
__device__ inline void read_wave_frags(const uint8_t *st, int wave, int j, int q, uint4_t (*c)[2],
                                       uint2_t *e, uint4_t *th) {
    const uint32_t ae0 = lds_addr(st) + kSexpOff + j * 8;
    if (wave < 3) {
        const uint32_t a0 = lds_addr(st) + stage_off(2 * (2 * wave), j, q);
        const uint32_t a1 = lds_addr(st) + stage_off(2 * (2 * wave + 1), j, q);
        // half 1 is the next 1 KB region of each block
        asm volatile(
            "ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\tds_read_b64 %4, %8\n\t"
            "ds_read_b128 %2, %6 offset:1024\n\tds_read_b128 %3, %7 offset:1024\n\t"
            "ds_read_b64 %5, %8 offset:128\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(c[0][0]), "=&v"(c[0][1]), "=&v"(c[1][0]), "=&v"(c[1][1]), "=&v"(e[0]),
              "=&v"(e[1])
            : "v"(a0), "v"(a1), "v"(ae0));
    } else {
        const uint32_t a0 = lds_addr(st) + stage_off(2 * 6, j, q);
        const uint32_t a1 = lds_addr(st) + stage_off(2 * (7 + (q >> 1)), j, (2 * q) & 3);
        const uint32_t a2 = lds_addr(st) + stage_off(2 * (7 + (q >> 1)), j, (2 * q + 1) & 3);
        asm volatile(
            "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\tds_read_b128 %6, %10\n\t"
            "ds_read_b64 %4, %11\n\t"
            "ds_read_b128 %2, %8 offset:1024\n\tds_read_b128 %3, %9 offset:1024\n\t"
            "ds_read_b128 %7, %10 offset:1024\n\tds_read_b64 %5, %11 offset:128\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(c[0][0]), "=&v"(c[0][1]), "=&v"(c[1][0]), "=&v"(c[1][1]), "=&v"(e[0]),
              "=&v"(e[1]), "=&v"(th[0]), "=&v"(th[1])
            : "v"(a0), "v"(a1), "v"(a2), "v"(ae0));
    }
}


__device__ inline void dequant16(uint4_t c, float sc, half8_t &a0, half8_t &a1) {
    a0 = make_half8(cvt_fp8x2<false>(c[0], sc), cvt_fp8x2<true>(c[0], sc),
                    cvt_fp8x2<false>(c[1], sc), cvt_fp8x2<true>(c[1], sc));
    a1 = make_half8(cvt_fp8x2<false>(c[2], sc), cvt_fp8x2<true>(c[2], sc),
                    cvt_fp8x2<false>(c[3], sc), cvt_fp8x2<true>(c[3], sc));
}

__device__ inline float block_scale(uint2_t e, int b) {
    const uint32_t w = b < 4 ? e[0] : e[1];
    return pow2f((int)(int8_t)((w >> (8 * (b & 3))) & 0xFF));
}

// Q^T B fragments for the dim-split: hb = head block, ks = k-step over the
// wave's 128 dims; dims 64*(2w + (ks>>1)) + 16q + 8(ks&1) + [0,8).
template <bool kQf32>
__device__ inline void load_q_split(const DecodeArgs &A, int p, int wave, int j, int q,
                                    half8_t (*qh)[4], half8_t (*ql)[4]) {
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int d = 64 * (2 * wave + (ks >> 1)) + 16 * q + 8 * (ks & 1);
            const long long off = (long long)p * A.q_stride + (long long)(16 * hb + j) * kD + d;
            if (kQf32) {
                const float *src = static_cast<const float *>(A.q) + off;
                const float4_t x0 = *reinterpret_cast<const float4_t *>(src);
                const float4_t x1 = *reinterpret_cast<const float4_t *>(src + 4);
                half8_t hi, lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    hi[i] = (half_t)x0[i];
                    lo[i] = (half_t)(x0[i] - (float)hi[i]);
                    hi[4 + i] = (half_t)x1[i];
                    lo[4 + i] = (half_t)(x1[i] - (float)hi[4 + i]);
                }
                qh[hb][ks] = hi;
                ql[hb][ks] = lo;
            } else {
                const uint4_t v = *reinterpret_cast<const uint4_t *>(
                    static_cast<const uint16_t *>(A.q) + off);
                half8_t h;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    h[2 * i] = (half_t)bf16_to_f32((uint16_t)(v[i] & 0xFFFF));
                    h[2 * i + 1] = (half_t)bf16_to_f32((uint16_t)(v[i] >> 16));
                }
                qh[hb][ks] = h;
            }
        }
}

struct SplitState {
    float m_run;        // owner-side softmax state of head 16w + j
    float l_run;
    float4_t o[4][8];   // O_w[head block][dim block]: heads 16mb+4q+r, dims 128w+16nb+j
};

// O_w += P . V_w for one tile: B fragments (rows R(8q + 4h + s/4) =
// 16h + 4q + s/4, dims 16nb + 4(s&3)) come from the wave's V slice via
// transposing reads, all 16 behind one wait.
__device__ inline void pv_split(uint32_t vt_base, int j, int q, const half8_t *pa,
                                const half8_t *pl, float4_t (*o)[8]) {
            uint2_t tb[16];
            {
                const uint32_t ab = vt_base + (4 * q + (j >> 2)) * kVRowBytes + 8 * (j & 3);
                asm volatile(
                    "ds_read_b64_tr_b16 %0, %16\n\tds_read_b64_tr_b16 %1, %16 offset:4608\n\t"
                    "ds_read_b64_tr_b16 %2, %16 offset:32\n\tds_read_b64_tr_b16 %3, %16 offset:4640\n\t"
                    "ds_read_b64_tr_b16 %4, %16 offset:64\n\tds_read_b64_tr_b16 %5, %16 offset:4672\n\t"
                    "ds_read_b64_tr_b16 %6, %16 offset:96\n\tds_read_b64_tr_b16 %7, %16 offset:4704\n\t"
                    "ds_read_b64_tr_b16 %8, %16 offset:128\n\tds_read_b64_tr_b16 %9, %16 offset:4736\n\t"
                    "ds_read_b64_tr_b16 %10, %16 offset:160\n\tds_read_b64_tr_b16 %11, %16 offset:4768\n\t"
                    "ds_read_b64_tr_b16 %12, %16 offset:192\n\tds_read_b64_tr_b16 %13, %16 offset:4800\n\t"
                    "ds_read_b64_tr_b16 %14, %16 offset:224\n\tds_read_b64_tr_b16 %15, %16 offset:4832\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(tb[0]), "=&v"(tb[1]), "=&v"(tb[2]), "=&v"(tb[3]), "=&v"(tb[4]),
                      "=&v"(tb[5]), "=&v"(tb[6]), "=&v"(tb[7]), "=&v"(tb[8]), "=&v"(tb[9]),
                      "=&v"(tb[10]), "=&v"(tb[11]), "=&v"(tb[12]), "=&v"(tb[13]), "=&v"(tb[14]),
                      "=&v"(tb[15])
                    : "v"(ab));
            }
            static_assert(16 * kVRowBytes == 4608, "tr-read offsets assume 288-byte V rows");
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) {
                const half8_t vb = __builtin_bit_cast(
                    half8_t, uint4_t{tb[2 * nb][0], tb[2 * nb][1], tb[2 * nb + 1][0], tb[2 * nb + 1][1]});
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    o[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[mb], vb, o[mb][nb], 0, 0, 0);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    o[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[mb], vb, o[mb][nb], 0, 0, 0);
            }
}

template <bool kQf32>
__global__ __launch_bounds__(256) void decode_fp8_kernel(const DecodeArgs A) {
    static_assert(kStages == 4 && kCopiesPerWave == 5, "wait_copies encodes these counts");
    __shared__ __attribute__((aligned(16))) uint8_t stages[kStages][kStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t vtile[4][kVTileBytes];
    __shared__ __attribute__((aligned(16))) float4_t sx[4][4][2][64];   // [owner][writer][h2][lane]
    __shared__ __attribute__((aligned(16))) half8_t pbuf[2][4][64];     // [hi, lo][head block][lane]
    __shared__ __attribute__((aligned(16))) float alpha_s[kH];
    __shared__ long long s_start[kMaxProb + 1];
    __shared__ long long s_rowbase[kMaxProb];   // LDS, so the ring loop issues no row loads
    __shared__ int s_badp[kMaxProb], s_bad[2];
    stage_rowbase(A, s_rowbase, s_badp);
    if (threadIdx.x < 2) s_bad[threadIdx.x] = 0;
    stage_start(A, s_start);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
    const int j = lane & 15;
    const int q = lane >> 4;
    const uint32_t vt_base = lds_addr(vtile[wave]);

    long long g0 = (long long)blockIdx.x * A.chunk;
    const long long g1 = min(g0 + (long long)A.chunk, A.total);
    int p = 0;
    int slot_s = 0;

    while (g0 < g1) {
        while (s_start[p + 1] <= g0) ++p;
        const long long seg_end = min(g1, s_start[p + 1]);
        const long long r0 = g0 - s_start[p];
        const long long r1 = min(seg_end - s_start[p], A.count[p]);
        const int n_tiles = (int)((r1 - r0 + kTile - 1) / kTile);
        const long long seg_base = s_rowbase[p];
        const bool gather = A.phys != nullptr;
        const int k4 = lane >> 2;
        // Physical rows of tile t needed by this lane's copies (tile rows k4,
        // 16 + k4 and lane>>1); rows past the segment end repeat its last
        // row (finite filler, masked in the softmax). Direct addressing is
        // pure arithmetic; gathered rows come from the phys array (prologue)
        // or from the phys slot that rode in with an earlier tile.
        auto rows_direct = [&](int t, long long &h0, long long &h1, long long &e) {
            const long long rb2 = r0 + (long long)t * kTile;
            h0 = seg_base + min(rb2 + k4, r1 - 1);
            h1 = seg_base + min(rb2 + 16 + k4, r1 - 1);
            e = seg_base + min(rb2 + (lane >> 1), r1 - 1);
        };
        auto phys_src = [&](int t) -> const long long * {
            if (!gather) return nullptr;
            long long gb = g0 + (long long)t * kTile;
            return A.phys + (gb < A.total ? gb : A.total);   // the array has 32 rows of padding
        };

        half8_t qh[4][4], ql[kQf32 ? 4 : 1][4];
        load_q_split<kQf32>(A, p, wave, j, q, qh, ql);
        // rows of the next tile to issue (gathered: read ahead, see below)
        long long nh0 = 0, nh1 = 0, ne = 0;
        scan_segment_rows(A, gather, p, g0, seg_end, r0, r1, seg_base, slot_s, s_bad);
        auto rows_global = [&](int t, long long &h0, long long &h1, long long &e) {
            const long long gb = g0 + (long long)t * kTile;
            const long long gl = seg_end - 1;
            h0 = unmark_row(A.phys[min(gb + k4, gl)]);
            h1 = unmark_row(A.phys[min(gb + 16 + k4, gl)]);
            e = unmark_row(A.phys[min(gb + (lane >> 1), gl)]);
        };
        for (int s = 0; s < kStages - 1 && s < n_tiles; ++s) {
            long long h0, h1, e;
            if (gather)
                rows_global(s, h0, h1, e);
            else
                rows_direct(s, h0, h1, e);
            issue_stage(A, stages[s], h0, h1, e, phys_src(s + kStages), lane, wave);
        }
        if (gather && kStages - 1 < n_tiles) rows_global(kStages - 1, nh0, nh1, ne);
        SplitState S;
        S.m_run = -INFINITY;
        S.l_run = 0.0f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) S.o[mb][nb] = float4_t{0, 0, 0, 0};

        float4_t ar[4];
        half8_t pa[4], pl[4];
        int t = 0;
        while (t < n_tiles) {
        for (; t < n_tiles; ++t) {
            if (t + kStages - 1 < n_tiles) {
                // refill the stage tile t-1 used (its readers passed B2 of t-1)
                if (!gather) rows_direct(t + kStages - 1, nh0, nh1, ne);
                issue_stage(A, stages[(t + kStages - 1) % kStages], nh0, nh1, ne,
                            phys_src(t + 2 * kStages - 1), lane, wave);
            }
            // The fp32-Q variant spills registers; spill stores share the vmcnt
            // counter with the copies, so it waits for the whole ring.
            wait_copies(kQf32 ? 0 : min(kStages - 1, n_tiles - 1 - t));
            lds_barrier();   // B1: tile t landed; last tile's P/alpha/S slots are consumed

            const uint8_t *st = stages[t % kStages];
            // gathered rows of tile t+kStages rode in with tile t; they are read
            // now, before the next iteration refills any stage
            if (gather && t + kStages < n_tiles) {
                lds_ld_phys3(lds_addr(st + kPhysOff), k4, lane >> 1, nh0, nh1, ne);
                nh0 = unmark_row(nh0);
                nh1 = unmark_row(nh1);
                ne = unmark_row(ne);
            }
            const long long rb = r0 + (long long)t * kTile;

            // ---- 1. partial S^T over this wave's dims; V_w slice to LDS ----------
            float4_t acc[2][4];
            uint4_t cf[2][2], th[2];
            uint2_t ef[2];
            read_wave_frags(st, wave, j, q, cf, ef, th);
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                half8_t a[4];
                dequant16(cf[h2][0], block_scale(ef[h2], 2 * wave), a[0], a[1]);
                if (wave < 3) {
                    dequant16(cf[h2][1], block_scale(ef[h2], 2 * wave + 1), a[2], a[3]);
                } else {
                    a[2] = __builtin_bit_cast(half8_t, cf[h2][1]);
                    a[3] = __builtin_bit_cast(half8_t, th[h2]);
                }
                // V_w row 16h2+j, dims 64*bb + 16q .. +15 (bb = 0,1 within the wave)
                const uint32_t vrow = vt_base + (16 * h2 + j) * kVRowBytes + 32 * q;
                asm volatile("ds_write_b128 %0, %1\n\tds_write_b128 %0, %2 offset:16\n\t"
                             "ds_write_b128 %0, %3 offset:128\n\tds_write_b128 %0, %4 offset:144"
                             :: "v"(vrow), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]) : "memory");
#pragma unroll
                for (int hb = 0; hb < 4; ++hb) {
                    float4_t c = float4_t{0, 0, 0, 0};
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ks], qh[hb][ks], c, 0, 0, 0);
                        if (kQf32)
                            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ks], ql[hb][ks], c, 0, 0, 0);
                    }
                    acc[h2][hb] = c;
                }
            }
            // ---- 2. reduce-scatter S, softmax of the wave's heads ----------------
            // sx layout: [owner][writer][h2][lane] float4
            const uint32_t sx_base = lds_addr(sx);
            {
                const float4_t sv[8] = {acc[0][0], acc[1][0], acc[0][1], acc[1][1],
                                        acc[0][2], acc[1][2], acc[0][3], acc[1][3]};
                lds_st128x8_mfma<0, 1024, 8192, 9216, 16384, 17408, 24576, 25600>(
                    sx_base + ((wave * 2) * 64 + lane) * 16, sv);
            }
            lds_barrier();   // B2: partials visible
            float4_t part[8];   // [w2*2 + h2]
            lds_ld128x8<0, 1024, 2048, 3072, 4096, 5120, 6144, 7168>(
                sx_base + ((wave * 8) * 64 + lane) * 16, part);
            float4_t sacc[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)   // sum in writer order 0..3
                sacc[h2] = ((part[h2] + part[2 + h2]) + part[4 + h2]) + part[6 + h2];
            float s[2][4];
            float tmax = -INFINITY;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool ok = rb + 16 * h2 + 4 * q + r < r1;
                    s[h2][r] = ok ? sacc[h2][r] * A.kq_log2 : -INFINITY;
                    tmax = fmaxf(tmax, s[h2][r]);
                }
            tmax = xmax_16_32(tmax);
            // exact running max as the reference point; P as f16 hi + lo
            const bool bump = tmax > S.m_run;
            const float m_new = bump ? tmax : S.m_run;
            const bool none = m_new == -INFINITY;
            const float alpha = (bump && S.m_run != -INFINITY) ? __builtin_amdgcn_exp2f(S.m_run - m_new) : 1.0f;
            half8_t pf, plo;
            float psum = 0.0f;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = none ? 0.0f : __builtin_amdgcn_exp2f(s[h2][r] - m_new);
                    psum += pv;
                    pf[4 * h2 + r] = (half_t)pv;
                    plo[4 * h2 + r] = (half_t)(pv - (float)pf[4 * h2 + r]);
                }
            S.l_run = S.l_run * alpha + psum;
            S.m_run = m_new;
            const uint32_t pbuf_base = lds_addr(pbuf);
            const uint32_t alpha_base = lds_addr(alpha_s);
            lds_st128(pbuf_base + (wave * 64 + lane) * 16, pf);
            lds_st128(pbuf_base + 4096 + (wave * 64 + lane) * 16, plo);
            if (q == 0) lds_st32(alpha_base + (16 * wave + j) * 4, alpha);
            lds_barrier();   // B3: P and rescale factors of all heads visible

            // ---- 3. O_w += P . V_w --------------------------------------------------
            lds_ld_alpha_p(alpha_base + 16 * q, pbuf_base + lane * 16, ar, pa);
            lds_ld128x4(pbuf_base + 4096 + lane * 16, pl);
            bool need_rescale = false;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
                need_rescale |= ar[mb][0] != 1.0f || ar[mb][1] != 1.0f || ar[mb][2] != 1.0f ||
                                ar[mb][3] != 1.0f;
            need_rescale = __any(need_rescale);
            if (need_rescale) break;   // rare: the rescale runs outside the hot loop
            pv_split(vt_base, j, q, pa, pl, S.o);
        }
        if (t < n_tiles) {
            // a softmax reference point moved: rescale O, then finish tile t
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb) S.o[mb][nb] *= ar[mb];
            pv_split(vt_base, j, q, pa, pl, S.o);
            ++t;
        }
        }

        // ---- emit: O_w rows of all heads over the wave's dims; m, l by owners ------
        {
            const float l = xsum_16_32(S.l_run);
            const long long slot = (long long)blockIdx.x * A.s_max + slot_s;
            float *wo = A.ws_o + slot * (kH * kD) + (4 * q) * kD + 128 * wave + j;
            asm volatile("" : "+v"(wo));
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) wo[(16 * mb + r) * kD + 16 * nb] = S.o[mb][nb][r];
            if (q == 0) {
                A.ws_ml[slot * 2 * kH + 16 * wave + j] = S.m_run;
                A.ws_ml[slot * 2 * kH + kH + 16 * wave + j] = l;
            }
            mark_slot(A, slot, p, slot_s, s_bad, s_badp);
        }
        ++slot_s;
        g0 = seg_end;
        lds_barrier();   // the next segment's copies reuse the ring
    }
    if (threadIdx.x == 0)
        for (int s2 = slot_s; s2 < A.s_max; ++s2) A.ws_prob[(long long)blockIdx.x * A.s_max + s2] = -1;
}

// ---- fp32-row kernel (reference launchers): fragments straight from global -----------
// kSepV: V rows come from f32_v_raw (the raw launcher with V != K); otherwise
// the K fragments are also the V tile (MLA: K == V).
template <bool kSepV>
__global__ __launch_bounds__(256) void decode_f32_kernel(const DecodeArgs A) {
    __shared__ half_t vt[kD * kVtStride];
    __shared__ long long s_start[kMaxProb + 1];
    stage_start(A, s_start);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
    const int j = lane & 15;
    const int q = lane >> 4;
    const int head = wave * 16 + j;

    long long g0 = (long long)blockIdx.x * A.chunk;
    const long long g1 = min(g0 + (long long)A.chunk, A.total);
    int p = 0;
    int slot_s = 0;
    auto row_allowed = [&](long long row) {
        return row < A.f32_n_raw || !A.f32_allowed || A.f32_allowed[row - A.f32_n_raw] != 0;
    };

    while (g0 < g1) {
        while (s_start[p + 1] <= g0) ++p;
        const long long seg_end = min(g1, s_start[p + 1]);
        const long long r0 = g0 - s_start[p];
        const long long r1 = min(seg_end - s_start[p], A.count[p]);

        half8_t qh[16], ql[16];
        load_q<true>(A, p, head, q, qh, ql);
        SegState S;
        seg_init(S);

        for (long long rb = r0; rb < r1; rb += kTile) {
            __syncthreads();   // previous tile's P.V reads of vt are done
            float4_t acc[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                acc[h2] = float4_t{0, 0, 0, 0};
                const long long r = rb + 16 * h2 + j;
                const bool valid = r < r1 && row_allowed(r);
                const float *frow = r < A.f32_n_raw ? A.f32_raw + r * kD
                                                    : A.f32_comp + (r - A.f32_n_raw) * kD;
                const int prow = vt_pos(16 * h2 + j);
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    half8_t a0, a1;
                    load_f32_block(frow, b, q, valid, a0, a1);
                    acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qh[2 * b], acc[h2], 0, 0, 0);
                    acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qh[2 * b + 1], acc[h2], 0, 0, 0);
                    acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, ql[2 * b], acc[h2], 0, 0, 0);
                    acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, ql[2 * b + 1], acc[h2], 0, 0, 0);
                    if ((b >> 1) == wave) {
                        if (kSepV) {
                            half8_t v0, v1;
                            load_f32_block(A.f32_v_raw + r * kD, b, q, valid, v0, v1);
                            vt_write(vt, b, q, prow, v0, v1);
                        } else {
                            vt_write(vt, b, q, prow, a0, a1);
                        }
                    }
                }
            }
            const half8_t pf = softmax_tile(acc, A.kq_log2, q, S, [&](int h2, int r) {
                const long long row = rb + 16 * h2 + 4 * q + r;
                return row < r1 && row_allowed(row);
            });
            __syncthreads();   // V^T tile complete
            pv_tile(vt, pf, j, q, S);
        }
        emit_partial(A, (long long)blockIdx.x * A.s_max + slot_s, wave, j, q, head, p, S);
        ++slot_s;
        g0 = seg_end;
    }
    if (threadIdx.x == 0)
        for (int s2 = slot_s; s2 < A.s_max; ++s2) A.ws_prob[(long long)blockIdx.x * A.s_max + s2] = -1;
}

// ---- warp-specialized FP8 decode: producers and consumers -------------------------
//
// One 8-wave workgroup per chunk, all 64 heads. Waves 0-3 are producers: wave
// d loads dims [128 d, 128 d + 128) of all 32 rows of a tile straight into
// registers two tiles ahead, dequantizes them, computes the partial S of the
// tile for all 64 heads over its dims (32 MFMAs) and writes it to LDS; in the
// next barrier interval it sums the four partials of heads 16 d + [0, 16),
// runs their softmax (exact running max, P as f16 hi + lo), interleaved with
// the next tile's QK MFMAs, and writes the tile's dequantized V slice. Waves
// 4-7 are consumers: wave 4 + c adds P . V over dims [128 c, 128 c + 128) for
// all 64 heads (64 MFMAs) two intervals behind the producers. With one
// producer and one consumer per SIMD, the consumer's MFMAs run while the
// producer's VALU work issues; one barrier per tile:
//   interval i: producers: softmax(i - 1), V(i - 1) -> LDS, QK(i) -> S(i);
//               consumers: P . V(i - 2).
// S partials, P, the rescale factors and V are double-buffered by tile parity.

// P in LDS: [buf][hi, lo][head tile][lane] f16 x 8: the MFMA A fragment of
// lane (j, q) is rows 4 q + [0, 4) and 16 + 4 q + [0, 4) of head j, which is
// what the producer lane (j, q) holds; both sides access it lane-contiguously.
__device__ inline uint32_t pws_off(int buf, int hl, int hb, int lane) {
    return (uint32_t)((((buf * 2 + hl) * 4 + hb) * 64 + lane) * 16);
}

template <int kMode, bool kPLo>
__global__ __launch_bounds__(512, 1) void decode_ws_kernel(const DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t vtile[2][4][kVTileBytes];   // [tile & 1][dim quarter]
    __shared__ __attribute__((aligned(16))) float4_t sx[2][4][4][2][64];  // [tile & 1][head tile][dim quarter][row half][lane]
    __shared__ __attribute__((aligned(16))) uint8_t pws[2 * 2 * 4 * 64 * 16];
    __shared__ __attribute__((aligned(16))) float alpha_s[2][kH];
    __shared__ long long s_start[kMaxProb + 1];
    __shared__ long long s_rowbase[kMaxProb];
    __shared__ int s_badp[kMaxProb], s_bad[2];
    stage_rowbase(A, s_rowbase, s_badp);
    if (threadIdx.x < 2) s_bad[threadIdx.x] = 0;
    stage_start(A, s_start);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = wave < 4;
    const int d = wave & 3;   // dim quarter; for a consumer also its softmax head tile
    const int j = lane & 15;
    const int q = lane >> 4;

    long long g0 = (long long)blockIdx.x * A.chunk;
    const long long g1 = min(g0 + (long long)A.chunk, A.total);
    int p = 0;
    int slot_s = 0;
    while (g0 < g1) {
        while (s_start[p + 1] <= g0) ++p;
        const long long seg_end = min(g1, s_start[p + 1]);
        const long long r0 = g0 - s_start[p];
        const long long r1 = min(seg_end - s_start[p], A.count[p]);
        const int n_tiles = 2 * (int)((r1 - r0 + 2 * kTile - 1) / (2 * kTile));   // even, >= 2
        const long long slot = (long long)blockIdx.x * A.s_max + slot_s;
        scan_segment_rows(A, kMode == 1, p, g0, seg_end, r0, r1, s_rowbase[p], slot_s, s_bad);
        if (producer) {
            const long long seg_base = s_rowbase[p];
            // kT: the wave of dims [384, 512): one FP8 block + the f16 RoPE tail
            auto produce = [&](auto tail_c) {
                constexpr bool kT = decltype(tail_c)::value;
                // gathered rows: this lane's cache row in row half hh of tile t (past
                // the end: the last row)
                auto row_gather = [&](int t, int hh) -> long long {
                    const long long lr = min((long long)t * kTile + 16 * hh + j, r1 - 1 - r0);
                    if (kMode == 1) return unmark_row(A.phys[g0 + lr]);
                    return clamp_row(seg_base + A.row_idx[(long long)p * A.row_idx_stride + r0 + lr],
                                     A.n_cache_rows);
                };
                // codes 128 d + 16 q + [0, 16) and 128 d + 64 + 16 q + [0, 16), or
                // (kT) codes 384 + 16 q + [0, 16) and tail dims 16 q + [0, 16);
                // e: the exponent word of blocks 2 d, 2 d + 1
                struct Tl { uint4_t c0, c1, c2; uint32_t e; };
                auto load = [&](long long r, Tl &T) {
                    const uint8_t *cr = A.codes + r * kNope + 128 * d + 16 * q;
                    T.c0 = *reinterpret_cast<const uint4_t *>(cr);
                    if (kT) {
                        const uint8_t *tr = reinterpret_cast<const uint8_t *>(A.tail) + r * (2 * kRot) + 32 * q;
                        T.c1 = *reinterpret_cast<const uint4_t *>(tr);
                        T.c2 = *reinterpret_cast<const uint4_t *>(tr + 16);
                    } else {
                        T.c1 = *reinterpret_cast<const uint4_t *>(cr + 64);
                    }
                    // only the word this wave uses: a loaded but unused register can be
                    // reallocated before the load returns, which forces a full wait
                    T.e = *reinterpret_cast<const uint32_t *>(A.sexp + r * 8 + (d >= 2 ? 4 : 0));
                };
                // direct rows: 32-bit row offsets from the segment's first row (a
                // segment is at most one chunk of rows), so that the loads take a
                // uniform 64-bit base and one 32-bit offset each
                const long long seg_r0 = seg_base + r0;
                const int seg_last = (int)(r1 - 1 - r0);
                const uint8_t *codes_s = A.codes + seg_r0 * kNope + 128 * d;
                const uint8_t *tail_s = reinterpret_cast<const uint8_t *>(A.tail) + seg_r0 * (2 * kRot);
                const uint8_t *sexp_s = reinterpret_cast<const uint8_t *>(A.sexp) + seg_r0 * 8 + (d >= 2 ? 4 : 0);
                auto load_direct = [&](int t, int hh, Tl &T) {
                    const uint32_t lr = (uint32_t)min(t * kTile + 16 * hh + j, seg_last);
                    T.c0 = *reinterpret_cast<const uint4_t *>(codes_s + (lr * kNope + 16 * q));
                    if (kT) {
                        T.c1 = *reinterpret_cast<const uint4_t *>(tail_s + (lr * (2 * kRot) + 32 * q));
                        T.c2 = *reinterpret_cast<const uint4_t *>(tail_s + (lr * (2 * kRot) + 32 * q + 16));
                    } else {
                        T.c1 = *reinterpret_cast<const uint4_t *>(codes_s + (lr * kNope + 16 * q + 64));
                    }
                    T.e = *reinterpret_cast<const uint32_t *>(sexp_s + lr * 8);
                };
                // Q^T fragments of all 64 heads over dims d: the raw bf16 loads are
                // issued before the first tiles' loads and converted after them, so
                // the two memory round trips overlap
                uint4_t qraw[4][4];
#pragma unroll
                for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        const int dd = 64 * (2 * d + (ks >> 1)) + 16 * q + 8 * (ks & 1);
                        qraw[hb][ks] = *reinterpret_cast<const uint4_t *>(
                            static_cast<const uint16_t *>(A.q) + (long long)p * A.q_stride +
                            (long long)(16 * hb + j) * kD + dd);
                    }
                half8_t qh[4][4];
                auto dequant = [&](const Tl (&cur)[2], half8_t (&av)[2][4]) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        dequant16(cur[hh].c0, pow2f((int)(int8_t)((cur[hh].e >> (16 * (d & 1))) & 0xFF)),
                                  av[hh][0], av[hh][1]);
                        if (kT) {
                            // explicit copies here, where the data is due: left to the
                            // compiler they become loop-carried copies at the loop head,
                            // which wait for the loads of the next tile as well
                            uint4_t t1, t2;
                            asm volatile("v_mov_b32 %0, %4\n\tv_mov_b32 %1, %5\n\tv_mov_b32 %2, %6\n\tv_mov_b32 %3, %7"
                                         : "=v"(t1[0]), "=v"(t1[1]), "=v"(t1[2]), "=v"(t1[3])
                                         : "v"(cur[hh].c1[0]), "v"(cur[hh].c1[1]), "v"(cur[hh].c1[2]), "v"(cur[hh].c1[3]));
                            asm volatile("v_mov_b32 %0, %4\n\tv_mov_b32 %1, %5\n\tv_mov_b32 %2, %6\n\tv_mov_b32 %3, %7"
                                         : "=v"(t2[0]), "=v"(t2[1]), "=v"(t2[2]), "=v"(t2[3])
                                         : "v"(cur[hh].c2[0]), "v"(cur[hh].c2[1]), "v"(cur[hh].c2[2]), "v"(cur[hh].c2[3]));
                            av[hh][2] = __builtin_bit_cast(half8_t, t1);
                            av[hh][3] = __builtin_bit_cast(half8_t, t2);
                        } else {
                            dequant16(cur[hh].c1, pow2f((int)(int8_t)((cur[hh].e >> (16 * (d & 1) + 8)) & 0xFF)),
                                      av[hh][2], av[hh][3]);
                        }
                    }
                };
                // loads of tile u + 2 into cur (gathered rows: those of tile u + 2
                // are in ph_use; the row numbers of tile u + 3 are fetched first)
                auto refill = [&](int u, Tl (&cur)[2], long long (&ph_use)[2], long long (&ph_next)[2]) {
                    if (kMode != 0) {
                        ph_next[0] = row_gather(u + 3, 0);
                        ph_next[1] = row_gather(u + 3, 1);
                        __builtin_amdgcn_sched_barrier(0);
                        load(ph_use[0], cur[0]);
                        load(ph_use[1], cur[1]);
                    } else {
                        load_direct(u + 2, 0, cur[0]);
                        load_direct(u + 2, 1, cur[1]);
                    }
                };
                // partial S of a tile over dims d
                auto qk = [&](const half8_t (&av)[2][4], float4_t (&acc)[4][2]) {
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            float4_t c = float4_t{0, 0, 0, 0};
#pragma unroll
                            for (int ks = 0; ks < 4; ++ks)
                                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[hh][ks], qh[hb][ks], c, 0, 0, 0);
                            acc[hb][hh] = c;
                        }
                };
                auto store_s = [&](int u, const float4_t (&acc)[4][2]) {
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh)
                            sx[u & 1][hb][d][hh][lane] = acc[hb][hh];   // compiler-visible: MFMA hazard waits inserted
                };
                // V slice of tile t -> LDS: rows with bit 2 set swap the 16-byte
                // halves of their 32-byte column groups, so that the 8 lanes of a
                // 16-byte store phase cover all banks (the transposing reads
                // apply the same swap)
                auto store_v = [&](int t, const half8_t (&av)[2][4]) {
                    const uint32_t sw = (j & 4) ? 16u : 0u;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const uint32_t vrow = lds_addr(vtile[t & 1][d]) + (16 * hh + j) * kVRowBytes + 32 * q;
                        const uint32_t va = vrow + sw, vb = vrow + (16u - sw);
                        asm volatile("ds_write_b128 %0, %2\n\tds_write_b128 %1, %3\n\t"
                                     "ds_write_b128 %0, %4 offset:128\n\tds_write_b128 %1, %5 offset:128"
                                     :: "v"(va), "v"(vb), "v"(av[hh][0]), "v"(av[hh][1]), "v"(av[hh][2]),
                                        "v"(av[hh][3]) : "memory");
                    }
                };
                float m_run = -INFINITY, l_run = 0.0f;   // head 16 d + j; l over this lane's rows
                auto read_s = [&](int t, float4_t (&sa)[2]) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        sa[hh] = ((sx[t & 1][d][0][hh][lane] + sx[t & 1][d][1][hh][lane]) +
                                  sx[t & 1][d][2][hh][lane]) + sx[t & 1][d][3][hh][lane];
                };
                // softmax of tile t for heads 16 d + [0, 16) -> P, alpha
                auto softmax = [&](int t, const float4_t (&sa)[2]) {
                    const int b = t & 1;
                    const long long left = r1 - (r0 + (long long)t * kTile);
                    const int nv = left < kTile ? (int)left : kTile;   // valid rows of the tile
                    float s8[2][4];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r) s8[hh][r] = sa[hh][r] * A.kq_log2;
                    if (nv < kTile) {   // (uniform) the segment's last tile: rows past its end take no part
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (16 * hh + 4 * q + r >= nv) s8[hh][r] = -INFINITY;
                    }
                    float tmax = -INFINITY;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, s8[hh][r]);
                    tmax = xmax_16_32(tmax);
                    // lazy reference point: it moves to the tile max only when that
                    // exceeds it by more than 2^kLazyLog2 in P (P up to 256 is exact
                    // enough as f16 hi + lo), so O is rescaled on few tiles
                    const bool bump = tmax > m_run + kLazyLog2;
                    const float m_new = bump ? tmax : m_run;
                    const bool none = m_new == -INFINITY;
                    const float alpha = (bump && m_run != -INFINITY) ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
                    float psum = 0.0f;
                    // kPLo: P as f16 hi + lo (p - hi), so that P . V carries ~22 bits
                    // of P. Otherwise P is one f16 and l sums the rounded values, so
                    // that O stays an exactly normalized average of V rows with
                    // weights off by at most 2^-11 relative. Element 4 hh + r of lane
                    // (j, q) is row 16 hh + 4 q + r of head j, the K order of the V
                    // fragments.
                    half8_t pf, pl;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float pv = none ? 0.0f : __builtin_amdgcn_exp2f(s8[hh][r] - m_new);
                            pf[4 * hh + r] = (half_t)pv;
                            if (kPLo) {
                                psum += pv;
                                pl[4 * hh + r] = (half_t)(pv - (float)pf[4 * hh + r]);
                            } else {
                                psum += (float)pf[4 * hh + r];
                            }
                        }
                    *reinterpret_cast<half8_t *>(pws + pws_off(b, 0, d, lane)) = pf;
                    if (kPLo) *reinterpret_cast<half8_t *>(pws + pws_off(b, 1, d, lane)) = pl;
                    l_run = l_run * alpha + psum;
                    m_run = m_new;
                    if (q == 0) alpha_s[b][16 * d + j] = alpha;
                };
                // interval u (1 <= u < n): S(u - 1) reads, V(u - 1) -> LDS,
                // dequantize u, loads of u + 2, QK(u) MFMAs with softmax(u - 1)
                // interleaved into their issue slots, S(u) -> LDS
                auto interval = [&](int u, Tl (&cur)[2], half8_t (&av)[2][4], long long (&ph_use)[2],
                                    long long (&ph_next)[2]) {
                    float4_t sa[2];
                    read_s(u - 1, sa);
                    store_v(u - 1, av);
                    dequant(cur, av);
                    __builtin_amdgcn_sched_barrier(0);
                    refill(u, cur, ph_use, ph_next);
                    __builtin_amdgcn_sched_barrier(0);
                    float4_t acc[4][2];
                    qk(av, acc);
                    softmax(u - 1, sa);
                    store_s(u, acc);
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // three VALU
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };

                // prologue (issue order = the loop's: tile 0, [rows of tile 2], tile 1)
                Tl T0[2], T1[2];
                long long ph0[2] = {0, 0}, ph1[2] = {0, 0};
                __builtin_amdgcn_sched_barrier(0);
                if (kMode != 0) {
                    const long long ra0 = row_gather(0, 0), ra1 = row_gather(0, 1);
                    const long long rb0 = row_gather(1, 0), rb1 = row_gather(1, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    load(ra0, T0[0]);
                    load(ra1, T0[1]);
                    __builtin_amdgcn_sched_barrier(0);
                    ph0[0] = row_gather(2, 0);
                    ph0[1] = row_gather(2, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    load(rb0, T1[0]);
                    load(rb1, T1[1]);
                } else {
                    load_direct(0, 0, T0[0]);
                    load_direct(0, 1, T0[1]);
                    __builtin_amdgcn_sched_barrier(0);
                    load_direct(1, 0, T1[0]);
                    load_direct(1, 1, T1[1]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        const uint4_t v = qraw[hb][ks];
                        half8_t x;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            x[2 * i] = (half_t)bf16_to_f32((uint16_t)(v[i] & 0xFFFF));
                            x[2 * i + 1] = (half_t)bf16_to_f32((uint16_t)(v[i] >> 16));
                        }
                        qh[hb][ks] = x;
                    }
                half8_t av[2][4];
                dequant(T0, av);   // interval 0
                __builtin_amdgcn_sched_barrier(0);
                refill(0, T0, ph0, ph1);
                __builtin_amdgcn_sched_barrier(0);
                {
                    float4_t acc[4][2];
                    qk(av, acc);
                    store_s(0, acc);
                }
                lds_barrier();
                for (int t = 1; t < n_tiles - 1; t += 2) {
                    interval(t, T1, av, ph1, ph0);
                    lds_barrier();
                    interval(t + 1, T0, av, ph0, ph1);
                    lds_barrier();
                }
                interval(n_tiles - 1, T1, av, ph1, ph0);
                lds_barrier();
                {   // interval n: softmax(n - 1), V(n - 1) -> LDS
                    float4_t sa[2];
                    read_s(n_tiles - 1, sa);
                    store_v(n_tiles - 1, av);
                    softmax(n_tiles - 1, sa);
                }
                lds_barrier();
                lds_barrier();              // interval n + 1
                // m, l of heads 16 d + j
                const float l = xsum_16_32(l_run);
                if (q == 0) {
                    A.ws_ml[slot * 2 * kH + 16 * d + j] = m_run;
                    A.ws_ml[slot * 2 * kH + kH + 16 * d + j] = l;
                }
            };
            if (d == 3)
                produce(std::true_type{});
            else
                produce(std::false_type{});
        } else {
            float4_t o[4][8];   // heads 16 hb + 4 q + r, dims 128 d + 16 nb + j
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int c = 0; c < 8; ++c) o[a][c] = float4_t{0, 0, 0, 0};
            // O += P(t) . V(t) over dims d for all 64 heads (after the rescale by alpha(t))
            auto pv = [&](int t) {
                const int b = t & 1;
                half8_t pa[4], pl[4];
                float4_t ar[4];
#pragma unroll
                for (int hb = 0; hb < 4; ++hb) {
                    pa[hb] = *reinterpret_cast<const half8_t *>(pws + pws_off(b, 0, hb, lane));
                    if (kPLo) pl[hb] = *reinterpret_cast<const half8_t *>(pws + pws_off(b, 1, hb, lane));
                    ar[hb] = *reinterpret_cast<const float4_t *>(&alpha_s[b][16 * hb + 4 * q]);
                }
                const uint32_t vt = lds_addr(vtile[b][d]);
                uint2_t tb[2][8];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t ab = vt + (4 * q + (j >> 2)) * kVRowBytes + 8 * ((j & 3) ^ ((q & 1) << 1)) + 128 * half;
                    asm volatile(
                        "ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %1, %8 offset:4608\n\t"
                        "ds_read_b64_tr_b16 %2, %8 offset:32\n\tds_read_b64_tr_b16 %3, %8 offset:4640\n\t"
                        "ds_read_b64_tr_b16 %4, %8 offset:64\n\tds_read_b64_tr_b16 %5, %8 offset:4672\n\t"
                        "ds_read_b64_tr_b16 %6, %8 offset:96\n\tds_read_b64_tr_b16 %7, %8 offset:4704"
                        : "=&v"(tb[half][0]), "=&v"(tb[half][1]), "=&v"(tb[half][2]), "=&v"(tb[half][3]),
                          "=&v"(tb[half][4]), "=&v"(tb[half][5]), "=&v"(tb[half][6]), "=&v"(tb[half][7])
                        : "v"(ab));
                }
                // P, alpha and the first half's V fragments (the second half's 8
                // reads may still be in flight; LDS returns in order)
                asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
                bool need = false;
#pragma unroll
                for (int hb = 0; hb < 4; ++hb)
                    need |= ar[hb][0] != 1.0f || ar[hb][1] != 1.0f || ar[hb][2] != 1.0f || ar[hb][3] != 1.0f;
                if (__any(need)) {   // rare: a reference point moved
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                        for (int nb = 0; nb < 8; ++nb) o[hb][nb] *= ar[hb];
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    if (half == 1) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    half8_t vb[4];
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb)
                        vb[nb] = __builtin_bit_cast(half8_t, uint4_t{tb[half][2 * nb][0], tb[half][2 * nb][1],
                                                                     tb[half][2 * nb + 1][0], tb[half][2 * nb + 1][1]});
                    // hi products first, then lo: dependent MFMAs sixteen apart
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                        for (int hb = 0; hb < 4; ++hb)
                            o[hb][4 * half + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                pa[hb], vb[nb], o[hb][4 * half + nb], 0, 0, 0);
                    if (kPLo) {
#pragma unroll
                        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                            for (int hb = 0; hb < 4; ++hb)
                                o[hb][4 * half + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    pl[hb], vb[nb], o[hb][4 * half + nb], 0, 0, 0);
                    }
                }
            };
            lds_barrier();   // interval 0
            lds_barrier();   // interval 1
            for (int t = 0; t < n_tiles; ++t) {   // interval t + 2
                pv(t);
                lds_barrier();
            }
            float *wo = A.ws_o + slot * (kH * kD) + (4 * q) * kD + 128 * d + j;
            asm volatile("" : "+v"(wo));
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) wo[(16 * hb + r) * kD + 16 * nb] = o[hb][nb][r];
        }
        mark_slot(A, slot, p, slot_s, s_bad, s_badp);
        ++slot_s;
        g0 = seg_end;
    }
    if (threadIdx.x == 0)
        for (int s2 = slot_s; s2 < A.s_max; ++s2) A.ws_prob[(long long)blockIdx.x * A.s_max + s2] = -1;
}

// ---- flat-stage FP8 decode (direct rows) ----------------------------------------------
//
// One 8-wave workgroup per chunk, all 64 heads, as decode_ws_kernel, with the
// tile copied HBM -> LDS by the consumers' global_load_lds instructions and
// read from there by everyone:
//  * Each 32-row tile takes 20 copy instructions (19 of 16 bytes per lane, one
//    of 4 for the exponents), each 1 KB of consecutive cache bytes (whole rows
//    of codes, then of tails), 5 per consumer wave, kFsLead tiles ahead.
//  * LDS layout of a stage, chosen so that every fragment read runs at the
//    full LDS rate (measured on gfx950: a 16-byte read of 16 lanes is
//    conflict-free when the lanes' rows are 480 bytes apart, and at half rate
//    for 464 or 448): code rows of 480 bytes (28 code chunks + 2 pad chunks
//    that re-read chunk 27), then tail rows of 128 bytes whose 16-byte chunk c
//    sits at position c ^ ((row >> 1) & 7), then the rows' 8 exponents, then
//    the f16 scale table the producers write for the consumers.
//  * Producer wave d: QK^T of heads [16d, 16d+16) on the scaled FP8 MFMA, then
//    the softmax one interval later; consumer wave c: P . V over dims
//    [128c, 128c+128) for all 64 heads, two intervals behind the QK.
constexpr int kFsCodeRow = kNope + 32;                    // 480: codes + 2 pad chunks
constexpr int kFsTailRow = 2 * kRot;                      // 128: f16 tail, swizzled chunks
constexpr int kFsTailOff = kTile * kFsCodeRow;            // 15360
constexpr int kFsExpOff = kFsTailOff + kTile * kFsTailRow; // 19456
constexpr int kFsBytes = kFsExpOff + kTile * 8;           // 19712
constexpr int kFsScaleOff = kFsBytes;                     // f16 2^e per [block][row]
constexpr int kFsSlot = kFsBytes + 8 * kTile * 2;          // 20224
// gathered rows: the physical rows of the tile kFsLead tiles later (32
// int64, copied by consumer wave 0) ride in the stage after the scale table
constexpr int kFsPhysOff = kFsSlot;
constexpr int kFsSlotGather = kFsSlot + kTile * 8;         // 20480
constexpr int kFsStages = 6;
constexpr int kFsLead = 3;                                 // tiles copied ahead of the producers
constexpr int kFsCodeChunks = kTile * (kFsCodeRow / 16);  // 960
constexpr int kFsChunks = kFsCodeChunks + kTile * (kFsTailRow / 16);   // 1216 = 19 x 64
static_assert(kFsCodeChunks % 64 == 0, "code and tail chunks take separate copy instructions");
// LDS chunk position of tail chunk c of tile row r (an involution on c)
__device__ __host__ constexpr int fs_tail_pos(int r, int c) { return c ^ ((r >> 1) & 7); }
static_assert(kFsChunks == 19 * 64, "codes + tails fill 19 copy instructions");

// Consumer side shared by the decode kernels: O[64 heads x 128 dims] of dim
// quarter d += P(t) . V(t) for the tiles of one segment, then the partial O.
template <bool kPLo>
__device__ inline void consume_segment(const DecodeArgs &A, uint8_t (*vtile)[4][kVTileBytes],
                                       const uint8_t *pws, const float (*alpha_s)[kH],
                                       int n_tiles, long long slot, int lane, int j, int q,
                                       int d, int lead) {
    float4_t o[4][8];   // heads 16 hb + 4 q + r, dims 128 d + 16 nb + j
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 8; ++c) o[a][c] = float4_t{0, 0, 0, 0};
    auto pv = [&](int t) {
        const int b = t & 1;
        half8_t pa[4], pl[4];
        float4_t ar[4];
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
            pa[hb] = *reinterpret_cast<const half8_t *>(pws + pws_off(b, 0, hb, lane));
            if (kPLo) pl[hb] = *reinterpret_cast<const half8_t *>(pws + pws_off(b, 1, hb, lane));
            ar[hb] = *reinterpret_cast<const float4_t *>(&alpha_s[b][16 * hb + 4 * q]);
        }
        const uint32_t vt = lds_addr(vtile[b][d]);
        uint2_t tb[2][8];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t ab = vt + (4 * q + (j >> 2)) * kVRowBytes + 8 * ((j & 3) ^ ((q & 1) << 1)) + 128 * half;
            asm volatile(
                "ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %1, %8 offset:4608\n\t"
                "ds_read_b64_tr_b16 %2, %8 offset:32\n\tds_read_b64_tr_b16 %3, %8 offset:4640\n\t"
                "ds_read_b64_tr_b16 %4, %8 offset:64\n\tds_read_b64_tr_b16 %5, %8 offset:4672\n\t"
                "ds_read_b64_tr_b16 %6, %8 offset:96\n\tds_read_b64_tr_b16 %7, %8 offset:4704"
                : "=&v"(tb[half][0]), "=&v"(tb[half][1]), "=&v"(tb[half][2]), "=&v"(tb[half][3]),
                  "=&v"(tb[half][4]), "=&v"(tb[half][5]), "=&v"(tb[half][6]), "=&v"(tb[half][7])
                : "v"(ab));
        }
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
        bool need = false;
#pragma unroll
        for (int hb = 0; hb < 4; ++hb)
            need |= ar[hb][0] != 1.0f || ar[hb][1] != 1.0f || ar[hb][2] != 1.0f || ar[hb][3] != 1.0f;
        if (__any(need)) {   // rare: a reference point moved
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb) o[hb][nb] *= ar[hb];
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (half == 1) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            half8_t vb[4];
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
                vb[nb] = __builtin_bit_cast(half8_t, uint4_t{tb[half][2 * nb][0], tb[half][2 * nb][1],
                                                             tb[half][2 * nb + 1][0], tb[half][2 * nb + 1][1]});
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int hb = 0; hb < 4; ++hb)
                    o[hb][4 * half + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        pa[hb], vb[nb], o[hb][4 * half + nb], 0, 0, 0);
            if (kPLo) {
#pragma unroll
                for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
                        o[hb][4 * half + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            pl[hb], vb[nb], o[hb][4 * half + nb], 0, 0, 0);
            }
        }
    };
    // the producers' barriers before P(0) and V(0) are published
    for (int i = 0; i < lead; ++i) lds_barrier();
    for (int t = 0; t < n_tiles; ++t) {   // interval t + lead
        pv(t);
        lds_barrier();
    }
    float *wo = A.ws_o + slot * (kH * kD) + (4 * q) * kD + 128 * d + j;
    asm volatile("" : "+v"(wo));
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) wo[(16 * hb + r) * kD + 16 * nb] = o[hb][nb][r];
}

// The LDS reads of one stage row for a producer lane (no wait): the 7 code
// chunks c[b] = dims 64 b + 16 q + [0, 16), the f16 tail chunks t[s] = dims
// 448 + 32 s + 8 q + [0, 8) (at tail_a[s]) and the row's 8 exponents. lds_rows_wait completes the
// reads of both row halves; their registers are tied to the wait so that
// nothing reads them before it.
__device__ inline void lds_read_row(uint32_t code_a, uint32_t tail_a0, uint32_t tail_a1, uint32_t exp_a,
                                    uint4_t (&c)[7], uint4_t (&t)[2], uint2_t &e) {
    asm volatile(
        "ds_read_b128 %0, %10\n\tds_read_b128 %1, %10 offset:64\n\t"
        "ds_read_b128 %2, %10 offset:128\n\tds_read_b128 %3, %10 offset:192\n\t"
        "ds_read_b128 %4, %10 offset:256\n\tds_read_b128 %5, %10 offset:320\n\t"
        "ds_read_b128 %6, %10 offset:384\n\tds_read_b128 %7, %11\n\t"
        "ds_read_b128 %8, %12\n\tds_read_b64 %9, %13"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]),
          "=&v"(c[6]), "=&v"(t[0]), "=&v"(t[1]), "=&v"(e)
        : "v"(code_a), "v"(tail_a0), "v"(tail_a1), "v"(exp_a));
}
__device__ inline void lds_row_wait(uint4_t (&c)[7], uint4_t (&t)[2], uint2_t &e) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]),
                   "+v"(c[6]), "+v"(t[0]), "+v"(t[1]), "+v"(e)
                 :: "memory");
}

typedef unsigned int uint8x_t __attribute__((ext_vector_type(8)));
// f(integral_constant<int, i>) for i = 0 .. N-1 (indices usable as constant
// builtin operands)
template <int N, typename F>
__device__ inline void static_for(F &&f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}
__device__ inline uint8x_t uint4x2_cat(uint4_t a, uint4_t b) {
    return uint8x_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
__device__ inline uint8x_t qf8v(const uint32_t (&w)[8]) {
    return uint8x_t{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
}

// max of two floats without the quieting of signalling NaNs that fmaxf adds
// for operands of unknown origin (the scores here are never NaN)
__device__ inline float vmax_f32(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ inline float xmax_16_32_raw(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = vmax_f32(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return vmax_f32(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// kLean: the producer form with fewer VALU instructions per tile (packed
// E8M0 row scales from one byte permute, the f16 scale table from
// v_ldexp_f16, P's row sums by v_dot2, one select for empty tiles, whole-tile
// copies from an SGPR base). The score scale log2(e)/sqrt(d) stays on S after
// the MFMA: folded into Q it would make the bf16 values inexact in the two
// E4M3 parts (a bf16 value's 8 significant bits split exactly into hi + lo).
// kGather: 0 direct rows; 1 physical rows from the phys array (phys_kernel
// ran: pages and / or row lists); 2 the int32 row list itself (no pages: row
// = the problem's base + entry, clamped into the cache)
template <bool kPLo, bool kLean, int kQf32 = 0, int kGather = 0>
__global__ __launch_bounds__(512, 1) void decode_flat_kernel(const DecodeArgs A) {
    static_assert(kLean || !kQf32, "fp32 Q takes the lean form");
    // Q parts on the scaled FP8 MFMA: a bf16 Q (8 significant bits) fits in
    // two E4M3 parts; an fp32 Q takes three (about 12 bits: the score error of
    // the dropped rest is ~2^-12 of |q| |k|)
    constexpr int kParts = kQf32 ? 3 : 2;
    static_assert(kLean || !kGather, "gathered rows take the lean form");
    // copies per consumer wave and tile: 5 of the tile, plus (gathered rows,
    // consumer wave 0) one of the physical rows of a later tile
    __shared__ __attribute__((aligned(16))) uint8_t stage[kFsStages][kGather ? kFsSlotGather : kFsSlot];
    __shared__ int s_bad[2];
    // P: [hi, lo (kPLo)][t & 1][head tile][lane] f16 x 8
    __shared__ __attribute__((aligned(16))) uint8_t pws[(kPLo ? 2 : 1) * 2 * 4 * 64 * 16];
    __shared__ __attribute__((aligned(16))) float alpha_s[2][kH];
    __shared__ __attribute__((aligned(16))) int rescale_s[2][4];   // [t & 1][head tile]: some alpha != 1
    __shared__ long long s_start[kMaxProb + 1];
    __shared__ long long s_rowbase[kMaxProb];
    __shared__ int s_badp[kMaxProb];
    // kQf32: each producer lane's f16 hi + lo tail fragments of Q, read back
    // per row half (held in registers they would push the producers past 256
    // VGPRs): [wave][hi s0, hi s1, lo s0, lo s1][lane]
    __shared__ __attribute__((aligned(16))) half8_t q_tail_s[kQf32 ? 4 * 4 * 64 : 1];
    stage_rowbase(A, s_rowbase, s_badp);
    if (threadIdx.x < 2) s_bad[threadIdx.x] = 0;
    stage_start(A, s_start);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = wave < 4;
    const int d = wave & 3;   // producer: head tile; consumer: dim quarter
    const int j = lane & 15;
    const int q = lane >> 4;

    long long g0 = (long long)blockIdx.x * A.chunk;
    const long long g1 = min(g0 + (long long)A.chunk, A.total);
    int p = 0;
    int slot_s = 0;
    while (g0 < g1) {
        while (s_start[p + 1] <= g0) ++p;
        const long long seg_end = min(g1, s_start[p + 1]);
        const long long r0 = g0 - s_start[p];
        const long long r1 = min(seg_end - s_start[p], A.count[p]);
        const int n_tiles = (int)((r1 - r0 + kTile - 1) / kTile);
        const long long slot = (long long)blockIdx.x * A.s_max + slot_s;
        const long long seg_r0 = s_rowbase[p] + r0;
        const int seg_last = (int)(r1 - 1 - r0);
        // ---- the producers: QK^T on the scaled FP8 MFMA and the softmax, one
        // interval apart (interval u: QK(u) with softmax(u - 1) in its issue slots)
        auto produce = [&]() {
            // Q of head 16 d + j as the scaled FP8 MFMA's B operand (q_prep_lane),
            // converted here or (kQf32 == 2) loaded as the prologue converted it
            uint32_t qf8[4][kParts][8];
            int qsc[kParts];
            half8_t qt[2], qtl[2];
            {
                if constexpr (kQf32 == 2) {
                    const uint4_t *src = reinterpret_cast<const uint4_t *>(static_cast<const uint32_t *>(A.q) +
                                                                           (long long)p * A.q_stride);
                    q_prep_load(src, 64 * d + lane, qf8, qsc, qt, qtl);
                } else {
                    const long long qoff = (long long)p * A.q_stride + (long long)(16 * d + j) * kD;
                    const void *qrow = kQf32 ? static_cast<const void *>(static_cast<const float *>(A.q) + qoff)
                                             : static_cast<const void *>(static_cast<const uint16_t *>(A.q) + qoff);
                    q_prep_lane<kQf32 != 0, kLean>(qrow, q, qf8, qsc, qt, qtl);
                }
                if constexpr (kQf32 != 0) {   // this lane's slots only: no other wave reads them
                    const uint32_t qa = lds_addr(&q_tail_s[(d * 4) * 64]) + 16 * lane;
                    asm volatile("ds_write_b128 %0, %1\n\tds_write_b128 %0, %2 offset:1024\n\t"
                                 "ds_write_b128 %0, %3 offset:2048\n\tds_write_b128 %0, %4 offset:3072"
                                 :: "v"(qa), "v"(qt[0]), "v"(qt[1]), "v"(qtl[0]), "v"(qtl[1]) : "memory");
                }
            }
            // stage 0 complete (the consumers' prologue copies); the Q work above
            // ran under those copies
            lds_barrier();
            float m_run = -INFINITY, l_run = 0.0f;   // head 16 d + j; l over this lane's rows
            // softmax of tile t (S^T in sa) for heads 16 d + [0, 16) -> P, alpha in LDS
            auto softmax = [&](int t, const float4_t (&sa)[2]) {
                const int b = t & 1;
                const long long left = r1 - (r0 + (long long)t * kTile);
                const int nv = left < kTile ? (int)left : kTile;
                float s8[2][4];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s8[hh][r] = sa[hh][r] * A.kq_log2;
                if (nv < kTile) {
                    int ln = lane;   // opaque: the row numbers are not held through the loop
                    asm volatile("" : "+v"(ln));
                    const int rq = 4 * (ln >> 4);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (16 * hh + rq + r >= nv) s8[hh][r] = -INFINITY;
                }
                float tmax = -INFINITY;
                if constexpr (kLean) {
                    tmax = s8[0][0];
#pragma unroll
                    for (int i = 1; i < 8; ++i) tmax = vmax_f32(tmax, s8[i >> 2][i & 3]);
                    tmax = xmax_16_32_raw(tmax);
                } else {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, s8[hh][r]);
                    tmax = xmax_16_32(tmax);
                }
                // lazy reference point (as decode_ws_kernel): it moves only when the
                // tile max exceeds it by more than 2^kLazyLog2 in P
                const bool bump = tmax > m_run + kLazyLog2;
                const float m_new = bump ? tmax : m_run;
                const bool none = m_new == -INFINITY;
                const float alpha = (bump && m_run != -INFINITY) ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
                // kLean: with no finite score yet every s8 is -inf, and exp2(-inf - 0) = 0
                const float m_use = none ? 0.0f : m_new;
                float psum = 0.0f;
                half8_t pf, pl;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float pv = kLean ? __builtin_amdgcn_exp2f(s8[hh][r] - m_use)
                                               : (none ? 0.0f : __builtin_amdgcn_exp2f(s8[hh][r] - m_new));
                        pf[4 * hh + r] = (half_t)pv;
                        if (kPLo) {
                            psum += pv;
                            pl[4 * hh + r] = (half_t)(pv - (float)pf[4 * hh + r]);
                        } else if (!kLean) {
                            psum += (float)pf[4 * hh + r];
                        }
                    }
                if constexpr (kLean && !kPLo) {   // the rounded P values, summed in pairs
                    const half2_t one2 = half2_t{(half_t)1.0f, (half_t)1.0f};
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        psum = __builtin_amdgcn_fdot2(half2_t{pf[2 * i], pf[2 * i + 1]}, one2, psum, false);
                }
                lds_st128(lds_addr(pws) + (uint32_t)(((b * 4 + d) * 64 + lane) * 16), pf);
                if constexpr (kPLo) lds_st128(lds_addr(pws) + 8192u + (uint32_t)(((b * 4 + d) * 64 + lane) * 16), pl);
                l_run = l_run * alpha + psum;
                m_run = m_new;
                if (q == 0) {
                    int ln = lane;   // opaque, as above (q == 0: ln is the head's j)
                    asm volatile("" : "+v"(ln));
                    lds_st32(lds_addr(&alpha_s[b][16 * d]) + 4 * ln, alpha);
                }
                const int moved = __any(alpha != 1.0f) ? 1 : 0;
                if (lane == 0) lds_st32(lds_addr(&rescale_s[b][d]), __int_as_float(moved));
            };
            // QK^T of tile u from its stage: the A operand is the raw codes (lane
            // (j, q): row 16 hh + j, dims 128 ks + 16 q + [0, 16) and 128 ks + 64 +
            // 16 q + [0, 16); its scale operand is the row's exponent of dims
            // 128 ks + 32 q + [0, 32), i.e. of block 2 ks + q / 2), so the codes
            // need no conversion; dims 448..511 of k-step 3 are zeros and the f16
            // tail takes two f16 MFMAs. The wave also writes the f16 scale 2^e of
            // blocks 2d, 2d + 1 of the tile's rows to the stage's scale table, which
            // the consumers' V conversion reads.
            auto qk = [&](int u, float4_t (&acc)[2], auto &&pre) {
                const uint32_t st = lds_addr(stage[u % kFsStages]);
                // tail chunks q and 4 + q of rows j and 16 + j (same swizzle);
                // rebuilt per tile from an opaque lane id so that they are not
                // held through the whole loop
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const uint32_t tpos0 = 16 * fs_tail_pos(ln & 15, ln >> 4);
                const uint32_t tpos1 = tpos0 ^ 64;
                typedef int int8v __attribute__((ext_vector_type(8)));
                const uint4_t z4 = uint4_t{0, 0, 0, 0};
                // one row half at a time: the softmax of the previous tile runs
                // while half 0's reads land; the reads of half 1 go out after the
                // MFMAs of half 0 are issued and land while those run, so only one
                // half's fragments are live
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    uint4_t kc[7];      // dims 64 b + 16 q + [0, 16)
                    uint4_t kt[2];      // f16 tail dims 448 + 32 s + 8 q + [0, 8)
                    uint2_t ke;         // exponents
                    const uint32_t ta = st + kFsTailOff + (16 * hh + j) * kFsTailRow;
                    lds_read_row(st + (16 * hh + j) * kFsCodeRow + 16 * q, ta + tpos0, ta + tpos1,
                                 st + kFsExpOff + (16 * hh + j) * 8, kc, kt, ke);
                    half8_t qtv[2], qtlv[2];
                    if constexpr (kQf32) {
                        const uint32_t qa = lds_addr(&q_tail_s[(d * 4) * 64]) + 16 * ln;
                        asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
                                     "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072"
                                     : "=&v"(qtv[0]), "=&v"(qtv[1]), "=&v"(qtlv[0]), "=&v"(qtlv[1]) : "v"(qa));
                    } else {
                        qtv[0] = qt[0];
                        qtv[1] = qt[1];
                    }
                    if (hh == 0) pre();
                    lds_row_wait(kc, kt, ke);
                    if constexpr (kQf32)   // landed with the wait
                        asm volatile("" : "+v"(qtv[0]), "+v"(qtv[1]), "+v"(qtlv[0]), "+v"(qtlv[1]));
                    if (q < 2 && (d < 3 || q == 0)) {
                        if constexpr (kLean) {
                            const int e = __builtin_amdgcn_sbfe((int)ke[d >> 1], 8 * ((2 * d + q) & 3), 8);
                            const half_t f = __builtin_amdgcn_ldexph((half_t)1.0f, e);
                            const uint32_t ta = st + kFsScaleOff + ((2 * d + q) * kTile + 16 * hh + j) * 2;
                            asm volatile("ds_write_b16 %0, %1" :: "v"(ta), "v"(f) : "memory");
                        } else {
                            const int e = (int)(int8_t)((ke[(2 * d + q) >> 2] >> (8 * ((2 * d + q) & 3))) & 0xFF);
                            const half_t f = (half_t)pow2f(e);
                            const uint32_t ta = st + kFsScaleOff + ((2 * d + q) * kTile + 16 * hh + j) * 2;
                            asm volatile("ds_write_b16 %0, %1" :: "v"(ta), "v"(f) : "memory");
                        }
                    }
                    // kLean: byte ks of scl = E8M0 of block 2 ks + q / 2 (the block the
                    // hardware's K group q of k-step ks falls in), as 2^(e + 1)
                    uint32_t scl = 0;
                    if constexpr (kLean)
                        scl = __builtin_amdgcn_perm(ke[1], ke[0], (q >> 1) ? 0x07050301u : 0x06040200u) ^ 0x80808080u;
                    // two accumulation chains; the third part (fp32 Q) joins chain 0
                    float4_t c2[2] = {float4_t{0, 0, 0, 0}, float4_t{0, 0, 0, 0}};
                    static_for<4>([&](auto ksc) {
                        constexpr int ks = decltype(ksc)::value;
                        const uint32_t ew = ks < 2 ? ke[0] : ke[1];
                        const int sa = kLean ? (int)scl
                                             : __builtin_amdgcn_sbfe((int)ew, 16 * (ks & 1) + 8 * (q >> 1), 8) + 127;
                        uint4_t k_hi = z4;   // dims 448.. of k-step 3 are zeros
                        if constexpr (ks < 3) k_hi = kc[2 * ks + 1];
                        const int8v av = __builtin_bit_cast(int8v, uint4x2_cat(kc[2 * ks], k_hi));
#pragma unroll
                        for (int part = 0; part < kParts; ++part) {
                            // k-step 3's dims 448.. are zeros: its upper 16 bytes are constants
                            const uint8x_t qv = ks < 3 ? qf8v(qf8[ks][part])
                                                       : uint8x_t{qf8[ks][part][0], qf8[ks][part][1],
                                                                  qf8[ks][part][2], qf8[ks][part][3], 0, 0, 0, 0};
                            const int8v bv = __builtin_bit_cast(int8v, qv);
                            c2[part & 1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                av, bv, c2[part & 1], 0, 0, kLean ? ks : 0, sa, ks, qsc[part]);
                        }
                    });
                    c2[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kt[0]), qtv[0],
                                                                   c2[0], 0, 0, 0);
                    c2[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kt[1]), qtv[1],
                                                                   c2[1], 0, 0, 0);
                    if constexpr (kQf32) {
                        c2[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kt[0]), qtlv[0],
                                                                       c2[0], 0, 0, 0);
                        c2[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kt[1]), qtlv[1],
                                                                       c2[1], 0, 0, 0);
                    }
                    acc[hh] = c2[0] + c2[1];
                }
            };

            float4_t sprev[2];
            __builtin_amdgcn_sched_barrier(0);
            qk(0, sprev, [] {});                // interval 0
            lds_barrier();
            for (int u = 1; u < n_tiles; ++u) { // interval u: the softmax of u - 1
                float4_t acc[2];                // first, under the first reads of u
                qk(u, acc, [&] { softmax(u - 1, sprev); });
                sprev[0] = acc[0];
                sprev[1] = acc[1];
                lds_barrier();
            }
            softmax(n_tiles - 1, sprev);        // interval n
            lds_barrier();
            lds_barrier();                      // interval n + 1: P . V(n - 1)
            const float l = xsum_16_32(l_run);
            if (q == 0) {
                int ln = lane;   // opaque: the address is not held through the loop
                asm volatile("" : "+v"(ln));
                float *ml = A.ws_ml + slot * 2 * kH + 16 * d + ln;
                ml[0] = m_run;
                ml[kH] = l;
            }
        };
        // ---- the consumers: the copies (kFsLead tiles ahead) and P . V over their
        // 128 dims for all 64 heads, two intervals behind the producers' QK, with
        // V converted from the FP8 stage
        auto consume = [&](auto tc) {
            constexpr bool kTailQ = decltype(tc)::value;   // dim quarter 3 (64 FP8 + 64 f16 dims)
            const int c = d;
            // copy instruction n = 5 c + k moves chunks 64 n + [0, 64) of the
            // stage: n < 15 code chunks, 15 <= n < 19 tail chunks, n = 19 the
            // exponents (n is wave-uniform, so each copy is one scalar-branched
            // global_load_lds with a 32-bit lane offset from the segment base).
            // The lane's row and byte offset are computed per segment: hoisted to
            // the kernel start they would stay live through the producers' code.
            int c_row[5];
            uint32_t c_off[5];
            int ln = lane;
            asm volatile("" : "+v"(ln));
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const int n = 5 * c + k;
                const int s = 64 * n + ln;
                if (n == 19) {           // exponents: 4 bytes per lane
                    c_row[k] = ln >> 1;
                    c_off[k] = 4 * (ln & 1);
                } else if (n < kFsCodeChunks / 64) {
                    const int cc2 = s % (kFsCodeRow / 16);
                    c_row[k] = s / (kFsCodeRow / 16);
                    c_off[k] = 16 * min(cc2, kNope / 16 - 1);   // the pad chunks re-read chunk 27
                } else {
                    const int s2 = s - kFsCodeChunks;
                    c_row[k] = s2 / (kFsTailRow / 16);
                    c_off[k] = 16 * fs_tail_pos(c_row[k], s2 % (kFsTailRow / 16));
                }
            }
            const uint8_t *codes_s = A.codes + seg_r0 * kNope;
            const uint8_t *tail_s = reinterpret_cast<const uint8_t *>(A.tail) + seg_r0 * (2 * kRot);
            const uint8_t *sexp_s = reinterpret_cast<const uint8_t *>(A.sexp) + seg_r0 * 8;
            // copies of tile u into its stage slot (rows past the segment repeat its
            // last row: every tile issues the same 5 copies per wave, so the vmcnt
            // waits are exact)
            // kLean: a whole tile inside the segment takes its copies from a
            // tile base in SGPRs plus a per-segment lane offset (no per-tile
            // clamp or 64-bit multiply); the segment's last tile clamps as below
            uint32_t c_voff[5];
            if constexpr (kLean) {
#pragma unroll
                for (int k = 0; k < 5; ++k) {
                    const int n = 5 * c + k;
                    const uint32_t rb = n == 19 ? 8u : (n < kFsCodeChunks / 64 ? (uint32_t)kNope : 2u * kRot);
                    c_voff[k] = (uint32_t)c_row[k] * rb + c_off[k];
                }
            }
            // gathered rows: the copies of tile u from physical rows rr (this
            // lane's 5 rows; unmarked, so a row outside the cache reads row 0 and
            // the slot is marked bad), plus the physical rows of tile u + kFsLead
            // into this wave's slot of the stage (32 int64, 4 bytes per lane),
            // clamped inside the phys array (it has kTile rows of padding)
            auto issue_rows = [&](int u, const long long (&rr)[5]) {
                uint8_t *st = stage[u % kFsStages];
#pragma unroll
                for (int k = 0; k < 5; ++k) {
                    const int n = 5 * c + k;
                    if (n == 19)
                        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(A.sexp) + rr[k] * 8 + c_off[k],
                                                         st + kFsExpOff, 4, 0, 0);
                    else if (n < kFsCodeChunks / 64)
                        __builtin_amdgcn_global_load_lds(A.codes + rr[k] * kNope + c_off[k], st + 1024 * n, 16, 0, 0);
                    else
                        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(A.tail) + rr[k] * (2 * kRot) + c_off[k],
                                                         st + 1024 * n, 16, 0, 0);
                }
                if (c == 0) {
                    int ln2 = lane;
                    asm volatile("" : "+v"(ln2));
                    if constexpr (kGather == 1) {
                        const long long gi = min(g0 + (long long)kTile * (u + kFsLead), A.total);
                        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(A.phys + gi) + 4 * ln2,
                                                         st + kFsPhysOff, 4, 0, 0);
                    } else {
                        // 32 int32 entries (lanes 32..63 repeat lanes 0..31), clamped
                        // to the segment's last row: no entry past the problem's list
                        const int e = min(kTile * (u + kFsLead) + (ln2 & 31), seg_last);
                        __builtin_amdgcn_global_load_lds(
                            reinterpret_cast<const uint8_t *>(A.row_idx + (long long)p * A.row_idx_stride + r0 + e),
                            st + kFsPhysOff, 4, 0, 0);
                    }
                }
            };
            const long long seg_base = s_rowbase[p];
            // gathered rows: a row outside the cache seen by this lane (every row
            // of the segment passes through some consumer lane's copies); the
            // slot mark reads it after the producers' last barrier, which comes
            // after every copy issue
            bool cbad = false;
            auto report_bad = [&]() {
                if constexpr (kGather != 0)
                    if (__builtin_expect(__any(cbad), 0) && lane == 0) s_bad[slot_s & 1] = 1;
            };
            auto issue = [&](int u) {
                uint8_t *st = stage[u % kFsStages];
                if constexpr (kGather) {
                    // tile u's rows rode in with tile u - kFsLead (landed: wave 0's wait
                    // for that tile and the barrier after it have passed); rows past
                    // the segment repeat its last row
                    const uint32_t ph = lds_addr(stage[(u - kFsLead) % kFsStages] + kFsPhysOff);
                    long long rr[5];
                    const int last = seg_last - kTile * u;
                    if constexpr (kGather == 1) {
#pragma unroll
                        for (int k = 0; k < 5; ++k) {
                            const int e = max(min(c_row[k], last), 0);
                            asm volatile("ds_read_b64 %0, %1" : "=v"(rr[k]) : "v"(ph + 8 * e));
                        }
                        asm volatile("s_waitcnt lgkmcnt(0)"
                                     : "+v"(rr[0]), "+v"(rr[1]), "+v"(rr[2]), "+v"(rr[3]), "+v"(rr[4]) :: "memory");
#pragma unroll
                        for (int k = 0; k < 5; ++k) {
                            cbad |= rr[k] < 0;
                            rr[k] = unmark_row(rr[k]);
                        }
                    } else {
                        int ix[5];
#pragma unroll
                        for (int k = 0; k < 5; ++k) {
                            const int e = max(min(c_row[k], last), 0);
                            asm volatile("ds_read_b32 %0, %1" : "=v"(ix[k]) : "v"(ph + 4 * e));
                        }
                        asm volatile("s_waitcnt lgkmcnt(0)"
                                     : "+v"(ix[0]), "+v"(ix[1]), "+v"(ix[2]), "+v"(ix[3]), "+v"(ix[4]) :: "memory");
#pragma unroll
                        for (int k = 0; k < 5; ++k) {
                            const long long v = seg_base + ix[k];
                            cbad |= v < 0 || v >= A.n_cache_rows;
                            rr[k] = clamp_row(v, A.n_cache_rows);
                        }
                    }
                    issue_rows(u, rr);
                    return;
                }
                if constexpr (kLean) {
                    if (kTile * u + kTile - 1 <= seg_last) {
                        const uint32_t r0 = (uint32_t)(kTile * u);
#pragma unroll
                        for (int k = 0; k < 5; ++k) {
                            const int n = 5 * c + k;
                            // opaque per use: a 32-bit offset (saddr + voffset form),
                            // not a hoisted 64-bit extension
                            uint32_t vo = c_voff[k];
                            asm volatile("" : "+v"(vo));
                            if (n == 19)
                                __builtin_amdgcn_global_load_lds(sexp_s + r0 * 8 + vo, st + kFsExpOff, 4, 0, 0);
                            else if (n < kFsCodeChunks / 64)
                                __builtin_amdgcn_global_load_lds(codes_s + r0 * kNope + vo, st + 1024 * n, 16, 0, 0);
                            else
                                __builtin_amdgcn_global_load_lds(tail_s + r0 * (2 * kRot) + vo, st + 1024 * n, 16, 0, 0);
                        }
                        return;
                    }
                }
#pragma unroll
                for (int k = 0; k < 5; ++k) {
                    const int n = 5 * c + k;
                    const uint32_t lr = (uint32_t)min(kTile * u + c_row[k], seg_last);
                    if (n == 19)
                        __builtin_amdgcn_global_load_lds(sexp_s + (lr * 8 + c_off[k]), st + kFsExpOff, 4, 0, 0);
                    else if (n < kFsCodeChunks / 64)
                        __builtin_amdgcn_global_load_lds(codes_s + (lr * kNope + c_off[k]), st + 1024 * n, 16, 0, 0);
                    else
                        __builtin_amdgcn_global_load_lds(tail_s + (lr * (2 * kRot) + c_off[k]), st + 1024 * n, 16, 0, 0);
                }
            };
            float4_t o[4][8];   // heads 16 hb + 4 q + r, dims 128 c + 16 nb + j
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 8; ++b) o[a][b] = float4_t{0, 0, 0, 0};
            // K order of the P . V fragments: element i of lane group q is tile
            // row R(q, i) = 16 (i >> 2) + 4 q + (i & 3), the S^T rows the producer
            // lane (j, q) holds. V fragment of dims 16 nb + [0, 16): the FP8 rows
            // through the transposing 8-bit read (lane (m, g) supplies row
            // R(g, m >> 1), bytes 8 (m & 1) + [0, 8)), then code -> f16 times the
            // row's f16 block scale; the f16 tail through two transposing 16-bit
            // reads (lane (m, g) supplies row 4 g + (m >> 2), dims 4 (m & 3) + [0, 4)
            // of the chunk pair 2 nb', 2 nb' + 1 of dims 448 + 16 nb' + [0, 16)).
            // (the row offset is rebuilt per tile from an opaque lane id: held
            // through the loop it is one more long-lived register)
            auto tr8_row_of = [&]() {
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const int jj = ln & 15, qq = ln >> 4;
                return (uint32_t)((16 * ((jj >> 1) >> 2) + 4 * qq + ((jj >> 1) & 3)) * kFsCodeRow +
                                  128 * c + 8 * (jj & 1));
            };
            auto pv = [&](int t) {
                const int b = t & 1;
                const uint32_t st = lds_addr(stage[t % kFsStages]);
                const uint32_t tr8_row = tr8_row_of();
                int lnp = lane;   // opaque, as tr8_row_of
                asm volatile("" : "+v"(lnp));
                const int qp = lnp >> 4;
                half8_t pa[4];
                uint4_t mv;         // the producers' rescale flags of tile t
                uint2_t sc[2][2];   // [block of the quarter][row group]: f16 x 2 scale pairs
                uint2_t tb[8];      // FP8 fragments (nb < 4 or c < 3)
                uint2_t tt[4][2];   // tail fragments (c == 3, nb >= 4)
                asm volatile(
                    "ds_read_b128 %0, %5\n\tds_read_b128 %1, %5 offset:1024\n\t"
                    "ds_read_b128 %2, %5 offset:2048\n\tds_read_b128 %3, %5 offset:3072\n\t"
                    "ds_read_b128 %4, %6"
                    : "=&v"(pa[0]), "=&v"(pa[1]), "=&v"(pa[2]), "=&v"(pa[3]), "=&v"(mv)
                    : "v"(lds_addr(pws) + (uint32_t)((b * 4 * 64 + lnp) * 16)),
                      "v"(lds_addr(&rescale_s[b][0])));
                half8_t pl[4];   // kPLo: the lo halves of P, landed with the first wait below
                if constexpr (kPLo)
                    asm volatile(
                        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
                        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072"
                        : "=&v"(pl[0]), "=&v"(pl[1]), "=&v"(pl[2]), "=&v"(pl[3])
                        : "v"(lds_addr(pws) + 8192u + (uint32_t)((b * 4 * 64 + lnp) * 16)));
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                    if (kTailQ && bb == 1) continue;
                    const uint32_t ta = st + kFsScaleOff + ((2 * c + bb) * kTile + 4 * qp) * 2;
                    asm volatile("ds_read_b64 %0, %2\n\tds_read_b64 %1, %2 offset:32"
                                 : "=&v"(sc[bb][0]), "=&v"(sc[bb][1]) : "v"(ta));
                }
                constexpr int n8 = kTailQ ? 4 : 8;
#pragma unroll
                for (int nb = 0; nb < n8; ++nb)
                    asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2"
                                 : "=&v"(tb[nb]) : "v"(st + tr8_row), "n"(16 * nb));
                if constexpr (kTailQ) {
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb) {
                        int ln = lane;   // opaque: the addresses are not held across tiles
                        asm volatile("" : "+v"(ln));
                        const int r16 = 4 * (ln >> 4) + ((ln & 15) >> 2);
                        const uint32_t a = st + kFsTailOff + r16 * kFsTailRow + 8 * (ln & 1) +
                                           16 * fs_tail_pos(r16, 2 * nb + ((ln & 3) >> 1));
                        asm volatile("ds_read_b64_tr_b16 %0, %2\n\t"
                                     "ds_read_b64_tr_b16 %1, %2 offset:%3"
                                     : "=&v"(tt[nb][0]), "=&v"(tt[nb][1])
                                     : "v"(a), "n"(16 * kFsTailRow));
                    }
                }
                // fragments nb < 4 first: the reads of nb >= 4 (the last 4 FP8
                // reads, or the 8 tail reads) land while their MFMAs run
                asm volatile("s_waitcnt lgkmcnt(%14)"
                             : "+v"(pa[0]), "+v"(pa[1]), "+v"(pa[2]), "+v"(pa[3]), "+v"(mv),
                               "+v"(sc[0][0]), "+v"(sc[0][1]), "+v"(sc[1][0]), "+v"(sc[1][1]),
                               "+v"(tb[0]), "+v"(tb[1]), "+v"(tb[2]), "+v"(tb[3]), "+v"(tt[0][0])
                             : "n"(kTailQ ? 8 : 4) : "memory");
                if constexpr (kPLo)   // issued before the last reads: landed with that wait
                    asm volatile("" : "+v"(pl[0]), "+v"(pl[1]), "+v"(pl[2]), "+v"(pl[3]));
                // rare: a producer moved a reference point; the accumulators of
                // its heads are rescaled by alpha (1 for the other heads)
                if (__builtin_amdgcn_readfirstlane((int)(mv[0] | mv[1] | mv[2] | mv[3]))) {
                    float4_t ar[4];
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
                        ar[hb] = *reinterpret_cast<const float4_t *>(&alpha_s[b][16 * hb + 4 * q]);
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                        for (int nb = 0; nb < 8; ++nb) o[hb][nb] *= ar[hb];
                }
                auto frag = [&](int nb) {
                    if (!kTailQ || nb < 4) {
                        const int bb = nb >> 2;
                        // (whole-vector casts: a bit_cast of one element of these
                        // asm-produced vectors was observed to read element 0)
                        const half4_t sl = __builtin_bit_cast(half4_t, sc[bb][0]);
                        const half4_t sh = __builtin_bit_cast(half4_t, sc[bb][1]);
                        const half2_t s01 = half2_t{sl[0], sl[1]}, s23 = half2_t{sl[2], sl[3]};
                        const half2_t s45 = half2_t{sh[0], sh[1]}, s67 = half2_t{sh[2], sh[3]};
                        return make_half8(cvt_fp8x2<false>(tb[nb][0], 1.0f) * s01,
                                          cvt_fp8x2<true>(tb[nb][0], 1.0f) * s23,
                                          cvt_fp8x2<false>(tb[nb][1], 1.0f) * s45,
                                          cvt_fp8x2<true>(tb[nb][1], 1.0f) * s67);
                    }
                    return __builtin_bit_cast(half8_t, uint4_t{tt[nb - 4][0][0], tt[nb - 4][0][1],
                                                               tt[nb - 4][1][0], tt[nb - 4][1][1]});
                };
                // fragment nb + 1 is converted while the MFMAs of nb run
                half8_t vb = frag(0);
#pragma unroll
                for (int nb = 0; nb < 8; ++nb) {
                    if (nb == 3)
                        asm volatile("s_waitcnt lgkmcnt(0)"
                                     : "+v"(tb[4]), "+v"(tb[5]), "+v"(tb[6]), "+v"(tb[7]), "+v"(tt[0][0]),
                                       "+v"(tt[0][1]), "+v"(tt[1][0]), "+v"(tt[1][1]), "+v"(tt[2][0]),
                                       "+v"(tt[2][1]), "+v"(tt[3][0]), "+v"(tt[3][1])
                                     :: "memory");
                    const half8_t vn = nb < 7 ? frag(nb + 1) : vb;
#pragma unroll
                    for (int hb = 0; hb < 4; ++hb)
                        o[hb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[hb], vb, o[hb][nb], 0, 0, 0);
                    if constexpr (kPLo) {
#pragma unroll
                        for (int hb = 0; hb < 4; ++hb)
                            o[hb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[hb], vb, o[hb][nb], 0, 0, 0);
                    }
                    vb = vn;
                }
            };
            // the tiles after the next kFsLead - 1 have landed (this wave's copies)
            auto wait_ring = [&]() {
                if (kGather && c == 0)
                    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(6 * (kFsLead - 1)) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(5 * (kFsLead - 1)) : "memory");
            };
            // prologue: tiles 0 .. kFsLead - 1; tile 0 lands before the first barrier
            if constexpr (kGather != 0) {
                // their rows straight from the phys array (or the row list), all
                // loaded before any copy
                long long rr[kFsLead][5];
#pragma unroll
                for (int u = 0; u < kFsLead; ++u)
#pragma unroll
                    for (int k = 0; k < 5; ++k) {
                        const int e = min(kTile * u + c_row[k], seg_last);
                        if constexpr (kGather == 1) {
                            const long long v = A.phys[g0 + e];
                            cbad |= v < 0;
                            rr[u][k] = unmark_row(v);
                        } else {
                            const long long v = seg_base + A.row_idx[(long long)p * A.row_idx_stride + r0 + e];
                            cbad |= v < 0 || v >= A.n_cache_rows;
                            rr[u][k] = clamp_row(v, A.n_cache_rows);
                        }
                    }
#pragma unroll
                for (int u = 0; u < kFsLead; ++u) issue_rows(u, rr[u]);
                report_bad();
            } else {
#pragma unroll
                for (int u = 0; u < kFsLead; ++u) issue(u);
            }
            wait_ring();
            lds_barrier();
            // interval u: copies of u + kFsLead, P . V(u - 2); before the barrier
            // that ends it, tile u + 1 has landed (this wave's copies)
            for (int u = 0; u < n_tiles + 2; ++u) {
                issue(u + kFsLead);
                report_bad();
                if (u >= 2) pv(u - 2);
                wait_ring();
                lds_barrier();
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            // the lane offset is rebuilt here: hoisted to the kernel start it would
            // stay live through both loops
            int lo = (4 * q) * kD + j;
            asm volatile("" : "+v"(lo));
            float *wo = A.ws_o + slot * (kH * kD) + 128 * c + lo;
            asm volatile("" : "+v"(wo));
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) wo[(16 * hb + r) * kD + 16 * nb] = o[hb][nb][r];
        };
        if (n_tiles > 0) {
            if (producer) {
                produce();   // its first barrier: stage 0 complete
            } else {
                if (d == 3) consume(std::true_type{});
                else consume(std::false_type{});
            }
        }
        // a segment with no rows (padding of the chunked row space) has no partial;
        // a gathered row outside the cache, met by a consumer's copies, marks the
        // slot (s_bad: written before the tile loop's last barrier)
        if (threadIdx.x == 0) {
            A.ws_prob[slot] = n_tiles > 0 ? (p | ((s_badp[p] | s_bad[slot_s & 1]) ? kBadSlot : 0)) : -1;
            s_bad[slot_s & 1] = 0;
        }
        ++slot_s;
        g0 = seg_end;
        lds_barrier();   // the next segment reuses the stages
    }
    if (threadIdx.x == 0)
        for (int s2 = slot_s; s2 < A.s_max; ++s2) A.ws_prob[(long long)blockIdx.x * A.s_max + s2] = -1;
}

// Physical cache row of every logical row of a gathered step (row_idx and/or
// page table), plus 32 rows of padding that repeat the last row.
__global__ __launch_bounds__(256) void phys_kernel(const DecodeArgs A) {
    __shared__ long long s_start[kMaxProb + 1];
    stage_start(A, s_start);
    const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
    if (g >= A.total + kTile) return;
    const long long gg = g < A.total ? g : A.total - 1;
    int lo = 0, hi = A.n_prob - 1;     // last problem with start <= gg
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_start[mid] <= gg) lo = mid; else hi = mid - 1;
    }
    const long long r = phys_row(A, lo, min(gg - s_start[lo], A.count[lo] - 1));
    A.phys[g] = (r >= 0 && r < A.n_cache_rows) ? r : kBadRow;
}

// One block per (problem, head): combine the partials with the sink. The
// per-slot scalars (problem id, running max, sum) are read with vector loads,
// one slot per thread, so their latencies overlap (a scalar-load loop pays one
// L2 round trip per slot); the slots' scale factors then go through LDS and
// thread t accumulates dims 4t..4t+3 over the slots in slot order, several
// slots' 16-byte loads in flight at once.
__global__ __launch_bounds__(128) void decode_merge_kernel(const DecodeArgs A) {
    __shared__ float s_sc[128], s_dl[128];
    __shared__ float s_mx[2];
    const int p = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const float sink = A.sinks[(long long)p * A.sinks_stride + h] * kLog2e;
    const MergeRope R = merge_rope(A, p, 4 * tid);
    const long long b0 = A.start[p], b1 = b0 + A.count[p];
    long long s0 = 0, n_slot = 0;
    if (b1 > b0) {
        s0 = (b0 / A.chunk) * A.s_max;
        n_slot = ((b1 - 1) / A.chunk) * A.s_max + A.s_max - s0;
    }
    float mx = sink;
    int bad = 0;
    // the first 128 slots' scalars are kept for the second pass (one round
    // trip for them instead of two)
    float m_first = -INFINITY, l_first = 0.0f;
    bool ok_first = false;
    for (long long i = tid; i < n_slot; i += 128) {
        const long long slot = s0 + i;
        const float m = A.ws_ml[slot * 2 * kH + h];
        const float l = A.ws_ml[slot * 2 * kH + kH + h];
        const int pr = A.ws_prob[slot];
        const bool ok = (pr & ~kBadSlot) == p;
        if (ok) {
            mx = fmaxf(mx, m);
            bad |= pr & kBadSlot;
        }
        if (i == tid) {
            m_first = m;
            l_first = l;
            ok_first = ok;
        }
    }
    bad = __syncthreads_or(bad);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) s_mx[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(s_mx[0], s_mx[1]);
    float den = __builtin_amdgcn_exp2f(sink - mx);
    float4_t acc = float4_t{0, 0, 0, 0};
    for (long long base = 0; base < n_slot; base += 128) {
        float sc = 0.0f, dl = 0.0f;
        if (base + tid < n_slot) {
            const long long slot = s0 + base + tid;
            const float m = base == 0 ? m_first : A.ws_ml[slot * 2 * kH + h];
            const float l = base == 0 ? l_first : A.ws_ml[slot * 2 * kH + kH + h];
            const bool ok = base == 0 ? ok_first : (A.ws_prob[slot] & ~kBadSlot) == p;
            if (ok && m != -INFINITY) {
                sc = __builtin_amdgcn_exp2f(m - mx);
                dl = l * sc;
            }
        }
        __syncthreads();   // the previous batch's readers are done
        s_sc[tid] = sc;
        s_dl[tid] = dl;
        __syncthreads();
        const int nb = (int)std::min<long long>(128, n_slot - base);
        const float *o0 = A.ws_o + (s0 + base) * (kH * kD) + h * kD + 4 * tid;
#pragma unroll 16
        for (int j = 0; j < nb; ++j) {
            const float c = s_sc[j];
            const float4_t o = *reinterpret_cast<const float4_t *>(o0 + (long long)j * (kH * kD));
            den += s_dl[j];
            acc = c != 0.0f ? acc + o * c : acc;   // a select: unused slots may hold anything
        }
    }
    // a problem that met a row outside the cache gets NaN, never a plausible value
    const float4_t res = bad ? float4_t{NAN, NAN, NAN, NAN} : acc * (1.0f / den);
    merge_store(A, p, h, 4 * tid, res, R);
}

// The merge for problems of many slots (a long problem split over many
// workgroups): one block per (problem, head, half of the dims) combines the
// partials with the sink. The per-slot scalars (problem id, running max, sum) are read with
// vector loads, one slot per thread, so their latencies overlap; their scale
// factors go through LDS. Each wave then accumulates its own quarter of the
// slots (slot j to wave j mod 4, in slot order), thread t dims 4t..4t+3 of the
// half, several slots' 16-byte loads in flight, and the four waves' sums are
// added in wave order: a fixed order, so the result is deterministic.
constexpr int kMergeThreads = 256;
constexpr long long kMergeWideSlots = 8;   // chunks per problem above which the wide merge runs
__global__ __launch_bounds__(kMergeThreads) void decode_merge_wide_kernel(const DecodeArgs A) {
    __shared__ float s_sc[kMergeThreads];
    __shared__ float s_red[kMergeThreads / 64];
    __shared__ float4_t s_acc[3][64];
    const int p = blockIdx.x;
    const int h = blockIdx.y;
    const int half = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const float sink = A.sinks[(long long)p * A.sinks_stride + h] * kLog2e;
    const MergeRope R = merge_rope(A, p, half * (kD / 2) + 4 * lane);
    const long long b0 = A.start[p], b1 = b0 + A.count[p];
    long long s0 = 0, n_slot = 0;
    if (b1 > b0) {
        s0 = (b0 / A.chunk) * A.s_max;
        n_slot = ((b1 - 1) / A.chunk) * A.s_max + A.s_max - s0;
    }
    auto block_reduce = [&](float v, bool is_max) {
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v, off);
            v = is_max ? fmaxf(v, o) : v + o;
        }
        __syncthreads();   // s_red's previous readers are done
        if (lane == 0) s_red[wave] = v;
        __syncthreads();
        return is_max ? fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]))
                      : (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    };
    float mx = sink;
    int bad = 0;
    // the first kMergeThreads slots' scalars are kept for the second pass
    float m_first = -INFINITY, l_first = 0.0f;
    bool ok_first = false;
    for (long long i = tid; i < n_slot; i += kMergeThreads) {
        const long long slot = s0 + i;
        const float m = A.ws_ml[slot * 2 * kH + h];
        const float l = A.ws_ml[slot * 2 * kH + kH + h];
        const int pr = A.ws_prob[slot];
        const bool ok = (pr & ~kBadSlot) == p;
        if (ok) {
            mx = fmaxf(mx, m);
            bad |= pr & kBadSlot;
        }
        if (i == tid) {
            m_first = m;
            l_first = l;
            ok_first = ok;
        }
    }
    bad = __syncthreads_or(bad);
    mx = block_reduce(mx, true);
    float den_part = 0.0f;
    float4_t acc = float4_t{0, 0, 0, 0};
    const float *o_base = A.ws_o + h * kD + half * (kD / 2) + 4 * lane;
    for (long long base = 0; base < n_slot; base += kMergeThreads) {
        float sc = 0.0f;
        if (base + tid < n_slot) {
            const long long slot = s0 + base + tid;
            const float m = base == 0 ? m_first : A.ws_ml[slot * 2 * kH + h];
            const float l = base == 0 ? l_first : A.ws_ml[slot * 2 * kH + kH + h];
            const bool ok = base == 0 ? ok_first : (A.ws_prob[slot] & ~kBadSlot) == p;
            if (ok && m != -INFINITY) {
                sc = __builtin_amdgcn_exp2f(m - mx);
                den_part += l * sc;
            }
        }
        __syncthreads();   // the previous batch's readers are done
        s_sc[tid] = sc;
        __syncthreads();
        const int nb = (int)min((long long)kMergeThreads, n_slot - base);
        const float *ob = o_base + (s0 + base) * (kH * kD);
#pragma unroll 8
        for (int jj = wave; jj < nb; jj += 4) {
            const float c = s_sc[jj];
            const float4_t o = *reinterpret_cast<const float4_t *>(ob + (long long)jj * (kH * kD));
            acc = c != 0.0f ? acc + o * c : acc;   // a select: unused slots may hold anything
        }
    }
    const float den = block_reduce(den_part, false) + __builtin_amdgcn_exp2f(sink - mx);
    if (wave > 0) s_acc[wave - 1][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        acc = ((acc + s_acc[0][lane]) + s_acc[1][lane]) + s_acc[2][lane];
        // a problem that met a row outside the cache gets NaN, never a plausible value
        const float4_t res = bad ? float4_t{NAN, NAN, NAN, NAN} : acc * (1.0f / den);
        merge_store(A, p, h, half * (kD / 2) + 4 * lane, res, R);
    }
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
    long long start[kMaxProb + 1] = {};   // problem offsets in the chunked row space
};


// Rows of work that one extra problem segment costs a workgroup (its Q
// fragments and first tiles load before any compute, and it writes one
// partial of 128 KB): about five 32-row tiles.
constexpr long long kSegCostRows = 5 * kTile;

// Chunks of whole tiles, at least kMinChunk rows, about wg_per_cu workgroups
// per CU. Two layouts: (a) the problems' rows concatenated and cut evenly (a
// chunk may span problem boundaries: s_max problems per chunk), or (b) every
// problem cut separately, its first chunk aligned (one problem per chunk, a
// few more chunks). (b) wins when chunks are short next to the per-segment
// cost, e.g. a batch of 16 sequences of ~2000 selected rows.
// target_wg: workgroups to aim for (0: wg_per_cu per CU). with_phys: the
// workspace also holds the physical-row array of gathered FP8 steps.
Plan make_plan(const long long *count, int n_prob, int wg_per_cu, long long target_wg = 0,
               bool with_phys = true, int min_chunk = kMinChunk) {
    Plan pl;
    long long total = 0;
    for (int p = 0; p < n_prob; ++p) total += count[p];
    const long long target = target_wg > 0 ? target_wg : (long long)num_cus() * wg_per_cu;
    auto round_tile = [](long long x) { return ((x + kTile - 1) / kTile) * kTile; };
    long long chunk_a = total > 0 ? round_tile((total + target - 1) / target) : kTile;
    if (chunk_a < min_chunk) chunk_a = min_chunk;
    int smax_a = 1;
    {
        long long st = 0;
        const long long n_wg = total > 0 ? (total + chunk_a - 1) / chunk_a : 0;
        std::vector<int> segs((size_t)std::max<long long>(n_wg, 1), 0);
        for (int p = 0; p < n_prob; ++p) {
            if (count[p] > 0)
                for (long long w = st / chunk_a; w <= (st + count[p] - 1) / chunk_a; ++w) ++segs[(size_t)w];
            st += count[p];
        }
        for (int c : segs) smax_a = std::max(smax_a, c);
    }
    long long chunk_b = chunk_a;
    auto wgs_b = [&](long long ch) {
        long long n = 0;
        for (int p = 0; p < n_prob; ++p) n += (count[p] + ch - 1) / ch;
        return n;
    };
    while (wgs_b(chunk_b) > std::max<long long>(target, n_prob)) chunk_b += kTile;
    const bool use_b = smax_a > 1 && chunk_b + kSegCostRows < chunk_a + smax_a * kSegCostRows;
    pl.start[0] = 0;
    if (use_b) {
        pl.chunk = (int)chunk_b;
        for (int p = 0; p < n_prob; ++p)
            pl.start[p + 1] = pl.start[p] + ((count[p] + chunk_b - 1) / chunk_b) * chunk_b;
        pl.s_max = 1;
    } else {
        pl.chunk = (int)chunk_a;
        for (int p = 0; p < n_prob; ++p) pl.start[p + 1] = pl.start[p] + count[p];
        pl.s_max = smax_a;
    }
    const long long space = pl.start[n_prob];
    pl.n_wg = space > 0 ? (int)((space + pl.chunk - 1) / pl.chunk) : 0;
    const size_t slots = (size_t)std::max(pl.n_wg, 1) * pl.s_max;
    pl.ws_bytes = slots * ((size_t)kH * kD * 4 + 2 * kH * 4) + slots * 4 + 256 * 4 +
                  (with_phys ? (size_t)(space + kTile) * sizeof(long long) : 0);
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
    c += align(slots * 4);
    A.phys = reinterpret_cast<long long *>(c);   // used only by gathered steps (reset below)
}

// Kernel for the bf16-Q partials, chosen per call (ds4hip_decode_opts): direct
// rows with one f16 P run the flat-stage kernel (its lean form) unless the
// caller asks for the register-load kernel; row lists, pages and the
// hi + lo P form always run the register-load kernel (the flat kernel's
// producers have no registers left for a second P fragment).
template <int kMode>
void launch_ws(const DecodeArgs &A, const Plan &pl, hipStream_t st, const ds4hip_decode_opts &o) {
    if (kMode < 2 && o.kernel != DS4HIP_DECODE_KERNEL_REGLOAD) {
        if (kMode == 0 && o.exact_p)
            hipLaunchKernelGGL((decode_flat_kernel<true, true>), dim3(pl.n_wg), dim3(512), 0, st, A);
        else if (kMode == 0)
            hipLaunchKernelGGL((decode_flat_kernel<false, true>), dim3(pl.n_wg), dim3(512), 0, st, A);
        else if (o.exact_p)
            hipLaunchKernelGGL((decode_flat_kernel<true, true, false, 1>), dim3(pl.n_wg), dim3(512), 0, st, A);
        else
            hipLaunchKernelGGL((decode_flat_kernel<false, true, false, 1>), dim3(pl.n_wg), dim3(512), 0, st, A);
        return;
    }
    if (o.exact_p)
        hipLaunchKernelGGL((decode_ws_kernel<kMode, true>), dim3(pl.n_wg), dim3(512), 0, st, A);
    else
        hipLaunchKernelGGL((decode_ws_kernel<kMode, false>), dim3(pl.n_wg), dim3(512), 0, st, A);
}

// q_pre: an fp32 Q already converted by q_prep_lane (ds4hip_flash_attn_q_prep_f32)
template <bool kFp8, bool kQf32>
int launch(DecodeArgs &A, const Plan &pl, hipStream_t st, int phases = 3,
           const ds4hip_decode_opts &o = ds4hip_decode_opts{0, 0}, bool q_pre = false) {
    A.chunk = pl.chunk;
    A.s_max = pl.s_max;
    A.kq_log2 = kLog2e / sqrtf((float)kD);
    if ((phases & 1) && pl.n_wg > 0) {
        // position lists without pages: the kernel resolves the rows itself
        // (bf16 Q: decode_ws_kernel<2>; fp32 Q: the flat kernel's list form);
        // the fp32 register kernel needs the phys pass for them
        const bool flat_f32 = kQf32 && o.kernel != DS4HIP_DECODE_KERNEL_REGLOAD;
        const bool idx_only = kFp8 && A.row_idx && !A.page_table && (!kQf32 || flat_f32);
        if (kFp8 && A.phys && !idx_only) {
            const long long n = A.total + kTile;
            hipLaunchKernelGGL(phys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, A);
        }
        if (kFp8 && !kQf32) {
            if (idx_only)
                launch_ws<2>(A, pl, st, o);
            else if (A.phys)
                launch_ws<1>(A, pl, st, o);
            else
                launch_ws<0>(A, pl, st, o);
        }
        else if (kFp8 && o.kernel != DS4HIP_DECODE_KERNEL_REGLOAD) {
            // fp32 Q: the flat-stage kernel with Q in three FP8 parts and, as
            // every fp32-Q decode, P as f16 hi + lo
            if (q_pre && idx_only)
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 2, 2>), dim3(pl.n_wg), dim3(512), 0, st, A);
            else if (q_pre && A.phys)
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 2, 1>), dim3(pl.n_wg), dim3(512), 0, st, A);
            else if (q_pre)
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 2, 0>), dim3(pl.n_wg), dim3(512), 0, st, A);
            else if (idx_only)
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 1, 2>), dim3(pl.n_wg), dim3(512), 0, st, A);
            else if (A.phys)
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 1, 1>), dim3(pl.n_wg), dim3(512), 0, st, A);
            else
                hipLaunchKernelGGL((decode_flat_kernel<true, true, 1, 0>), dim3(pl.n_wg), dim3(512), 0, st, A);
        }
        else if (kFp8)
            hipLaunchKernelGGL(decode_fp8_kernel<kQf32>, dim3(pl.n_wg), dim3(256), 0, st, A);
        else if (A.f32_v_raw)
            hipLaunchKernelGGL(decode_f32_kernel<true>, dim3(pl.n_wg), dim3(256), 0, st, A);
        else
            hipLaunchKernelGGL(decode_f32_kernel<false>, dim3(pl.n_wg), dim3(256), 0, st, A);
        const int e = hip_status(hipGetLastError());
        if (e) return e;
    }
    if (phases & 2)
    {
        // problems of few slots (a long batch of problems, e.g. 43 layers over
        // 256 workgroups) merge with one block per (problem, head); a problem
        // split over many workgroups takes the wide merge, whose four waves
        // per half of the dims keep more slots' loads in flight
        long long max_slots = 0;   // chunks a problem spans
        for (int p = 0; p < A.n_prob; ++p) {
            const long long b0 = A.start[p], b1 = b0 + A.count[p];
            if (b1 > b0)
                max_slots = std::max(max_slots, (b1 - 1) / A.chunk - b0 / A.chunk + 1);
        }
        if (max_slots > kMergeWideSlots)
            hipLaunchKernelGGL(decode_merge_wide_kernel, dim3(A.n_prob, kH, 2), dim3(kMergeThreads), 0, st, A);
        else
            hipLaunchKernelGGL(decode_merge_kernel, dim3(A.n_prob, kH), dim3(128), 0, st, A);
    }
    return hip_status(hipGetLastError());
}

}  // namespace

extern "C" int ds4hip_flash_attn_decode_fp8_workspace_size(const long long *n_rows_per_prob,
                                                           int n_prob, size_t *bytes) {
    if (!bytes || n_prob <= 0 || n_prob > kMaxProb || !n_rows_per_prob) return kEINVAL;
    for (int p = 0; p < n_prob; ++p)
        if (n_rows_per_prob[p] < 0) return kEINVAL;
    // the flat kernel's shorter minimum chunk gives the most slots
    *bytes = make_plan(n_rows_per_prob, n_prob, kFp8WgPerCu, 0, true, kMinChunkFlat).ws_bytes;
    return 0;
}

extern "C" int ds4hip_flash_attn_decode_fp8(
        const void *q, int q_is_f32, long long q_stride, const float *sinks,
        long long sinks_stride, float *out, long long out_stride, const uint8_t *codes,
        const int8_t *sexp, const uint16_t *tail, const long long *n_rows_per_prob,
        int n_prob, const long long *row_base, long long row_base_stride,
        const int32_t *row_idx, long long row_idx_stride, const int32_t *page_table,
        int page_table_stride, int page_rows, int n_head, int head_dim, int n_rot,
        long long n_cache_rows, const ds4hip_decode_opts *opts, void *workspace,
        size_t workspace_bytes, int phases, void *stream) {
    if (phases < 1 || phases > 3 || n_head != kH || head_dim != kD || n_rot != kRot || n_prob <= 0 || n_prob > kMaxProb ||
        !n_rows_per_prob || !q || !sinks || !out || !codes || !sexp || !tail || !workspace || n_cache_rows <= 0)
        return ds4hip_set_last_error(kEINVAL);
    const ds4hip_decode_opts o = opts ? *opts : ds4hip_decode_opts{};
    if ((o.exact_p != 0 && o.exact_p != 1) ||
        (o.kernel != DS4HIP_DECODE_KERNEL_AUTO && o.kernel != DS4HIP_DECODE_KERNEL_REGLOAD) ||
        (o.out_form != DS4HIP_DECODE_OUT_F32 && o.out_form != DS4HIP_DECODE_OUT_ROPE_Q8 &&
         o.out_form != DS4HIP_DECODE_OUT_ROPE_F32) ||
        (o.out_form != DS4HIP_DECODE_OUT_F32 && (o.out_pos < 0 || o.out_il < 0)) ||
        (o.out_form == DS4HIP_DECODE_OUT_ROPE_Q8 &&
         (!o.q8_out || !o.q8_scale || reinterpret_cast<uintptr_t>(o.q8_out) % 4)))
        return ds4hip_set_last_error(kEINVAL);
    // q_is_f32 2: the converted form (only the flat-stage kernel reads it); its
    // problems kQPrepWords apart at least
    if (q_is_f32 < 0 || q_is_f32 > 2 ||
        (q_is_f32 == 2 && (o.kernel == DS4HIP_DECODE_KERNEL_REGLOAD || (n_prob > 1 && q_stride < kQPrepWords) ||
                           q_stride % 4 || reinterpret_cast<uintptr_t>(q) % 16)))
        return ds4hip_set_last_error(kEINVAL);
    int page_shift = 0;
    if (page_table) {
        if (page_rows <= 0 || (page_rows & (page_rows - 1)) || page_table_stride <= 0)
            return ds4hip_set_last_error(kEINVAL);
        while ((1 << page_shift) < page_rows) ++page_shift;
    }
    DecodeArgs A = {};
    for (int p = 0; p < n_prob; ++p) {
        const long long n = n_rows_per_prob[p];
        if (n < 0) return ds4hip_set_last_error(kEINVAL);
        // direct rows: every problem's rows inside the cache (with a device
        // row_base array the kernels check the base; gathered rows are
        // checked one by one on the device)
        if (!row_idx && !page_table &&
            (n > n_cache_rows || (!row_base && (row_base_stride < 0 || (long long)p * row_base_stride + n > n_cache_rows))))
            return ds4hip_set_last_error(kEINVAL);
        A.count[p] = n;
    }
    A.n_cache_rows = n_cache_rows;
    // short problems: the flat kernel takes one-tile chunks (more workgroups,
    // a shorter chain each; the token slice's ~640-row decodes 88.1 -> 86.7
    // us per layer); the register-load kernels keep two-tile chunks
    const bool regload_kernel = o.kernel == DS4HIP_DECODE_KERNEL_REGLOAD ||
                                (!q_is_f32 && row_idx && !page_table);
    const Plan pl = make_plan(n_rows_per_prob, n_prob, kFp8WgPerCu, 0, true,
                              regload_kernel ? kMinChunk : kMinChunkFlat);
    for (int p = 0; p <= n_prob; ++p) A.start[p] = pl.start[p];
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
    if (!row_idx && !page_table) A.phys = nullptr;
    if (o.out_form != DS4HIP_DECODE_OUT_F32) {
        A.out_form = o.out_form == DS4HIP_DECODE_OUT_ROPE_Q8 ? 1 : 2;
        A.rope_pos = o.out_pos;
        A.rope_pos_dev = o.out_pos_dev;
        A.rope = rope_params(kRot, o.out_il, true);
        A.q8_out = o.q8_out;
        A.q8_scale = o.q8_scale;
    }
    const hipStream_t st = (hipStream_t)stream;
    const int rc = q_is_f32 ? launch<true, true>(A, pl, st, phases, o, q_is_f32 == 2)
                            : launch<true, false>(A, pl, st, phases, o);
    return ds4hip_set_last_error(rc);
}

namespace {
// one 256-thread block per problem: producer lane (wave d, lane) of the flat
// kernel converts its fragments of Q
__global__ __launch_bounds__(256) void q_prep_kernel(const float *q, long long q_stride, uint32_t *out,
                                                     long long out_stride) {
    const int d = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t qf8[4][3][8];
    int qsc[3];
    half8_t qt[2], qtl[2];
    q_prep_lane<true, true>(q + (long long)blockIdx.x * q_stride + (long long)(16 * d + (lane & 15)) * kD, lane >> 4,
                            qf8, qsc, qt, qtl);
    q_prep_store(reinterpret_cast<uint4_t *>(out + (long long)blockIdx.x * out_stride), threadIdx.x, qf8, qsc, qt,
                 qtl);
}
}  // namespace

extern "C" int ds4hip_flash_attn_q_prep_f32(const float *q, long long q_stride, int n_prob, void *out,
                                            long long out_stride, void *stream) {
    if (!q || !out || n_prob <= 0 || n_prob > kMaxProb || (n_prob > 1 && (q_stride < kH * kD || out_stride < kQPrepWords)) ||
        (reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) % 16 || q_stride % 4 || out_stride % 4)
        return ds4hip_set_last_error(kEINVAL);
    hipLaunchKernelGGL(q_prep_kernel, dim3(n_prob), dim3(256), 0, (hipStream_t)stream, q, q_stride,
                       static_cast<uint32_t *>(out), out_stride);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" long long ds4hip_flash_attn_q_prep_words(void) { return kQPrepWords; }

// fp32 launchers of the reference (cuda/flash_attn.cuh:73,142). The split-K
// partials live in a workspace: the caller's (the _prealloc forms), or the
// library's per-stream scratch (see stream_scratch).
namespace {
Plan f32_plan(long long n_rows) { return make_plan(&n_rows, 1, 2, 0, false); }

int run_f32(const float *Q, const float *raw, const float *v_raw, int n_raw, const float *comp,
            int n_comp, const int32_t *allowed, const float *sinks, float *out, void *ws,
            size_t ws_bytes, hipStream_t st, const Plan *plan = nullptr) {
    DecodeArgs A = {};
    A.count[0] = (long long)n_raw + n_comp;
    const Plan pl = plan ? *plan : f32_plan(A.count[0]);
    A.start[0] = pl.start[0];
    A.start[1] = pl.start[1];
    if (!ws) {
        // the reference-named launchers take no workspace: the library's
        // per-stream scratch (allocates only when a call outgrows it)
        const int e = stream_scratch(st, pl.ws_bytes, &ws);
        if (e) return e;
    } else if (ws_bytes < pl.ws_bytes) {
        return kEINVAL;
    }
    A.q = Q;
    A.q_stride = 0;
    A.sinks = sinks;
    A.out = out;
    A.f32_raw = raw;
    A.f32_v_raw = (v_raw && v_raw != raw) ? v_raw : nullptr;
    A.f32_comp = comp;
    A.f32_allowed = allowed;
    A.f32_n_raw = n_raw;
    A.n_prob = 1;
    A.total = A.start[1];
    carve(A, ws, pl);
    return launch<false, true>(A, pl, st);
}

bool raw_args_ok(const float *Q, const float *K, const float *V, const float *sinks,
                 const float *out, int n_head, int n_kv, int head_dim) {
    return head_dim == kD && n_head == kH && n_kv >= 0 && Q && sinks && out &&
           (n_kv == 0 || (K && V));
}

bool mixed_args_ok(const float *Q, const float *raw_kv, const float *comp_kv,
                   const float *sinks, const float *out, int n_head, int n_raw, int n_comp,
                   int head_dim) {
    return head_dim == kD && n_head == kH && n_raw >= 0 && n_comp >= 0 && Q && sinks && out &&
           (n_raw == 0 || raw_kv) && (n_comp == 0 || comp_kv);
}
}  // namespace

extern "C" int ds4hip_flash_attn_decode_f32_workspace_size(long long n_rows, size_t *bytes) {
    if (!bytes || n_rows < 0) return kEINVAL;
    *bytes = f32_plan(n_rows).ws_bytes;
    return 0;
}

extern "C" int ds4hip_flash_attn_decode_raw_f32_prealloc(const float *Q, const float *K,
                                                         const float *V, const float *sinks,
                                                         float *out, int n_head, int n_kv,
                                                         int head_dim, void *workspace,
                                                         size_t workspace_bytes, void *stream) {
    if (!raw_args_ok(Q, K, V, sinks, out, n_head, n_kv, head_dim) || !workspace)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(run_f32(Q, K, V, n_kv, nullptr, 0, nullptr, sinks, out,
                                         workspace, workspace_bytes, (hipStream_t)stream));
}

extern "C" int ds4hip_flash_attn_decode_mixed_f32_prealloc(
        const float *Q, const float *raw_kv, const float *comp_kv, const int32_t *comp_allowed,
        const float *sinks, float *out, int n_head, int n_raw, int n_comp, int head_dim,
        void *workspace, size_t workspace_bytes, void *stream) {
    if (!mixed_args_ok(Q, raw_kv, comp_kv, sinks, out, n_head, n_raw, n_comp, head_dim) ||
        !workspace)
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(run_f32(Q, raw_kv, nullptr, n_raw, comp_kv, n_comp,
                                         comp_allowed, sinks, out, workspace, workspace_bytes,
                                         (hipStream_t)stream));
}

extern "C" int ds4hip_flash_attn_decode_raw_f32(const float *Q, const float *K, const float *V,
                                                const float *sinks, float *out, int n_head,
                                                int n_kv, int head_dim, void *stream) {
    // cuda/flash_attn.cu:259-269 drops the launch on a bad shape; the 128-row
    // cap of the reference kernel is lifted. K and V may be the same buffer
    // (MLA layout, cuda/flash_attn.cu:30-33) or two buffers.
    if (!raw_args_ok(Q, K, V, sinks, out, n_head, n_kv, head_dim))
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(run_f32(Q, K, V, n_kv, nullptr, 0, nullptr, sinks, out, nullptr,
                                         0, (hipStream_t)stream));
}

extern "C" int ds4hip_flash_attn_decode_mixed_f32(const float *Q, const float *raw_kv,
                                                  const float *comp_kv,
                                                  const int32_t *comp_allowed,
                                                  const float *sinks, float *out, int n_head,
                                                  int n_raw, int n_comp, int head_dim,
                                                  void *stream) {
    if (!mixed_args_ok(Q, raw_kv, comp_kv, sinks, out, n_head, n_raw, n_comp, head_dim))
        return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(run_f32(Q, raw_kv, nullptr, n_raw, comp_kv, n_comp, comp_allowed,
                                         sinks, out, nullptr, 0, (hipStream_t)stream));
}

// ---- allocation-free fp32 decode (no counterpart in the reference) -------------------
// For callers that cannot allocate (code under graph capture, serving loops):
// the split-K partials live in a file-scope device array instead of a
// workspace. The plan is capped at kNoAllocSlots chunks so that any row count
// fits. Every call on one GPU shares that GPU's copy of the array: calls that
// overlap on one GPU (two streams, two host threads) race. Nothing in it needs
// to start at zero: every partial slot and slot tag is written before the
// merge reads it.
namespace {
constexpr int kNoAllocSlots = 64;
constexpr long long kNoAllocMaxRows = 1ll << 22;
constexpr size_t kNoAllocScratchBytes = 8u << 20 | 512u << 10;   // 8.5 MiB
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch array (looked up once per device, with
// that device current); the array's name is not a device address in host code.
int scratch_ptr(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return kEINVAL;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}
}  // namespace

extern "C" int ds4hip_flash_attn_decode_mixed_f32_noalloc(
        const float *Q, const float *raw_kv, const float *comp_kv, const int32_t *comp_allowed,
        const float *sinks, float *out, int n_head, int n_raw, int n_comp, int head_dim,
        void *stream) {
    if (!mixed_args_ok(Q, raw_kv, comp_kv, sinks, out, n_head, n_raw, n_comp, head_dim) ||
        (long long)n_raw + n_comp > kNoAllocMaxRows)
        return ds4hip_set_last_error(kEINVAL);
    const long long n = (long long)n_raw + n_comp;
    const Plan pl = make_plan(&n, 1, 2, kNoAllocSlots, false);
    if (pl.ws_bytes > kNoAllocScratchBytes) return ds4hip_set_last_error(kEINVAL);
    void *ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc) return ds4hip_set_last_error(rc);
    return ds4hip_set_last_error(run_f32(Q, raw_kv, nullptr, n_raw, comp_kv, n_comp,
                                         comp_allowed, sinks, out, ws, kNoAllocScratchBytes,
                                         (hipStream_t)stream, &pl));
}
