// prefill.hip — causal chunked-prefill attention over the FP8 KV cache on
// gfx950 MFMA.
//
// Math (the decode math of cuda/flash_attn.cuh:9-26 applied per query): query
// token t of a chunk sits at absolute position n_cached + t and attends rows
// [0, n_cached + t] of its sequence (the chunk's own rows are already in the
// cache), per head h:
//   out = sum_k exp(s_k - M) V_k / (exp(sink_h - M) + sum_k exp(s_k - M)),
//   s_k = (q_h . K_k) / sqrt(512), K == V (one latent KV head).
//
// Work split. 64 heads share one KV head, so a workgroup takes two queries x
// 64 heads = 128 rows and streams keys once for all of them. Four waves:
//   * QK^T: wave w owns rows [32w, 32w+32) (query w/2, heads 32(w&1)..) and
//     computes S^T[32 keys x 32 rows] over all 512 dims with
//     v_mfma_f32_16x16x32_f16 (A = K from LDS, B = Q^T held in registers);
//   * softmax on its own rows (exp2 domain, lazy rescale: the reference
//     max moves only when a row max exceeds it by 2^8);
//   * P.V: wave w owns dims [128w, 128w+128) of all 128 rows (O: 256 fp32
//     accumulators per lane), A = P from LDS (every wave's P tile is
//     published there), B = V^T read from the same f16 tile with
//     ds_read_b64_tr_b16.
// The FP8 tile (32 rows x 584 B) is loaded into registers one tile ahead,
// dequantized once per workgroup (v_cvt_scalef32_pk_f16_fp8) and written to a
// double-buffered f16 LDS tile of 1056-byte rows whose 16-byte halves of each
// 32-byte column group swap on rows 8..15 of every 16 (row_swz). Inside a tile the keys are taken in the order pi (below):
// the S^T rows of an MFMA, the P fragment and the V^T fragment then agree
// without any register shuffling.

#include "ds4hip_common.h"
#include "../../include/ds4hip.h"


using namespace ds4hip;

namespace {

constexpr int kH = 64;
constexpr int kD = 512;
constexpr int kRot = 64;
constexpr int kNope = kD - kRot;
constexpr int kTile = 32;            // keys per tile
constexpr int kRowB = 2 * kD + 32;   // one f16 row + 32 B

// Byte-offset swizzle of row r of an f16 tile: rows 8..15 of every 16 swap
// the 16-byte halves of their 32-byte column groups. Chosen by measurement:
// 1056-byte rows with this swap ran 2% faster than 1040-byte rows and than
// unswapped 1056-byte rows, though a bank-conflict pattern test shows its
// 16-lane K reads 2-way conflicted and the unswapped form conflict-free.
__device__ inline uint32_t row_swz(int r) {
    return 16u * ((r >> 3) & 1);
}
constexpr int kStageB = kTile * kRowB;
constexpr int kRows = 128;           // query rows (2 queries x 64 heads) per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescale = 8.0f;     // fixup kernel: log2 slack before O is rescaled
constexpr float kLazy = 15.0f;       // fast kernel: largest log2 growth of a row max (P <= 2^15)

struct PrefillArgs {
    const uint16_t *q;   // [n_q][64][512] bf16
    const float *sinks;  // [64]
    float *out;          // [n_q][64][512]
    const uint8_t *codes;
    const int8_t *sexp;
    const uint16_t *tail;
    int *fail;           // [n_pairs] query pairs the fast kernel could not finish
    int n_q;
    int n_cached;
    float kq_log2;
};

// Tile-local key of S^T row / P column `idx` (0..31).
__device__ inline int pi_key(int idx) {
    const int h = idx >> 4, g = (idx >> 2) & 3, k = idx & 3;
    return 16 * h + 8 * (g >> 1) + (g & 1) + 2 * k;
}

__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)p;
}

__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

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

// Raw FP8 bytes of one tile held by one thread: row tid/8 of the tile, code
// bytes [56j, 56j+56) (j = tid%8, seven 8-byte groups, each inside one
// 64-dim block), the row's 8 scale exponents and tail granule j (f16 dims
// 448+8j .. +8). Rows past the end of the sequence repeat its last row, so
// every LDS row stays finite (those keys are masked).
struct Raw {
    uint2_t c[7];
    uint2_t e;
    uint4_t t;
};

__device__ inline void load_raw(const PrefillArgs &A, int tile, int n_all, int tid, Raw &R) {
    int row = tile * kTile + (tid >> 3);
    row = row < n_all ? row : n_all - 1;
    const int j = tid & 7;
    const uint8_t *cp = A.codes + (long long)row * kNope + 56 * j;
#pragma unroll
    for (int i = 0; i < 7; ++i) R.c[i] = *reinterpret_cast<const uint2_t *>(cp + 8 * i);
    R.e = *reinterpret_cast<const uint2_t *>(A.sexp + (long long)row * 8);
    R.t = *reinterpret_cast<const uint4_t *>(A.tail + (long long)row * kRot + 8 * j);
}

template <bool kHi>
__device__ inline half2_t cvt2(uint32_t w, float scale) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, scale, kHi);
}

// Dequantizes the thread's share of a tile into the f16 LDS tile.
__device__ inline void store_tile(uint8_t *stage, int tid, const Raw &R) {
    const int row = tid >> 3, j = tid & 7;
    uint8_t *rp = stage + row * kRowB;
    const uint32_t x = row_swz(row);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const int d = 56 * j + 8 * i;       // first dim of the group
        const int b = d >> 6;                       // its 64-dim block
        const uint32_t ew = b < 4 ? R.e[0] : R.e[1];
        const int e = (int)(int8_t)(ew >> (8 * (b & 3)));
        const float sc = __uint_as_float((uint32_t)(e + 127) << 23);
        const half2_t h0 = cvt2<false>(R.c[i][0], sc), h1 = cvt2<true>(R.c[i][0], sc);
        const half2_t h2 = cvt2<false>(R.c[i][1], sc), h3 = cvt2<true>(R.c[i][1], sc);
        *reinterpret_cast<half8_t *>(rp + ((2 * d) ^ x)) =
            half8_t{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
    }
    *reinterpret_cast<uint4_t *>(rp + ((2 * kNope + 16 * j) ^ x)) = R.t;
}

// V^T fragments of 4 of the wave's dim tiles (DT0 .. DT0+3): vb[i] holds,
// for lane (n, g), V[pi(4g+r)][128w+16(DT0+i)+n] then V[pi(16+4g+r)][...].
template <int DT0>
__device__ inline void read_vt4(uint32_t a0, uint32_t a1, half8_t *vb) {
    constexpr int o0 = 32 * DT0;
    uint2_t tb[8];
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8 offset:%10\n\tds_read_b64_tr_b16 %1, %9 offset:%10\n\t"
        "ds_read_b64_tr_b16 %2, %8 offset:%11\n\tds_read_b64_tr_b16 %3, %9 offset:%11\n\t"
        "ds_read_b64_tr_b16 %4, %8 offset:%12\n\tds_read_b64_tr_b16 %5, %9 offset:%12\n\t"
        "ds_read_b64_tr_b16 %6, %8 offset:%13\n\tds_read_b64_tr_b16 %7, %9 offset:%13\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(tb[0]), "=&v"(tb[1]), "=&v"(tb[2]), "=&v"(tb[3]), "=&v"(tb[4]), "=&v"(tb[5]),
          "=&v"(tb[6]), "=&v"(tb[7])
        : "v"(a0), "v"(a1), "i"(o0), "i"(o0 + 32), "i"(o0 + 64), "i"(o0 + 96));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        vb[i] = __builtin_bit_cast(
            half8_t, uint4_t{tb[2 * i][0], tb[2 * i][1], tb[2 * i + 1][0], tb[2 * i + 1][1]});
}

__device__ inline void load_q(const PrefillArgs &A, int qi, int w, int n16, int g,
                              half8_t (*qf)[16]) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int head = 32 * (w & 1) + 16 * rt + n16;
        const uint16_t *src = A.q + ((long long)qi * kH + head) * kD + 8 * g;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const uint4_t v = *reinterpret_cast<const uint4_t *>(src + 32 * s);
            half8_t h;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[2 * i] = (half_t)bf16_to_f32((uint16_t)(v[i] & 0xFFFF));
                h[2 * i + 1] = (half_t)bf16_to_f32((uint16_t)(v[i] >> 16));
            }
            qf[rt][s] = h;
        }
    }
}

// One P . V step: O[rt8][dt] += P_hi . V + P_lo . V for the 8 row tiles of
// all waves, over this wave's 8 dim tiles (V^T read in two halves of 4).
// The P fragments are read one row tile ahead of their MFMAs, and a
// scheduling barrier closes every row tile so the compiler cannot hoist all
// reads to the front (which would need 64 more VGPRs than exist).
// kPLo: P passed as f16 hi + lo halves (~22 bits, twice the P . V MFMAs);
// otherwise one f16 with l summing the rounded P, so O stays an exactly
// normalized average whose weights are off by at most 2^-11 relative.
// The fixup kernel (prefill_fp8_kernel) always carries hi + lo.
constexpr bool kPrefillPLo = true;

template <bool kPLo>
__device__ inline void pv_step(const half8_t (*phi)[64], const half8_t (*plo)[64], int lane,
                               uint32_t a0, uint32_t a1, float4_t (*o)[8]) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        half8_t vb[4];
        if (half == 0)
            read_vt4<0>(a0, a1, vb);
        else
            read_vt4<4>(a0, a1, vb);
        half8_t ph[2], pl[2];
        ph[0] = phi[0][lane];
        if (kPLo) pl[0] = plo[0][lane];
#pragma unroll
        for (int rt8 = 0; rt8 < 8; ++rt8) {
            if (rt8 < 7) {
                ph[(rt8 + 1) & 1] = phi[rt8 + 1][lane];
                if (kPLo) pl[(rt8 + 1) & 1] = plo[rt8 + 1][lane];
            }
            // hi products of the 4 dim tiles, then lo: dependent MFMAs 4 apart
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[rt8][4 * half + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    ph[rt8 & 1], vb[i], o[rt8][4 * half + i], 0, 0, 0);
            if (kPLo) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[rt8][4 * half + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        pl[rt8 & 1], vb[i], o[rt8][4 * half + i], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Two-barrier form of the prefill. The launcher runs it as kFix = true, the
// fixup kernel: only query pairs flagged by prefill_fast_kernel (a row max that
// outgrew the fixed reference by more than 2^kLazy) run, and the reference max
// moves whenever a row max exceeds it by 2^8, with O rescaled. kFix = false
// (not launched) is the same pass with the fast kernel's fixed reference.
// P is carried as f16 hi + lo (p - hi), so P . V keeps ~22 bits of P.
template <bool kFix>
__global__ __launch_bounds__(256) void prefill_fp8_kernel(const PrefillArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t stages[2][kStageB];
    __shared__ __attribute__((aligned(16))) half8_t phi[8][64];      // [row tile][lane]
    __shared__ __attribute__((aligned(16))) half8_t plo[8][64];
    __shared__ __attribute__((aligned(16))) float alpha_s[kRows];
    __shared__ __attribute__((aligned(16))) int flag_s[4];
    __shared__ __attribute__((aligned(16))) float fin_s[2][kRows];    // m, l per row

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    // heaviest query pairs first
    const int pair = (int)gridDim.x - 1 - (int)blockIdx.x;
    if (kFix && A.fail[pair] == 0) return;
    const int q0 = 2 * pair;
    const int qi = q0 + (w >> 1);                   // this wave's query
    const bool q_ok = qi < A.n_q;
    const int qpos = q_ok ? A.n_cached + qi : -1;   // last key this wave's rows see
    const int n_all = A.n_cached + (q0 + 2 < A.n_q ? q0 + 2 : A.n_q);
    const int n_tiles = (n_all + kTile - 1) / kTile;

    // Q^T fragments: qf[rt][s] = Q[row 16rt+n16][dims 32s+8g .. +8]
    half8_t qf[2][16];
    load_q(A, q_ok ? qi : 0, w, n16, g, qf);

    float4_t o[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) o[a][b] = float4_t{0, 0, 0, 0};
    float m_use[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};
    bool failed = false;

    // lane-constant LDS offsets
    uint32_t ka[2];           // QK A rows (key tile kt), dims 8g
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        const int r = pi_key(16 * kt + n16);
        ka[kt] = r * kRowB + ((16 * g) ^ row_swz(r));
    }
    uint32_t va[2];           // V^T supplier rows (half h), dims 128w + 4(n16&3)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = pi_key(16 * h + 4 * g + (n16 >> 2));
        va[h] = r * kRowB + 256 * w + ((8 * (n16 & 3)) ^ row_swz(r));
    }

    Raw R;
    load_raw(A, 0, n_all, tid, R);
    store_tile(stages[0], tid, R);
    load_raw(A, 1, n_all, tid, R);

    int t = 0;
    while (t < n_tiles) {
        bool slow = false;
        for (; t < n_tiles; ++t) {
            lds_barrier();                                   // X: tile t is in stages[t&1]
            // dequantize tile t+1 (past the end: zero rows, never read) and
            // fetch tile t+2
            store_tile(stages[(t + 1) & 1], tid, R);
            load_raw(A, t + 2, n_all, tid, R);
            const uint8_t *st = stages[t & 1];
            // ---- S^T = K . Q^T ----
            float4_t acc[2][2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) acc[a][b] = float4_t{0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int off = 64 * s;
                const half8_t k0 = *reinterpret_cast<const half8_t *>(st + ka[0] + off);
                const half8_t k1 = *reinterpret_cast<const half8_t *>(st + ka[1] + off);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    acc[0][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qf[rt][s], acc[0][rt], 0, 0, 0);
                    acc[1][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qf[rt][s], acc[1][rt], 0, 0, 0);
                }
            }
            // ---- softmax on rows (rt, n16); lane holds keys pi(16kt+4g+r) ----
            const bool edge = t * kTile + kTile - 1 > qpos;
            bool need = false;
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                float s2[2][4];
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float v = acc[kt][rt][r] * A.kq_log2;
                        if (edge && t * kTile + pi_key(16 * kt + 4 * g + r) > qpos) v = -INFINITY;
                        s2[kt][r] = v;
                        mx = fmaxf(mx, v);
                    }
                mx = xmax_16_32(mx);
                float alpha = 1.0f;
                if (m_use[rt] == -INFINITY) {
                    m_use[rt] = mx;              // first tile: O and l are still zero
                } else if (kFix) {
                    if (mx > m_use[rt] + kRescale) {
                        alpha = __builtin_amdgcn_exp2f(m_use[rt] - mx);
                        m_use[rt] = mx;
                        need = true;
                    }
                } else if (mx > m_use[rt] + kLazy) {
                    failed = true;
                }
                l_part[rt] *= alpha;
                const float m = m_use[rt];
                half8_t hi, lo;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float p = s2[kt][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s2[kt][r] - m);
                        const half_t h = (half_t)p;
                        l_part[rt] += kPrefillPLo ? p : (float)h;
                        hi[4 * kt + r] = h;
                        lo[4 * kt + r] = (half_t)(p - (float)h);
                    }
                phi[2 * w + rt][lane] = hi;
                if (kPrefillPLo) plo[2 * w + rt][lane] = lo;
                if (kFix && g == 0) alpha_s[32 * w + 16 * rt + n16] = alpha;
            }
            if (kFix) {
                const bool wneed = __any(need);
                if (lane == 0) flag_s[w] = wneed ? 1 : 0;
            }
            lds_barrier();                                   // Y: P(t), alpha, flags
            if (kFix) {
                const int4 fl = *reinterpret_cast<const int4 *>(flag_s);
                if (fl.x | fl.y | fl.z | fl.w) {
                    slow = true;
                    break;
                }
            }
            // ---- O += P . V ----
            pv_step<kPrefillPLo>(phi, plo, lane, lds_addr(st) + va[0], lds_addr(st) + va[1], o);
        }
        if (kFix && slow) {
            // a row's reference max moved: finish tile t with O rows rescaled
            // (O passes through VGPRs; Q^T is dropped meanwhile and reloaded)
#pragma unroll
            for (int rt8 = 0; rt8 < 8; ++rt8) {
                const float4_t al = *reinterpret_cast<const float4_t *>(&alpha_s[16 * rt8 + 4 * g]);
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) o[rt8][dt] *= al;
            }
            const uint8_t *st = stages[t & 1];
            pv_step<kPrefillPLo>(phi, plo, lane, lds_addr(st) + va[0], lds_addr(st) + va[1], o);
            load_q(A, q_ok ? qi : 0, w, n16, g, qf);
            ++t;
        }
    }

    // ---- finish: l over the 4 key groups; publish m, l per row ----
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const float l = xsum_16_32(l_part[rt]);
        if (g == 0) {
            fin_s[0][32 * w + 16 * rt + n16] = m_use[rt];
            fin_s[1][32 * w + 16 * rt + n16] = l;
        }
    }
    if (!kFix) {
        const bool wf = __any(failed);
        if (lane == 0) flag_s[w] = wf ? 1 : 0;
    }
    lds_barrier();
    if (!kFix) {
        const int4 fl = *reinterpret_cast<const int4 *>(flag_s);
        if (fl.x | fl.y | fl.z | fl.w) {
            if (tid == 0) A.fail[pair] = 1;
            return;
        }
    }
#pragma unroll
    for (int rt8 = 0; rt8 < 8; ++rt8) {
        const int qq = q0 + (rt8 >> 2);
        if (qq >= A.n_q) continue;
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * rt8 + 4 * g + r;
            const int head = row & 63;
            const float m = fin_s[0][row], l = fin_s[1][row];
            const float sk = A.sinks[head] * kLog2e;
            // the sink joins the denominator relative to the row's reference max
            inv[r] = m == -INFINITY ? 0.0f : 1.0f / (l + __builtin_amdgcn_exp2f(sk - m));
        }
        float *dst = A.out + ((long long)qq * kH + ((16 * rt8) & 63) + 4 * g) * kD + 128 * w + n16;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r * kD + 16 * dt] = o[rt8][dt][r] * inv[r];
    }
}

// QK^T of one tile for the wave's 32 rows: acc[kt][rt] = S^T[keys pi(16kt+4g+r)][row 16rt+n16].
// S^T accumulation with VGPR accumulators (inline asm): O already takes all 256
// AGPRs, and compiler-placed QK^T accumulators in AGPRs made it shuffle O
// between register files every tile. Consecutive MFMAs on one accumulator are
// four apart in the loop below, past the accumulate-forwarding window.
__device__ inline void mfma_vgpr(float4_t &c, const half8_t &a, const half8_t &b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// First k-step: C = 0 inline, so no VALU write of the accumulator precedes it
// (a VALU write feeding an MFMA operand needs wait states the compiler does not
// insert for asm).
__device__ inline void mfma_vgpr0(float4_t &c, const half8_t &a, const half8_t &b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=v"(c) : "v"(a), "v"(b));
}

__device__ inline void qk_tile(const uint8_t *st, const uint32_t *ka, const half8_t (*qf)[16],
                               float4_t (*acc)[2]) {
    half8_t k0[2], k1[2];
    k0[0] = *reinterpret_cast<const half8_t *>(st + ka[0]);
    k1[0] = *reinterpret_cast<const half8_t *>(st + ka[1]);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        if (s < 15) {
            const int off = 64 * (s + 1);
            k0[(s + 1) & 1] = *reinterpret_cast<const half8_t *>(st + ka[0] + off);
            k1[(s + 1) & 1] = *reinterpret_cast<const half8_t *>(st + ka[1] + off);
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            if (s == 0) {
                mfma_vgpr0(acc[0][rt], k0[0], qf[rt][0]);
                mfma_vgpr0(acc[1][rt], k1[0], qf[rt][0]);
            } else {
                mfma_vgpr(acc[0][rt], k0[s & 1], qf[rt][s]);
                mfma_vgpr(acc[1][rt], k1[s & 1], qf[rt][s]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // the results are read by VALU next: 16x16x32 f16 (8 passes) needs 11 wait
    // states after the last write, which the compiler does not track for asm
    asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
}

// Softmax of one tile with the reference max fixed (set on the first tile):
// writes P hi/lo for the wave's two row tiles and accumulates l. A score more
// than 2^kLazy above the reference marks the wave failed.
template <bool kFirst, bool kPLo>
__device__ inline void softmax_fixed(const float4_t (*acc)[2], float kq_log2, int key0, int qpos,
                                     int g, float *m_use, float *l_part, bool &failed,
                                     half8_t *hi_out, half8_t *lo_out) {
    const bool edge = key0 + kTile - 1 > qpos;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        float s2[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = acc[kt][rt][r] * kq_log2;
                s2[kt][r] = (edge && key0 + pi_key(16 * kt + 4 * g + r) > qpos) ? -INFINITY : v;
            }
        if (kFirst) {
            float mx = fmaxf(fmaxf(fmaxf(s2[0][0], s2[0][1]), fmaxf(s2[0][2], s2[0][3])),
                             fmaxf(fmaxf(s2[1][0], s2[1][1]), fmaxf(s2[1][2], s2[1][3])));
            m_use[rt] = xmax_16_32(mx);
        }
        const float m = m_use[rt];
        half8_t hi, lo;
        float lsum = 0.0f;
        bool big = false;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = s2[kt][r] - m;
                big |= x > kLazy;
                const float p = s2[kt][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x);
                const half_t h = (half_t)p;
                lsum += kPLo ? p : (float)h;
                hi[4 * kt + r] = h;
                if (kPLo) lo[4 * kt + r] = (half_t)(p - (float)h);
            }
        l_part[rt] += lsum;
        failed |= big;
        hi_out[rt] = hi;
        lo_out[rt] = lo;
    }
}

// The fast kernel: software-pipelined over tiles with one barrier per tile.
// Iteration t: [barrier] S(t) = K(t) Q^T | dequantize tile t+1 (fetched one
// iteration earlier), fetch tile t+2 | softmax(t) | O += P(t-1) V(t-1). Three f16 stages (t-1 for V, t for K,
// t+1 being written) and two P buffers make every LDS hazard one barrier apart.
template <bool kPLo>
__global__ __launch_bounds__(256) void prefill_fast_kernel(const PrefillArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t stages[3][kStageB];
    __shared__ __attribute__((aligned(16))) half8_t pb[2][2][8][64];   // [buf][hi,lo][row tile][lane]
    __shared__ __attribute__((aligned(16))) int flag_s[4];
    __shared__ __attribute__((aligned(16))) float fin_s[2][kRows];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    const int pair = (int)gridDim.x - 1 - (int)blockIdx.x;
    const int q0 = 2 * pair;
    const int qi = q0 + (w >> 1);
    const bool q_ok = qi < A.n_q;
    const int qpos = q_ok ? A.n_cached + qi : -1;
    const int n_all = A.n_cached + (q0 + 2 < A.n_q ? q0 + 2 : A.n_q);
    const int n_tiles = (n_all + kTile - 1) / kTile;

    half8_t qf[2][16];
    load_q(A, q_ok ? qi : 0, w, n16, g, qf);
    float4_t o[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) o[a][b] = float4_t{0, 0, 0, 0};
    float m_use[2], l_part[2] = {0.f, 0.f};
    bool failed = false;

    uint32_t ka[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        const int r = pi_key(16 * kt + n16);
        ka[kt] = r * kRowB + ((16 * g) ^ row_swz(r));
    }
    uint32_t va[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = pi_key(16 * h + 4 * g + (n16 >> 2));
        va[h] = r * kRowB + 256 * w + ((8 * (n16 & 3)) ^ row_swz(r));
    }

    Raw R;
    load_raw(A, 0, n_all, tid, R);
    store_tile(stages[0], tid, R);
    load_raw(A, 1, n_all, tid, R);
    lds_barrier();
    {
        float4_t acc[2][2];
        qk_tile(stages[0], ka, qf, acc);
        store_tile(stages[1], tid, R);
        load_raw(A, 2, n_all, tid, R);
        half8_t hi[2], lo[2];
        softmax_fixed<true, kPLo>(acc, A.kq_log2, 0, qpos, g, m_use, l_part, failed, hi, lo);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            pb[0][0][2 * w + rt][lane] = hi[rt];
            if (kPLo) pb[0][1][2 * w + rt][lane] = lo[rt];
        }
    }
    int sp = 0, sc = 1, sn = 2;   // stages of tiles t-1, t, t+1
    for (int t = 1; t < n_tiles; ++t) {
        lds_barrier();
        float4_t acc[2][2];
        qk_tile(stages[sc], ka, qf, acc);
        // tile t+1 (fetched one iteration ago) is dequantized; t+2 is fetched
        store_tile(stages[sn], tid, R);
        load_raw(A, t + 2, n_all, tid, R);
        half8_t hi[2], lo[2];
        softmax_fixed<false, kPLo>(acc, A.kq_log2, t * kTile, qpos, g, m_use, l_part, failed, hi, lo);
        const int pbuf = (t - 1) & 1;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            pb[pbuf ^ 1][0][2 * w + rt][lane] = hi[rt];
            if (kPLo) pb[pbuf ^ 1][1][2 * w + rt][lane] = lo[rt];
        }
        pv_step<kPLo>(pb[pbuf][0], pb[pbuf][1], lane, lds_addr(stages[sp]) + va[0],
                lds_addr(stages[sp]) + va[1], o);
        const int tmp = sp;
        sp = sc;
        sc = sn;
        sn = tmp;
    }
    lds_barrier();
    {
        const int pbuf = (n_tiles - 1) & 1;
        pv_step<kPLo>(pb[pbuf][0], pb[pbuf][1], lane, lds_addr(stages[sp]) + va[0],
                lds_addr(stages[sp]) + va[1], o);
    }

    // ---- finish ----
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const float l = xsum_16_32(l_part[rt]);
        if (g == 0) {
            fin_s[0][32 * w + 16 * rt + n16] = m_use[rt];
            fin_s[1][32 * w + 16 * rt + n16] = l;
        }
    }
    const bool wf = __any(failed);
    if (lane == 0) flag_s[w] = wf ? 1 : 0;
    lds_barrier();
    const int4 fl = *reinterpret_cast<const int4 *>(flag_s);
    if (fl.x | fl.y | fl.z | fl.w) {
        if (tid == 0) A.fail[pair] = 1;
        return;
    }
#pragma unroll
    for (int rt8 = 0; rt8 < 8; ++rt8) {
        const int qq = q0 + (rt8 >> 2);
        if (qq >= A.n_q) continue;
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * rt8 + 4 * g + r;
            const float m = fin_s[0][row], l = fin_s[1][row];
            const float sk = A.sinks[row & 63] * kLog2e;
            inv[r] = m == -INFINITY ? 0.0f : 1.0f / (l + __builtin_amdgcn_exp2f(sk - m));
        }
        float *dst = A.out + ((long long)qq * kH + ((16 * rt8) & 63) + 4 * g) * kD + 128 * w + n16;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r * kD + 16 * dt] = o[rt8][dt][r] * inv[r];
    }
}

__global__ void zero_i32_kernel(int *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

extern "C" size_t ds4hip_flash_attn_prefill_fp8_workspace_size(int n_q) {
    return n_q > 0 ? (size_t)((n_q + 1) / 2) * sizeof(int) : 0;
}

extern "C" int ds4hip_flash_attn_prefill_fp8(const void *q, const float *sinks, float *out,
                                             const uint8_t *codes, const int8_t *sexp,
                                             const uint16_t *tail, int n_q, int n_cached,
                                             int n_head, int head_dim, int n_rot,
                                             void *workspace, size_t workspace_bytes, int exact_p,
                                             void *stream) {
    if (n_head != kH || head_dim != kD || n_rot != kRot || n_q < 0 || n_cached < 0 ||
        (exact_p != 0 && exact_p != 1) ||
        (n_q > 0 && (!q || !sinks || !out || !codes || !sexp || !tail || !workspace ||
                     workspace_bytes < ds4hip_flash_attn_prefill_fp8_workspace_size(n_q))))
        return ds4hip_set_last_error(kEINVAL);
    if (n_q == 0) return 0;
    const int n_pairs = (n_q + 1) / 2;
    PrefillArgs A;
    A.q = static_cast<const uint16_t *>(q);
    A.sinks = sinks;
    A.out = out;
    A.codes = codes;
    A.sexp = sexp;
    A.tail = tail;
    A.fail = static_cast<int *>(workspace);
    A.n_q = n_q;
    A.n_cached = n_cached;
    A.kq_log2 = kLog2e / sqrtf((float)kD);
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(zero_i32_kernel, dim3((n_pairs + 255) / 256), dim3(256), 0, st, A.fail,
                       n_pairs);
    if (exact_p)
        hipLaunchKernelGGL(prefill_fast_kernel<true>, dim3(n_pairs), dim3(256), 0, st, A);
    else
        hipLaunchKernelGGL(prefill_fast_kernel<false>, dim3(n_pairs), dim3(256), 0, st, A);
    hipLaunchKernelGGL(prefill_fp8_kernel<true>, dim3(n_pairs), dim3(256), 0, st, A);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
