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
// double-buffered f16 LDS tile. Row layout in LDS: eight 64-dim blocks of
// 128 B, each followed by 16 B of padding, plus 16 B per row (1168 B per
// row), so 16 lanes reading the same block column of 16 rows, 8 lanes writing
// the eight blocks of one row, and the transposing reads of 4 rows all fall in
// distinct banks. Inside a tile the keys are taken in the order pi (below):
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
constexpr int kBlkB = 144;           // 128 B of a 64-dim f16 block + 16 B pad
constexpr int kRowB = 8 * kBlkB + 16;
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

// Raw FP8 bytes of one tile held by one thread: row tid/8, 64-dim block
// j = tid%8 (j < 7: 64 codes and the block exponent) and tail granule j.
struct Raw {
    uint4_t c[4];
    uint4_t t;
    int e;
};

__device__ inline void load_raw(const PrefillArgs &A, int tile, int n_all, int tid, Raw &R) {
    const int row = tile * kTile + (tid >> 3), j = tid & 7;
    if (row < n_all) {
        const uint8_t *cp = A.codes + (long long)row * kNope + 64 * j;
        if (j < 7) {
#pragma unroll
            for (int i = 0; i < 4; ++i) R.c[i] = *reinterpret_cast<const uint4_t *>(cp + 16 * i);
            R.e = A.sexp[(long long)row * 8 + j];
        }
        R.t = *reinterpret_cast<const uint4_t *>(A.tail + (long long)row * kRot + 8 * j);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) R.c[i] = uint4_t{0, 0, 0, 0};
        R.t = uint4_t{0, 0, 0, 0};
        R.e = 0;
    }
}

template <bool kHi>
__device__ inline half2_t cvt2(uint32_t w, float scale) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, scale, kHi);
}

// Dequantizes the thread's share of a tile into the f16 LDS tile.
__device__ inline void store_tile(uint8_t *stage, int tid, const Raw &R) {
    const int row = tid >> 3, j = tid & 7;
    uint8_t *rp = stage + row * kRowB;
    if (j < 7) {
        const float sc = __uint_as_float((uint32_t)(R.e + 127) << 23);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 16 codes -> two 8-half chunks
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t w0 = R.c[i][2 * h], w1 = R.c[i][2 * h + 1];
                const half2_t a = cvt2<false>(w0, sc), b = cvt2<true>(w0, sc);
                const half2_t c = cvt2<false>(w1, sc), d = cvt2<true>(w1, sc);
                const half8_t v{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
                *reinterpret_cast<half8_t *>(rp + kBlkB * j + 32 * i + 16 * h) = v;
            }
        }
    }
    *reinterpret_cast<uint4_t *>(rp + kBlkB * 7 + 16 * j) = R.t;
}

// V^T fragments of the wave's 8 dim tiles: vb[dt] holds, for lane (n, g),
// V[pi(4g+r)][128w+16dt+n] then V[pi(16+4g+r)][...], r = 0..3.
__device__ inline void read_vt(uint32_t a0, uint32_t a1, half8_t *vb) {
    uint2_t tb[16];
    asm volatile(
        "ds_read_b64_tr_b16 %0, %16\n\tds_read_b64_tr_b16 %1, %17\n\t"
        "ds_read_b64_tr_b16 %2, %16 offset:32\n\tds_read_b64_tr_b16 %3, %17 offset:32\n\t"
        "ds_read_b64_tr_b16 %4, %16 offset:64\n\tds_read_b64_tr_b16 %5, %17 offset:64\n\t"
        "ds_read_b64_tr_b16 %6, %16 offset:96\n\tds_read_b64_tr_b16 %7, %17 offset:96\n\t"
        "ds_read_b64_tr_b16 %8, %16 offset:144\n\tds_read_b64_tr_b16 %9, %17 offset:144\n\t"
        "ds_read_b64_tr_b16 %10, %16 offset:176\n\tds_read_b64_tr_b16 %11, %17 offset:176\n\t"
        "ds_read_b64_tr_b16 %12, %16 offset:208\n\tds_read_b64_tr_b16 %13, %17 offset:208\n\t"
        "ds_read_b64_tr_b16 %14, %16 offset:240\n\tds_read_b64_tr_b16 %15, %17 offset:240\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(tb[0]), "=&v"(tb[1]), "=&v"(tb[2]), "=&v"(tb[3]), "=&v"(tb[4]), "=&v"(tb[5]),
          "=&v"(tb[6]), "=&v"(tb[7]), "=&v"(tb[8]), "=&v"(tb[9]), "=&v"(tb[10]), "=&v"(tb[11]),
          "=&v"(tb[12]), "=&v"(tb[13]), "=&v"(tb[14]), "=&v"(tb[15])
        : "v"(a0), "v"(a1));
    static_assert(kBlkB == 144, "tr-read offsets assume 144-byte blocks");
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
        vb[dt] = __builtin_bit_cast(
            half8_t, uint4_t{tb[2 * dt][0], tb[2 * dt][1], tb[2 * dt + 1][0], tb[2 * dt + 1][1]});
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
__device__ inline void pv_step(const half8_t (*phi)[64], const half8_t (*plo)[64], int lane,
                               uint32_t a0, uint32_t a1, float4_t (*o)[8]) {
    half8_t vb[8];
    read_vt(a0, a1, vb);
#pragma unroll
    for (int rt8 = 0; rt8 < 8; ++rt8) {
        const half8_t ph = phi[rt8][lane], pl = plo[rt8][lane];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            o[rt8][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb[dt], o[rt8][dt], 0, 0, 0);
            o[rt8][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb[dt], o[rt8][dt], 0, 0, 0);
        }
    }
}

// kFix = false: the fast kernel. The softmax reference max of a row is fixed
// by the first tile; later tiles may exceed it by up to 2^kLazy (P <= 2^15
// stays an f16 number). A row whose max grows further marks its query pair
// in A.fail and the pair's output is left to the fixup launch.
// kFix = true: the fixup kernel. Only flagged pairs run; the reference max
// moves whenever a row max exceeds it by 2^8, with O rescaled.
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
    for (int kt = 0; kt < 2; ++kt) ka[kt] = pi_key(16 * kt + n16) * kRowB + 16 * g;
    uint32_t va[2];           // V^T supplier rows (half h), dims 128w + 4(n16&3)
#pragma unroll
    for (int h = 0; h < 2; ++h)
        va[h] = pi_key(16 * h + 4 * g + (n16 >> 2)) * kRowB + kBlkB * 2 * w + 8 * (n16 & 3);

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
                const int off = kBlkB * (s >> 1) + 64 * (s & 1);
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
                        l_part[rt] += p;
                        const half_t h = (half_t)p;
                        hi[4 * kt + r] = h;
                        lo[4 * kt + r] = (half_t)(p - (float)h);
                    }
                phi[2 * w + rt][lane] = hi;
                plo[2 * w + rt][lane] = lo;
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
            pv_step(phi, plo, lane, lds_addr(st) + va[0], lds_addr(st) + va[1], o);
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
            pv_step(phi, plo, lane, lds_addr(st) + va[0], lds_addr(st) + va[1], o);
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
                                             void *workspace, size_t workspace_bytes,
                                             void *stream) {
    if (n_head != kH || head_dim != kD || n_rot != kRot || n_q < 0 || n_cached < 0 ||
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
    hipLaunchKernelGGL(prefill_fp8_kernel<false>, dim3(n_pairs), dim3(256), 0, st, A);
    hipLaunchKernelGGL(prefill_fp8_kernel<true>, dim3(n_pairs), dim3(256), 0, st, A);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
