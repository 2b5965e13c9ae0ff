// compressor.hip — streaming KV compressor, one decode step
// (cuda/compressor.cu:64-429; spec ds4.c compressor_decode_one).
//
// Step kernel: both projections (kv and gate, f16 or fp32 weights) in one
// launch, one wave per output row over the LDS-staged input; the gate row gets
// its APE bias and both rows are written straight into the state row
// (ratio + pos % ratio for ratio 4, pos % ratio otherwise) and into the
// caller's projection scratch.
// Emit kernel (only when (pos + 1) % ratio == 0, decided on the host): one
// workgroup pools the state per column (softmax over 8 or 128 rows),
// RMSNorm-s the pooled row, applies tail RoPE at pos + 1 - ratio, FP8
// round-trips the non-RoPE prefix (attention compressor only), and then —
// after a barrier, since the pool read the state — shifts the ratio-4 ring.

#include "ds4hip_common.h"
#include "step_bodies.h"
#include "../../include/ds4hip.h"

#include <cmath>

using namespace ds4hip;

namespace {

constexpr float kNegInf = -1.0e30f;   // cuda/compressor.cu:53
constexpr float kRmsEps = 1.0e-6f;    // cuda/compressor.cu:54
constexpr int kNRot = 64;             // cuda/compressor.cu:55
constexpr int kMaxIn = kCompMaxIn;

// One wave per output row of the two projections (rows [0, width) of w_kv,
// then [0, width) of w_gate), four per workgroup: eight 16-byte weight chunks
// per lane are in flight before their fmas (wave_rows_dot), which keeps the
// weight stream busy without fewer workgroups than CUs. Then the APE row and
// the state row (cuda/compressor.cu:78-110).
template <bool kW32>
__global__ __launch_bounds__(256) void comp_project_kernel(
        const float *__restrict__ x, const void *__restrict__ w_kv, const void *__restrict__ w_gate,
        const uint16_t *__restrict__ w_ape, int in_dim, int width, int ratio, int pos_mod,
        float *__restrict__ state_kv, float *__restrict__ state_score, float *__restrict__ kv_cur,
        float *__restrict__ sc_cur) {
    __shared__ __attribute__((aligned(16))) float xs[kMaxIn];
    stage_to_lds(xs, x, in_dim);
    __syncthreads();
    comp_project_rows<kW32>(xs, w_kv, w_gate, w_ape, in_dim, width, ratio, pos_mod, state_kv, state_score,
                            kv_cur, sc_cur, blockIdx.x);
}

struct RopeArgs {
    float theta_scale, freq_scale, ext_factor, attn_factor, corr_low, corr_high;
    int pos;
};

// cuda/rope.cu:214-250 (host) for n_rot = 64
RopeArgs rope_args(int il, int pos) {
    const bool compressed = il >= 2;
    RopeArgs R;
    const float base = compressed ? 160000.0f : 10000.0f;
    R.freq_scale = compressed ? 1.0f / 16.0f : 1.0f;
    R.ext_factor = compressed ? 1.0f : 0.0f;
    R.attn_factor = 1.0f;
    if (R.ext_factor != 0.0f) R.attn_factor /= 1.0f + 0.1f * logf(1.0f / R.freq_scale);
    R.corr_low = R.corr_high = 0.0f;
    if (R.ext_factor != 0.0f) {
        const float pi = 3.14159265358979323846f;
        auto corr_dim = [&](float t) {
            return (float)kNRot * logf(65536.0f / (t * 2.0f * pi)) / (2.0f * logf(base));
        };
        R.corr_low = fmaxf(0.0f, floorf(corr_dim(32.0f)));
        R.corr_high = fminf((float)(kNRot - 1), ceilf(corr_dim(1.0f)));
    }
    R.theta_scale = powf(base, -2.0f / (float)kNRot);
    R.pos = pos;
    return R;
}

// One workgroup of 512 threads; thread j owns column j (< head_dim <= 512).
__device__ inline void emit_body(float *__restrict__ state_kv, float *__restrict__ state_score,
                                 const float *__restrict__ w_norm, float *__restrict__ emit_out,
                                 int head_dim, int ratio, int is_attn, RopeArgs R) {
    __shared__ float pooled[512];
    __shared__ float red[8];
    const int j = threadIdx.x;
    const int coff = ratio == 4 ? 2 : 1;
    const int width = coff * head_dim;
    // ---- pool (cuda/compressor.cu:107-164)
    float v = 0.0f;
    if (j < head_dim) {
        float mx = kNegInf;
        if (ratio == 4) {
            for (int r = 0; r < 4; ++r) {
                mx = fmaxf(mx, state_score[(size_t)r * width + j]);
                mx = fmaxf(mx, state_score[(size_t)(4 + r) * width + head_dim + j]);
            }
        } else {
            for (int r = 0; r < ratio; ++r) mx = fmaxf(mx, state_score[(size_t)r * width + j]);
        }
        if (mx > kNegInf * 0.5f) {
            float den = 0.0f, sum = 0.0f;
            if (ratio == 4) {
                for (int r = 0; r < 4; ++r) {
                    const float wp = expf(state_score[(size_t)r * width + j] - mx);
                    const float wc = expf(state_score[(size_t)(4 + r) * width + head_dim + j] - mx);
                    den += wp + wc;
                    sum += wp * state_kv[(size_t)r * width + j];
                    sum += wc * state_kv[(size_t)(4 + r) * width + head_dim + j];
                }
            } else {
                for (int r = 0; r < ratio; ++r) {
                    const float w = expf(state_score[(size_t)r * width + j] - mx);
                    den += w;
                    sum += w * state_kv[(size_t)r * width + j];
                }
            }
            v = den > 0.0f ? sum / den : 0.0f;
        }
    }
    // ---- RMSNorm (cuda/compressor.cu:174-219)
    float ss = v * v;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((j & 63) == 0) red[j >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < 8; ++w) tot += red[w];
    const float scale = 1.0f / sqrtf(tot / (float)head_dim + kRmsEps);
    if (j < head_dim) pooled[j] = v * scale * w_norm[j];
    __syncthreads();
    // ---- tail RoPE at the window start (cuda/compressor.cu:325-331, rope.cu:136-201)
    const int n_nope = head_dim - kNRot;
    float out = j < head_dim ? pooled[j] : 0.0f;
    if (j >= n_nope && j < head_dim) {
        const int p = (j - n_nope) >> 1;   // pair index
        float te = (float)R.pos;
        for (int k = 0; k < p; ++k) te *= R.theta_scale;
        const float ti = R.freq_scale * te;
        float theta = ti, ms = R.attn_factor;
        if (R.ext_factor != 0.0f) {
            const float y = ((float)p - R.corr_low) / fmaxf(0.001f, R.corr_high - R.corr_low);
            const float mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * R.ext_factor;
            theta = ti * (1.0f - mix) + te * mix;
            ms *= 1.0f + 0.1f * logf(1.0f / R.freq_scale);
        }
        const float c = cosf(theta) * ms, s = sinf(theta) * ms;
        const float x0 = pooled[n_nope + 2 * p], x1 = pooled[n_nope + 2 * p + 1];
        out = ((j - n_nope) & 1) ? x0 * s + x1 * c : x0 * c - x1 * s;
    }
    // ---- FP8 round trip of the non-RoPE prefix (attention compressor only)
    if (is_attn && j < n_nope) {
        float a = fabsf(out);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
        const int e = fp8_block_exp(a);
        float q = fminf(fmaxf(ldexpf(out, -e), -448.0f), 448.0f);
        const uint32_t code = e4m3_encode(q);
        const uint32_t mag = code & 0x7Fu;
        float val;
        if (mag < 8) {
            val = (float)mag * 0.001953125f;
        } else {
            const uint32_t bits = ((mag >> 3) + 120u) << 23 | (mag & 7u) << 20;
            val = __uint_as_float(bits);
        }
        out = ldexpf((code & 0x80u) ? -val : val, e);
    }
    if (j < head_dim) emit_out[j] = out;
    // ---- ring shift, ratio 4 (cuda/compressor.cu:230-249); the pool above
    // finished reading the state
    __syncthreads();
    if (ratio == 4) {
        for (int i = j; i < 4 * width; i += 512) {
            const int r = i / width, c = i % width;
            const size_t top = (size_t)(4 + r) * width + c, bot = (size_t)r * width + c;
            const float kv = state_kv[top], sc = state_score[top];
            state_kv[bot] = kv;
            state_score[bot] = sc;
        }
    }
}

__global__ __launch_bounds__(512) void comp_emit_kernel(float *__restrict__ state_kv,
                                                        float *__restrict__ state_score,
                                                        const float *__restrict__ w_norm,
                                                        float *__restrict__ emit_out, int head_dim,
                                                        int ratio, int is_attn, RopeArgs R) {
    emit_body(state_kv, state_score, w_norm, emit_out, head_dim, ratio, is_attn, R);
}

// ---- batched step: n_seq sequences, one position each ----------------------------------

// Y = [kv | gate] projections, [2][n_seq][width]; writes each sequence's
// state row (cuda/compressor.cu:85) with the APE bias on the gate.
// Sums the n_kg k-group partials of both projections in group order (the
// same result on every run), adds the APE row to the gate and writes the
// state row. P: kv partials [n_kg][n_seq][width], then gate partials likewise.
__device__ inline void batch_update_body(const float *__restrict__ P, int n_kg, const uint16_t *__restrict__ w_ape,
                                         const int *__restrict__ pos, int n_seq, int width, int ratio,
                                         float *__restrict__ state_kv, float *__restrict__ state_score,
                                         long long state_stride, int b, int o) {
    const size_t n = (size_t)n_seq * width, j = (size_t)b * width + o;
    float kv = P[j], sc = P[(size_t)n_kg * n + j];
    for (int g = 1; g < n_kg; ++g) {
        kv += P[(size_t)g * n + j];
        sc += P[(size_t)(n_kg + g) * n + j];
    }
    const int pm = pos[b] % ratio;
    const int row = ratio == 4 ? ratio + pm : pm;
    const size_t off = (size_t)b * state_stride + (size_t)row * width + o;
    state_kv[off] = kv;
    state_score[off] = sc + f16_bits_to_f32(w_ape[(size_t)pm * width + o]);
}

__global__ __launch_bounds__(256) void comp_batch_update_kernel(
        const float *__restrict__ P, int n_kg, const uint16_t *__restrict__ w_ape,
        const int *__restrict__ pos, int n_seq, int width, int ratio, float *__restrict__ state_kv,
        float *__restrict__ state_score, long long state_stride) {
    const int o = blockIdx.x * 256 + threadIdx.x;
    if (o >= width) return;
    batch_update_body(P, n_kg, w_ape, pos, n_seq, width, ratio, state_kv, state_score, state_stride, blockIdx.y, o);
}

// The two compressors of a layer: job 0 (attention) on workgroups x <
// blk1, job 1 (indexer) on the rest
struct PairJob {
    const float *P;
    int n_kg, width, head_dim;
    const uint16_t *w_ape;
    const float *w_norm;
    float *state_kv, *state_score, *emit_out;
    long long state_stride;
};
struct PairArgs {
    PairJob j[2];
    int blk1;
};
__global__ __launch_bounds__(256) void comp_pair_update_kernel(const PairArgs A, const int *__restrict__ pos,
                                                               int n_seq, int ratio) {
    const int job = (int)blockIdx.x >= A.blk1 ? 1 : 0;
    const PairJob &J = A.j[job];
    const int o = ((int)blockIdx.x - (job ? A.blk1 : 0)) * 256 + threadIdx.x;
    if (o >= J.width) return;
    batch_update_body(J.P, J.n_kg, J.w_ape, pos, n_seq, J.width, ratio, J.state_kv, J.state_score, J.state_stride,
                      blockIdx.y, o);
}

// One workgroup per sequence; sequences whose position does not close a
// window return at once.
__global__ __launch_bounds__(512) void comp_batch_emit_kernel(
        float *__restrict__ state_kv, float *__restrict__ state_score, long long state_stride,
        const float *__restrict__ w_norm, float *__restrict__ emit_out, int head_dim, int ratio,
        int is_attn, RopeArgs R, const int *__restrict__ pos) {
    const int b = blockIdx.x;
    const int p = pos[b];
    if ((p + 1) % ratio) return;
    R.pos = p + 1 - ratio;
    emit_body(state_kv + (size_t)b * state_stride, state_score + (size_t)b * state_stride, w_norm,
              emit_out + (size_t)b * head_dim, head_dim, ratio, is_attn, R);
}

// workgroup x: sequence x % n_seq of job x / n_seq (job 0 attention, 1 the indexer)
__global__ __launch_bounds__(512) void comp_pair_emit_kernel(const PairArgs A, int n_seq, int ratio, RopeArgs R,
                                                             const int *__restrict__ pos) {
    const int job = (int)blockIdx.x >= n_seq ? 1 : 0;
    const int b = (int)blockIdx.x - job * n_seq;
    const int p = pos[b];
    if ((p + 1) % ratio) return;
    const PairJob &J = A.j[job];
    R.pos = p + 1 - ratio;
    emit_body(J.state_kv + (size_t)b * J.state_stride, J.state_score + (size_t)b * J.state_stride, J.w_norm,
              J.emit_out + (size_t)b * J.head_dim, J.head_dim, ratio, job == 0 ? 1 : 0, R);
}

int comp_step(bool is_attn, const float *x, const void *w_kv, const void *w_gate, bool w32,
              const uint16_t *w_ape, const float *w_norm, int in_dim, int head_dim_out, int ratio,
              int pos, int il, float *state_kv, float *state_score, float *emit_out,
              int *emitted_out_host, float *kv_cur, float *sc_cur, hipStream_t st) {
    if (!x || !w_kv || !w_gate || !w_ape || !w_norm || !state_kv || !state_score || !emit_out ||
        in_dim <= 0 || in_dim > kMaxIn || (in_dim % 8) || head_dim_out <= kNRot ||
        head_dim_out > 512 || (head_dim_out % 64) || (ratio != 4 && ratio != 128) || pos < 0)
        return kEINVAL;
    const int coff = ratio == 4 ? 2 : 1;
    const int width = coff * head_dim_out;
    const int pos_mod = pos % ratio;
    const bool emit = ((pos + 1) % ratio) == 0;
    const dim3 grid((2 * width + 4 * kCpRows - 1) / (4 * kCpRows));
    if (w32)
        hipLaunchKernelGGL(comp_project_kernel<true>, grid, dim3(256), 0, st, x, w_kv, w_gate,
                           w_ape, in_dim, width, ratio, pos_mod, state_kv, state_score, kv_cur, sc_cur);
    else
        hipLaunchKernelGGL(comp_project_kernel<false>, grid, dim3(256), 0, st, x, w_kv, w_gate,
                           w_ape, in_dim, width, ratio, pos_mod, state_kv, state_score, kv_cur, sc_cur);
    int rc = hip_status(hipGetLastError());
    if (emitted_out_host) *emitted_out_host = emit ? 1 : 0;   // cuda/compressor.cu:304
    if (rc || !emit) return rc;
    hipLaunchKernelGGL(comp_emit_kernel, dim3(1), dim3(512), 0, st, state_kv, state_score, w_norm,
                       emit_out, head_dim_out, ratio, is_attn ? 1 : 0,
                       rope_args(il, pos + 1 - ratio));
    return hip_status(hipGetLastError());
}

}  // namespace

extern "C" int ds4hip_compressor_emit_f32(int is_attn, const float *w_norm_f32, int head_dim_out,
                                          int compress_ratio, int pos, int il, float *state_kv, float *state_score,
                                          float *emit_out, void *stream) {
    if (!w_norm_f32 || !state_kv || !state_score || !emit_out || head_dim_out <= kNRot || head_dim_out > 512 ||
        (head_dim_out % 64) || (compress_ratio != 4 && compress_ratio != 128) || pos < 0 ||
        (pos + 1) % compress_ratio)
        return ds4hip_set_last_error(kEINVAL);
    hipLaunchKernelGGL(comp_emit_kernel, dim3(1), dim3(512), 0, (hipStream_t)stream, state_kv, state_score,
                       w_norm_f32, emit_out, head_dim_out, compress_ratio, is_attn ? 1 : 0,
                       rope_args(il, pos + 1 - compress_ratio));
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_compressor_decode_step_f32_prealloc(
        int is_attn, const float *x_f32, const uint16_t *w_kv_f16, const uint16_t *w_gate_f16,
        const uint16_t *w_ape_f16, const float *w_norm_f32, int in_dim, int head_dim_out,
        int compress_ratio, int pos, int il, float *state_kv, float *state_score,
        float *emit_out, int *emitted_out_host, float *scratch_kv_cur, float *scratch_sc_cur,
        void *stream) {
    return ds4hip_set_last_error(comp_step(
        is_attn != 0, x_f32, w_kv_f16, w_gate_f16, false, w_ape_f16, w_norm_f32, in_dim,
        head_dim_out, compress_ratio, pos, il, state_kv, state_score, emit_out, emitted_out_host,
        scratch_kv_cur, scratch_sc_cur, (hipStream_t)stream));
}

extern "C" int ds4hip_compressor_decode_step_f32(int is_attn, const float *x_f32,
                                                 const uint16_t *w_kv_f16,
                                                 const uint16_t *w_gate_f16,
                                                 const uint16_t *w_ape_f16,
                                                 const float *w_norm_f32, int in_dim,
                                                 int head_dim_out, int compress_ratio, int pos,
                                                 int il, float *state_kv, float *state_score,
                                                 float *emit_out, int *emitted_out_host,
                                                 void *stream) {
    // The projection results live only in the state rows; no scratch needed.
    return ds4hip_set_last_error(comp_step(
        is_attn != 0, x_f32, w_kv_f16, w_gate_f16, false, w_ape_f16, w_norm_f32, in_dim,
        head_dim_out, compress_ratio, pos, il, state_kv, state_score, emit_out, emitted_out_host,
        nullptr, nullptr, (hipStream_t)stream));
}

extern "C" int ds4hip_compressor_decode_step_w32(int is_attn, const float *x_f32,
                                                 const float *w_kv_f32, const float *w_gate_f32,
                                                 const uint16_t *w_ape_f16,
                                                 const float *w_norm_f32, int in_dim,
                                                 int head_dim_out, int compress_ratio, int pos,
                                                 int il, float *state_kv, float *state_score,
                                                 float *emit_out, int *emitted_out_host,
                                                 void *stream) {
    return ds4hip_set_last_error(comp_step(
        is_attn != 0, x_f32, w_kv_f32, w_gate_f32, true, w_ape_f16, w_norm_f32, in_dim,
        head_dim_out, compress_ratio, pos, il, state_kv, state_score, emit_out, emitted_out_host,
        nullptr, nullptr, (hipStream_t)stream));
}


extern "C" size_t ds4hip_compressor_batch_scratch_bytes(int n_seq, int in_dim, int head_dim_out,
                                                       int compress_ratio) {
    if (n_seq <= 0 || in_dim <= 0 || head_dim_out <= 0 ||
        (compress_ratio != 4 && compress_ratio != 128))
        return 0;
    const int width = (compress_ratio == 4 ? 2 : 1) * head_dim_out;
    return (size_t)2 * ds4hip_mm_k_groups(width, in_dim, 2) * n_seq * width * sizeof(float);
}

extern "C" int ds4hip_compressor_decode_step_batch_w32(
        int is_attn, int n_seq, const float *x_f32, const float *w_kv_f32,
        const float *w_gate_f32, const uint16_t *w_ape_f16, const float *w_norm_f32, int in_dim,
        int head_dim_out, int compress_ratio, const int *pos_host, const int *pos_dev, int il,
        float *state_kv, float *state_score, long long state_stride, float *emit_out,
        int *emitted_out_host, float *scratch, size_t scratch_bytes, void *stream) {
    const int ratio = compress_ratio;
    if (n_seq <= 0 || n_seq > 16 || !x_f32 || !w_kv_f32 || !w_gate_f32 || !w_ape_f16 ||
        !w_norm_f32 || !pos_host || !pos_dev || !state_kv || !state_score || !emit_out ||
        !scratch || in_dim <= 0 || (in_dim % 32) || head_dim_out <= kNRot || head_dim_out > 512 ||
        (head_dim_out % 64) || (ratio != 4 && ratio != 128))
        return ds4hip_set_last_error(kEINVAL);
    const int coff = ratio == 4 ? 2 : 1;
    const int width = coff * head_dim_out;
    if (state_stride < (long long)coff * ratio * width ||
        scratch_bytes < ds4hip_compressor_batch_scratch_bytes(n_seq, in_dim, head_dim_out, ratio))
        return ds4hip_set_last_error(kEINVAL);
    bool any = false;
    for (int b = 0; b < n_seq; ++b) {
        if (pos_host[b] < 0) return ds4hip_set_last_error(kEINVAL);
        const bool e = ((pos_host[b] + 1) % ratio) == 0;
        if (emitted_out_host) emitted_out_host[b] = e ? 1 : 0;
        any |= e;
    }
    const hipStream_t st = (hipStream_t)stream;
    const int n_kg = ds4hip_mm_k_groups(width, in_dim, 2);
    const int rc = ds4hip_mm_f32_parts(w_kv_f32, x_f32, scratch, width, in_dim, n_seq, st,
                                       w_gate_f32, scratch + (size_t)n_kg * n_seq * width);
    if (rc) return ds4hip_set_last_error(rc);
    hipLaunchKernelGGL(comp_batch_update_kernel, dim3((width + 255) / 256, n_seq), dim3(256), 0,
                       st, scratch, n_kg, w_ape_f16, pos_dev, n_seq, width, ratio, state_kv,
                       state_score, state_stride);
    if (any)
        hipLaunchKernelGGL(comp_batch_emit_kernel, dim3(n_seq), dim3(512), 0, st, state_kv,
                           state_score, state_stride, w_norm_f32, emit_out, head_dim_out, ratio,
                           is_attn ? 1 : 0, rope_args(il, 0), pos_dev);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

namespace {
// scratch floats of one job's two projections' partials
size_t pair_job_floats(int n_seq, int in_dim, int head_dim_out, int ratio) {
    const int width = (ratio == 4 ? 2 : 1) * head_dim_out;
    return (size_t)2 * ds4hip_mm_k_groups(width, in_dim, 2) * n_seq * width;
}
bool pair_job_ok(const ds4hip_compressor_batch_job *j, int ratio) {
    const int coff = ratio == 4 ? 2 : 1;
    return j && j->w_kv_f32 && j->w_gate_f32 && j->w_ape_f16 && j->w_norm_f32 && j->state_kv &&
           j->state_score && j->emit_out && j->head_dim_out > kNRot && j->head_dim_out <= 512 &&
           j->head_dim_out % 64 == 0 && j->state_stride >= (long long)coff * ratio * coff * j->head_dim_out;
}
}  // namespace

extern "C" size_t ds4hip_compressor_pair_batch_scratch_bytes(int n_seq, int in_dim, int attn_head_dim_out,
                                                            int index_head_dim_out, int compress_ratio) {
    if (n_seq <= 0 || in_dim <= 0 || attn_head_dim_out <= 0 || index_head_dim_out <= 0 ||
        (compress_ratio != 4 && compress_ratio != 128))
        return 0;
    return (pair_job_floats(n_seq, in_dim, attn_head_dim_out, compress_ratio) +
            pair_job_floats(n_seq, in_dim, index_head_dim_out, compress_ratio)) *
           sizeof(float);
}

extern "C" int ds4hip_compressor_pair_step_batch_w32(int n_seq, const float *x_f32, int in_dim, int compress_ratio,
                                                     const int *pos_host, const int *pos_dev, int il,
                                                     const ds4hip_compressor_batch_job *attn,
                                                     const ds4hip_compressor_batch_job *index,
                                                     int *emitted_out_host, float *scratch, size_t scratch_bytes,
                                                     void *stream) {
    const int ratio = compress_ratio;
    if (n_seq <= 0 || n_seq > 16 || !x_f32 || !pos_host || !pos_dev || !scratch || in_dim <= 0 || in_dim % 32 ||
        (ratio != 4 && ratio != 128) || !pair_job_ok(attn, ratio) || !pair_job_ok(index, ratio) ||
        scratch_bytes < ds4hip_compressor_pair_batch_scratch_bytes(n_seq, in_dim, attn->head_dim_out,
                                                                   index->head_dim_out, ratio))
        return ds4hip_set_last_error(kEINVAL);
    bool any = false;
    for (int b = 0; b < n_seq; ++b) {
        if (pos_host[b] < 0) return ds4hip_set_last_error(kEINVAL);
        const bool e = ((pos_host[b] + 1) % ratio) == 0;
        if (emitted_out_host) emitted_out_host[b] = e ? 1 : 0;
        any |= e;
    }
    const hipStream_t st = (hipStream_t)stream;
    const int coff = ratio == 4 ? 2 : 1;
    const ds4hip_compressor_batch_job *jobs[2] = {attn, index};
    PairArgs A = {};
    // each job's partials as its own ds4hip_compressor_decode_step_batch_w32
    // call lays them out (its k-slice, kv then gate), so the sums are the same
    const float *W[4];
    float *part[4];
    int rows[4], ks[4];
    float *base = scratch;
    for (int k = 0; k < 2; ++k) {
        const int width = coff * jobs[k]->head_dim_out;
        const int n_kg = ds4hip_mm_k_groups(width, in_dim, 2);
        PairJob &J = A.j[k];
        J.P = base;
        J.n_kg = n_kg;
        J.width = width;
        J.head_dim = jobs[k]->head_dim_out;
        J.w_ape = jobs[k]->w_ape_f16;
        J.w_norm = jobs[k]->w_norm_f32;
        J.state_kv = jobs[k]->state_kv;
        J.state_score = jobs[k]->state_score;
        J.emit_out = jobs[k]->emit_out;
        J.state_stride = jobs[k]->state_stride;
        W[2 * k] = jobs[k]->w_kv_f32;
        W[2 * k + 1] = jobs[k]->w_gate_f32;
        part[2 * k] = base;
        part[2 * k + 1] = base + (size_t)n_kg * n_seq * width;
        rows[2 * k] = rows[2 * k + 1] = width;
        ks[2 * k] = ks[2 * k + 1] = ds4hip_mm_kslice(width, in_dim, 2);
        base += (size_t)2 * n_kg * n_seq * width;
    }
    int rc = ds4hip_mm_f32_parts_mats(W, part, rows, ks, 4, x_f32, in_dim, n_seq, st);
    if (rc) return ds4hip_set_last_error(rc);
    A.blk1 = (A.j[0].width + 255) / 256;
    hipLaunchKernelGGL(comp_pair_update_kernel, dim3(A.blk1 + (A.j[1].width + 255) / 256, n_seq), dim3(256), 0, st,
                       A, pos_dev, n_seq, ratio);
    if (any)
        hipLaunchKernelGGL(comp_pair_emit_kernel, dim3(2 * n_seq), dim3(512), 0, st, A, n_seq, ratio,
                           rope_args(il, 0), pos_dev);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
