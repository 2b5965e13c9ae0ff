// misc.cpp — oracle: tail RoPE YaRN, matvecs (f16, Q8_0, bf16) and the
// streaming KV compressor decode step.
// TEST INFRASTRUCTURE ONLY (see ds4_oracle.h).

#include "ds4_oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

// YaRN constants (cuda/rope.cu:114-119).
constexpr float kFreqBase = 10000.0f;
constexpr float kScaleFactor = 16.0f;
constexpr float kBetaFast = 32.0f;
constexpr float kBetaSlow = 1.0f;
constexpr float kCompressFreqBase = 160000.0f;
constexpr int kOrigCtx = 65536;

// cuda/rope.cu:123-126
int compress_ratio(int il) { return il < 2 ? 0 : ((il & 1) == 0 ? 4 : 128); }

// cuda/rope.cu:130-133
float yarn_ramp(float low, float high, int i0) {
    const float y = ((float)(i0 / 2) - low) / std::fmax(0.001f, high - low);
    return 1.0f - std::fmin(1.0f, std::fmax(0.0f, y));
}

float f16v(uint16_t h) { return orc_f16_to_f32(h); }

}  // namespace

// cuda/rope.cu:136-259 (forward) and cuda/attn_out.cu:54-107,207-251
// (inverse: the sin term negated).
extern "C" void orc_rope_tail(const float *x_in, float *x_out, int n_heads, int head_dim,
                              int n_rot, int pos, int il, int inverse) {
    const bool compressed = compress_ratio(il) != 0;
    const float freq_base = compressed ? kCompressFreqBase : kFreqBase;
    const float freq_scale = compressed ? 1.0f / kScaleFactor : 1.0f;
    const float ext_factor = compressed ? 1.0f : 0.0f;
    float attn_factor = 1.0f;
    if (ext_factor != 0.0f) attn_factor /= 1.0f + 0.1f * std::log(1.0f / freq_scale);
    float corr_low = 0.0f, corr_high = 0.0f;
    if (ext_factor != 0.0f) {
        const float pi = 3.14159265358979323846f;
        auto corr_dim = [&](float target) {
            return (float)n_rot * std::log((float)kOrigCtx / (target * 2.0f * pi)) /
                   (2.0f * std::log(freq_base));
        };
        corr_low = std::fmax(0.0f, std::floor(corr_dim(kBetaFast)));
        corr_high = std::fmin((float)(n_rot - 1), std::ceil(corr_dim(kBetaSlow)));
    }
    const int n_nope = head_dim - n_rot;
    const float theta_scale = std::pow(freq_base, -2.0f / (float)n_rot);
    for (int h = 0; h < n_heads; ++h) {
        const float *xi = x_in + (size_t)h * head_dim;
        float *xo = x_out + (size_t)h * head_dim;
        std::vector<float> tailv(xi + n_nope, xi + head_dim);
        if (xo != xi) std::memcpy(xo, xi, sizeof(float) * (size_t)n_nope);
        float theta_extrap = (float)pos;
        for (int p = 0; p < n_rot / 2; ++p) {
            if (p > 0) theta_extrap *= theta_scale;       // running product (rope.cu:172-177)
            const int i = 2 * p;
            const float theta_interp = freq_scale * theta_extrap;
            float theta = theta_interp;
            float mscale = attn_factor;
            if (ext_factor != 0.0f) {
                const float ramp_mix = yarn_ramp(corr_low, corr_high, i) * ext_factor;
                theta = theta_interp * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
                mscale *= 1.0f + 0.1f * std::log(1.0f / freq_scale);
            }
            const float c = std::cos(theta) * mscale;
            const float s = (inverse ? -1.0f : 1.0f) * std::sin(theta) * mscale;
            const float x0 = tailv[i], x1 = tailv[i + 1];
            xo[n_nope + i] = x0 * c - x1 * s;
            xo[n_nope + i + 1] = x0 * s + x1 * c;
        }
    }
}

// cuda/router.cu:69-97
extern "C" void orc_mul_mv_f16_f32(const uint16_t *w, const float *x, float *y, int out_dim,
                                   int in_dim) {
    for (int o = 0; o < out_dim; ++o) {
        double acc = 0.0;
        for (int i = 0; i < in_dim; ++i) acc += (double)f16v(w[(size_t)o * in_dim + i]) * x[i];
        y[o] = (float)acc;
    }
}

// cuda/attn_out.cu:119-145 / cuda/dense_q8.cu quantize: per 32 elements,
// d = amax/127, id = 1/d, q = clamp(rint(x*id), -128, 127), scale kept fp32.
extern "C" void orc_q8_quantize_act(const float *x, int n, int8_t *xq, float *xscale) {
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[b * 32 + i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < 32; ++i) {
            long v = std::lrint(x[b * 32 + i] * id);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            xq[b * 32 + i] = (int8_t)v;
        }
        xscale[b] = d;
    }
}

namespace {
// One Q8_0 row dot: sum_b f16(d_w) * xscale[b] * (int32 dot), fp64 accumulate
// of the per-block terms (each per-block term itself rounded to fp32 as the
// reference's fma operands are fp32 products).
float q8_row_dot(const uint8_t *row, const int8_t *xq, const float *xscale, int n_blocks) {
    double acc = 0.0;
    for (int b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = row + (size_t)b * 34;
        uint16_t dbits;
        std::memcpy(&dbits, blk, 2);
        const int8_t *qs = reinterpret_cast<const int8_t *>(blk + 2);
        int32_t s = 0;
        for (int i = 0; i < 32; ++i) s += (int32_t)qs[i] * (int32_t)xq[b * 32 + i];
        const float dd = f16v(dbits) * xscale[b];
        acc += (double)dd * (double)s;
    }
    return (float)acc;
}
}  // namespace

// cuda/attn_out.cu:159-197 + :255-291
extern "C" void orc_q8_grouped_matvec(const uint8_t *W, const float *x, float *y,
                                      int n_groups, int group_dim, int rank) {
    const int bpg = group_dim / 32;
    std::vector<int8_t> xq((size_t)n_groups * group_dim);
    std::vector<float> xs((size_t)n_groups * bpg);
    orc_q8_quantize_act(x, n_groups * group_dim, xq.data(), xs.data());
    for (int r = 0; r < n_groups * rank; ++r) {
        const int g = r / rank;
        y[r] = q8_row_dot(W + (size_t)r * bpg * 34, xq.data() + (size_t)g * group_dim,
                          xs.data() + (size_t)g * bpg, bpg);
    }
}

extern "C" void orc_q8_matvec(const uint8_t *W, const float *x, float *y, int n_rows, int n_cols) {
    const int bpr = n_cols / 32;
    std::vector<int8_t> xq((size_t)n_cols);
    std::vector<float> xs((size_t)bpr);
    orc_q8_quantize_act(x, n_cols, xq.data(), xs.data());
    for (int r = 0; r < n_rows; ++r) y[r] = q8_row_dot(W + (size_t)r * bpr * 34, xq.data(), xs.data(), bpr);
}

extern "C" void orc_bf16_matvec(const uint16_t *W, const float *x, float *y, int n_rows, int n_cols) {
    for (int r = 0; r < n_rows; ++r) {
        double acc = 0.0;
        for (int c = 0; c < n_cols; ++c)
            acc += (double)orc_bf16_to_f32(W[(size_t)r * n_cols + c]) * x[c];
        y[r] = (float)acc;
    }
}

// cuda/compressor.cu:64-349 (launch_compressor_decode_step_f32).
// The step after the two projections (kv, sc: the W x products).
static int compressor_after_projection(int is_attn, const float *kv_in, const float *sc_in,
                                       const uint16_t *w_ape, const float *w_norm,
                                       int head_dim_out, int ratio, int pos, int il,
                                       float *state_kv, float *state_score, float *emit_out);

extern "C" int orc_compressor_step(int is_attn, const float *x, const uint16_t *w_kv,
                                   const uint16_t *w_gate, const uint16_t *w_ape,
                                   const float *w_norm, int in_dim, int head_dim_out,
                                   int ratio, int pos, int il, float *state_kv,
                                   float *state_score, float *emit_out) {
    const int width = (ratio == 4 ? 2 : 1) * head_dim_out;
    std::vector<float> kv((size_t)width), sc((size_t)width);
    orc_mul_mv_f16_f32(w_kv, x, kv.data(), width, in_dim);
    orc_mul_mv_f16_f32(w_gate, x, sc.data(), width, in_dim);
    return compressor_after_projection(is_attn, kv.data(), sc.data(), w_ape, w_norm,
                                       head_dim_out, ratio, pos, il, state_kv, state_score,
                                       emit_out);
}

// The same step with fp32 projection weights (fp64 accumulation).
extern "C" int orc_compressor_step_w32(int is_attn, const float *x, const float *w_kv,
                                       const float *w_gate, const uint16_t *w_ape,
                                       const float *w_norm, int in_dim, int head_dim_out,
                                       int ratio, int pos, int il, float *state_kv,
                                       float *state_score, float *emit_out) {
    const int width = (ratio == 4 ? 2 : 1) * head_dim_out;
    std::vector<float> kv((size_t)width), sc((size_t)width);
    for (int o = 0; o < width; ++o) {
        double a = 0.0, b = 0.0;
        for (int i = 0; i < in_dim; ++i) {
            a += (double)w_kv[(size_t)o * in_dim + i] * x[i];
            b += (double)w_gate[(size_t)o * in_dim + i] * x[i];
        }
        kv[o] = (float)a;
        sc[o] = (float)b;
    }
    return compressor_after_projection(is_attn, kv.data(), sc.data(), w_ape, w_norm,
                                       head_dim_out, ratio, pos, il, state_kv, state_score,
                                       emit_out);
}

static int compressor_after_projection(int is_attn, const float *kv, const float *sc,
                                       const uint16_t *w_ape, const float *w_norm,
                                       int head_dim_out, int ratio, int pos, int il,
                                       float *state_kv, float *state_score, float *emit_out) {
    const int coff = ratio == 4 ? 2 : 1;
    const int width = coff * head_dim_out;
    const int pos_mod = pos % ratio;
    const bool emit = ((pos + 1) % ratio) == 0;
    // compressor.cu:64-90: APE add and state-row write.
    const int row = ratio == 4 ? ratio + pos_mod : pos_mod;
    for (int j = 0; j < width; ++j) {
        const float s = sc[j] + f16v(w_ape[(size_t)pos_mod * width + j]);
        state_kv[(size_t)row * width + j] = kv[j];
        state_score[(size_t)row * width + j] = s;
    }
    if (!emit) return 0;
    // compressor.cu:107-164: softmax pool per column.
    const float kNegInf = -1.0e30f;
    for (int j = 0; j < head_dim_out; ++j) {
        float mx = kNegInf;
        if (ratio == 4) {
            for (int r = 0; r < 4; ++r) {
                mx = std::fmax(mx, state_score[(size_t)r * width + j]);
                mx = std::fmax(mx, state_score[(size_t)(4 + r) * width + head_dim_out + j]);
            }
        } else {
            for (int r = 0; r < ratio; ++r) mx = std::fmax(mx, state_score[(size_t)r * width + j]);
        }
        if (mx <= kNegInf * 0.5f) { emit_out[j] = 0.0f; continue; }
        float denom = 0.0f, sum = 0.0f;
        if (ratio == 4) {
            for (int r = 0; r < 4; ++r) {
                const float sp = state_score[(size_t)r * width + j];
                const float scv = state_score[(size_t)(4 + r) * width + head_dim_out + j];
                const float wp = std::exp(sp - mx), wc = std::exp(scv - mx);
                denom += wp + wc;
                sum += wp * state_kv[(size_t)r * width + j];
                sum += wc * state_kv[(size_t)(4 + r) * width + head_dim_out + j];
            }
        } else {
            for (int r = 0; r < ratio; ++r) {
                const float w = std::exp(state_score[(size_t)r * width + j] - mx);
                denom += w;
                sum += w * state_kv[(size_t)r * width + j];
            }
        }
        emit_out[j] = denom > 0.0f ? sum / denom : 0.0f;
    }
    // compressor.cu:174-219: RMSNorm (fp64 sum of squares, the ds4 CPU form).
    double ss = 0.0;
    for (int j = 0; j < head_dim_out; ++j) ss += (double)emit_out[j] * emit_out[j];
    const float scale = 1.0f / std::sqrt((float)(ss / head_dim_out) + 1.0e-6f);
    for (int j = 0; j < head_dim_out; ++j) emit_out[j] = emit_out[j] * scale * w_norm[j];
    // compressor.cu:325-331: tail RoPE at the first position of the window.
    orc_rope_tail(emit_out, emit_out, 1, head_dim_out, 64, pos + 1 - ratio, il, 0);
    // compressor.cu:334-339: FP8 round trip on the attention path.
    if (is_attn) {
        std::vector<float> tmp(emit_out, emit_out + head_dim_out);
        orc_fp8_quant_row(tmp.data(), head_dim_out, 64, nullptr, nullptr, nullptr, emit_out);
    }
    // compressor.cu:230-249: ring shift for ratio 4.
    if (ratio == 4) {
        for (int r = 0; r < 4; ++r)
            for (int j = 0; j < width; ++j) {
                const size_t top = (size_t)(4 + r) * width + j, bot = (size_t)r * width + j;
                state_kv[bot] = state_kv[top];
                state_score[bot] = state_score[top];
            }
    }
    return 1;
}

// ---- RMSNorm (cuda/norm.cu:4-7, the ds4.c rms_norm_weight spec the device
// kernels are checked against): ss in fp64, scale = 1 / sqrtf((float)(ss / n)
// + eps), y = x * scale * w (w NULL: unit gain).
extern "C" void orc_rms_norm_f32(const float *x, const float *w, float *y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float scale = 1.0f / std::sqrt((float)(ss / (double)n) + eps);
    for (int i = 0; i < n; ++i) y[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

// Per-row form (cuda/norm.cuh:26-45): weight_dim 0 = unit gain, n_per_row =
// one weight row shared by all rows, n_rows * n_per_row = a weight row each.
extern "C" void orc_rms_norm_batch_f32(const float *x, const float *w, int weight_dim, float *y,
                                       int n_rows, int n_per_row, float eps) {
    for (int r = 0; r < n_rows; ++r) {
        const float *wr = weight_dim == 0 ? nullptr
                          : weight_dim == n_per_row ? w : w + (size_t)r * n_per_row;
        orc_rms_norm_f32(x + (size_t)r * n_per_row, wr, y + (size_t)r * n_per_row, n_per_row, eps);
    }
}
