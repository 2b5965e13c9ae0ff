// attn.cpp — oracle: single-query decode attention with attention sinks, and
// a causal chunked-prefill restatement of the same per-query math.
// TEST INFRASTRUCTURE ONLY (see ds4_oracle.h).

#include "ds4_oracle.h"

#include <cmath>
#include <thread>
#include <vector>

namespace {

// One head of cuda/flash_attn.cuh:96-117: max seeded with the sink, masked
// rows (nullptr row) skipped, denominator seeded with exp(sink - max).
// K rows are supplied already f16-rounded (the reference rounds on read,
// cuda/flash_attn.cu:185,223).
void head_attention(const float *qh, const float *const *krows, int n,
                    float sink, float kq_scale, int head_dim,
                    std::vector<float> &scores, float *oh,
                    const float *const *vrows = nullptr) {
    if (!vrows) vrows = krows;
    scores.resize((size_t)n);
    float mx = sink;
    for (int k = 0; k < n; ++k) {
        if (!krows[k]) { scores[k] = -INFINITY; continue; }
        float dot = 0.0f;
        for (int d = 0; d < head_dim; ++d) dot += qh[d] * krows[k][d];
        const float s = dot * kq_scale;
        scores[k] = s;
        if (s > mx) mx = s;
    }
    float denom = std::exp(sink - mx);
    for (int d = 0; d < head_dim; ++d) oh[d] = 0.0f;
    for (int k = 0; k < n; ++k) {
        if (!krows[k]) continue;
        const float w = std::exp(scores[k] - mx);
        denom += w;
        for (int d = 0; d < head_dim; ++d) oh[d] += w * vrows[k][d];
    }
    const float inv = 1.0f / denom;
    for (int d = 0; d < head_dim; ++d) oh[d] *= inv;
}

void run_heads(const float *Q, const float *const *krows, int n, const float *sinks,
               float *out, int n_head, int head_dim, int n_threads) {
    const float kq_scale = 1.0f / std::sqrt((float)head_dim);
    if (n_threads <= 1) {
        std::vector<float> scores;
        for (int h = 0; h < n_head; ++h)
            head_attention(Q + (size_t)h * head_dim, krows, n, sinks[h], kq_scale,
                           head_dim, scores, out + (size_t)h * head_dim);
        return;
    }
    std::vector<std::thread> pool;
    for (int t = 0; t < n_threads; ++t) {
        pool.emplace_back([=]() {
            std::vector<float> scores;
            for (int h = t; h < n_head; h += n_threads)
                head_attention(Q + (size_t)h * head_dim, krows, n, sinks[h], kq_scale,
                               head_dim, scores, out + (size_t)h * head_dim);
        });
    }
    for (auto &th : pool) th.join();
}

// f16-rounded fp32 copy of FP8-cache rows (fp8_kv.cu:179 dequant, then the
// f16 round-trip of kv_cache_push, cuda/forward_layer.cu:182-190).
void dequant_rows(const uint8_t *codes, const int8_t *sexp, const uint16_t *tail,
                  const int64_t *rows, int n_rows, int head_dim, int n_rot,
                  std::vector<float> &buf) {
    const int n_nope = head_dim - n_rot;
    buf.resize((size_t)n_rows * head_dim);
    for (int r = 0; r < n_rows; ++r) {
        const int64_t p = rows ? rows[r] : r;
        const uint8_t *c = codes + (size_t)p * n_nope;
        const int8_t *e = sexp + (size_t)p * 8;
        const uint16_t *t = tail + (size_t)p * n_rot;
        float *o = buf.data() + (size_t)r * head_dim;
        for (int d = 0; d < n_nope; ++d) o[d] = orc_fp8_deq(c[d], e[d / 64]);
        for (int d = 0; d < n_rot; ++d) o[n_nope + d] = orc_f16_to_f32(t[d]);
    }
}

}  // namespace

extern "C" void orc_attn_decode_mixed_f32(const float *Q, const float *raw_kv, int n_raw,
                                          const float *comp_kv, int n_comp,
                                          const int32_t *comp_allowed, const float *sinks,
                                          float *out, int n_head, int head_dim) {
    const int n = n_raw + n_comp;
    std::vector<float> buf((size_t)(n > 0 ? n : 1) * head_dim);
    std::vector<const float *> rows((size_t)(n > 0 ? n : 1));
    for (int k = 0; k < n; ++k) {
        const bool is_raw = k < n_raw;
        const int kk = is_raw ? k : k - n_raw;
        if (!is_raw && comp_allowed && comp_allowed[kk] == 0) { rows[k] = nullptr; continue; }
        const float *src = (is_raw ? raw_kv : comp_kv) + (size_t)kk * head_dim;
        float *dst = buf.data() + (size_t)k * head_dim;
        for (int d = 0; d < head_dim; ++d) dst[d] = orc_f16_round(src[d]);
        rows[k] = dst;
    }
    run_heads(Q, rows.data(), n, sinks, out, n_head, head_dim, 1);
}

// cuda/flash_attn.cu:148-244 with K and V read from separate buffers (both
// f16-rounded on read).
extern "C" void orc_attn_decode_kv_f32(const float *Q, const float *K, const float *V, int n_kv,
                                       const float *sinks, float *out, int n_head,
                                       int head_dim) {
    std::vector<float> kb((size_t)(n_kv > 0 ? n_kv : 1) * head_dim), vb(kb.size());
    std::vector<const float *> kr((size_t)(n_kv > 0 ? n_kv : 1)), vr(kr.size());
    for (int k = 0; k < n_kv; ++k) {
        for (int d = 0; d < head_dim; ++d) {
            kb[(size_t)k * head_dim + d] = orc_f16_round(K[(size_t)k * head_dim + d]);
            vb[(size_t)k * head_dim + d] = orc_f16_round(V[(size_t)k * head_dim + d]);
        }
        kr[k] = kb.data() + (size_t)k * head_dim;
        vr[k] = vb.data() + (size_t)k * head_dim;
    }
    const float kq_scale = 1.0f / std::sqrt((float)head_dim);
    std::vector<float> scores;
    for (int h = 0; h < n_head; ++h)
        head_attention(Q + (size_t)h * head_dim, kr.data(), n_kv, sinks[h], kq_scale, head_dim,
                       scores, out + (size_t)h * head_dim, vr.data());
}

extern "C" void orc_attn_decode_fp8(const float *Q, const uint8_t *codes, const int8_t *sexp,
                                    const uint16_t *tail, const int64_t *rows, int n_rows,
                                    const float *sinks, float *out, int n_head, int head_dim,
                                    int n_rot, int n_threads) {
    std::vector<float> buf;
    dequant_rows(codes, sexp, tail, rows, n_rows, head_dim, n_rot, buf);
    std::vector<const float *> ptrs((size_t)(n_rows > 0 ? n_rows : 1));
    for (int r = 0; r < n_rows; ++r) ptrs[r] = buf.data() + (size_t)r * head_dim;
    run_heads(Q, ptrs.data(), n_rows, sinks, out, n_head, head_dim, n_threads);
}

extern "C" void orc_attn_prefill_fp8(const float *Q, int n_q, const uint8_t *codes,
                                     const int8_t *sexp, const uint16_t *tail, int n_cached,
                                     const float *sinks, float *out, int n_head, int head_dim,
                                     int n_rot, int n_threads) {
    const int n_all = n_cached + n_q;
    std::vector<float> buf;
    dequant_rows(codes, sexp, tail, nullptr, n_all, head_dim, n_rot, buf);
    std::vector<const float *> ptrs((size_t)n_all);
    for (int r = 0; r < n_all; ++r) ptrs[r] = buf.data() + (size_t)r * head_dim;
    for (int t = 0; t < n_q; ++t) {
        run_heads(Q + (size_t)t * n_head * head_dim, ptrs.data(), n_cached + t + 1, sinks,
                  out + (size_t)t * n_head * head_dim, n_head, head_dim, n_threads);
    }
}
