// indexer.cpp — oracle: lightning-indexer scores and top-k selection.
// TEST INFRASTRUCTURE ONLY (see ds4_oracle.h).

#include "ds4_oracle.h"

#include <algorithm>
#include <cmath>
#include <vector>

static inline float key_at(const void *keys, int kind, size_t i) {
    switch (kind) {
    case 0: return static_cast<const float *>(keys)[i];
    case 1: return orc_f16_to_f32(static_cast<const uint16_t *>(keys)[i]);
    default: return orc_bf16_to_f32(static_cast<const uint16_t *>(keys)[i]);
    }
}

// cuda/indexer_allowed.cu:68-171 (score = sum_h w_h * relu(q_h . k_c)),
// evaluated in the fixed fma order the HIP kernel uses (ds4_oracle.h).
extern "C" void orc_indexer_scores(const float *q, const float *w, const void *keys,
                                   int key_kind, int n_comp, int n_head, int head_dim,
                                   float *scores) {
    std::vector<float> k((size_t)head_dim);
    for (int c = 0; c < n_comp; ++c) {
        for (int d = 0; d < head_dim; ++d) k[d] = key_at(keys, key_kind, (size_t)c * head_dim + d);
        float s = 0.0f;
        for (int h = 0; h < n_head; ++h) {
            const float *qh = q + (size_t)h * head_dim;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; ++d) dot = std::fmaf(qh[d], k[d], dot);
            const float r = dot > 0.0f ? dot : 0.0f;
            s = std::fmaf(w[h], r, s);
        }
        scores[c] = s;
    }
}

// cuda/indexer_allowed.cu:200-279 and :283-305: repeated argmax over the
// not-yet-selected entries, strict greater-than, so ties go to the lowest
// index; when n_comp <= top_k every entry is allowed (short circuit).
extern "C" void orc_topk_mask(const float *scores, int n_comp, int top_k, int32_t *mask) {
    if (n_comp <= 0) return;
    if (top_k <= 0) { for (int c = 0; c < n_comp; ++c) mask[c] = 0; return; }
    if (n_comp <= top_k) { for (int c = 0; c < n_comp; ++c) mask[c] = 1; return; }
    for (int c = 0; c < n_comp; ++c) mask[c] = 0;
    for (int k = 0; k < top_k; ++k) {
        float best = -INFINITY;
        int bi = -1;
        for (int c = 0; c < n_comp; ++c)
            if (mask[c] == 0 && scores[c] > best) { best = scores[c]; bi = c; }
        mask[bi >= 0 ? bi : 0] = 1;
    }
}

// Sparse-decode selection: {last n_recent} U top-(top_k - n_recent) of the
// rest by (score desc, index asc). Written as a stable sort, the textbook
// statement of the same order the argmax loop produces.
extern "C" int orc_topk_positions(const float *scores, int n_comp, int top_k, int n_recent,
                                  int32_t *pos_out) {
    if (n_comp <= 0 || top_k <= 0) return 0;
    if (n_comp <= top_k) {
        for (int c = 0; c < n_comp; ++c) pos_out[c] = c;
        return n_comp;
    }
    const int n_old = n_comp - n_recent;
    std::vector<int> idx((size_t)n_old);
    for (int c = 0; c < n_old; ++c) idx[c] = c;
    std::stable_sort(idx.begin(), idx.end(),
                     [&](int a, int b) { return scores[a] > scores[b]; });
    const int take = top_k - n_recent;
    std::vector<int> sel(idx.begin(), idx.begin() + take);
    for (int c = n_old; c < n_comp; ++c) sel.push_back(c);
    std::sort(sel.begin(), sel.end());
    for (size_t i = 0; i < sel.size(); ++i) pos_out[i] = sel[i];
    return (int)sel.size();
}
