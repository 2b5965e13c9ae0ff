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

// cuda/indexer_allowed.cu:68-115 (f16 keys) and :120-171 (fp32 keys), one
// block per key c, thread h = head h (block of roundup32(n_head) threads):
//   dot_h = sum_d q_h[d] * k_c[d], accumulated left to right from 0.0f as
//           `dot += qh[d] * kv[d]` (:85-88, :136-139), which nvcc compiles to
//           one fma per step (its default contraction);
//   relu:   `if (dot < 0.0f) dot = 0.0f` (:89), so NaN and -0 pass unchanged;
//   partial_h = dot_h * w[h] (:90), a rounded product (not fused into a sum);
//   each 32-lane warp sums its partials with the xor butterfly
//           partial += shfl_xor(partial, off), off = 16, 8, 4, 2, 1 (:96-99);
//   warp 0 reads the warp sums (lanes >= n_warps read 0.0f) and runs the
//           butterfly with off = 4, 2, 1 over MAX_WARPS = 8 lanes (:103-110);
//   score = lane 0's value.
// Heads >= n_head contribute 0.0f (:80). The butterfly is written out lane by
// lane below; every lane of a butterfly ends with the same value (IEEE
// addition is commutative), so lane 0 is the reference's result.
static float xor_butterfly(float *v, int n_lanes, int first_off) {
    std::vector<float> nv((size_t)n_lanes);
    for (int off = first_off; off > 0; off >>= 1) {
        for (int l = 0; l < n_lanes; ++l) nv[l] = v[l] + v[l ^ off];
        for (int l = 0; l < n_lanes; ++l) v[l] = nv[l];
    }
    return v[0];
}

extern "C" void orc_indexer_scores(const float *q, const float *w, const void *keys,
                                   int key_kind, int n_comp, int n_head, int head_dim,
                                   float *scores) {
    // the launcher's block is min(roundup32(n_head), 256) threads (:318-321)
    const int n_warps = std::min((n_head + 31) / 32, 8);
    std::vector<float> k((size_t)head_dim), lane((size_t)32 * n_warps);
    for (int c = 0; c < n_comp; ++c) {
        for (int d = 0; d < head_dim; ++d) k[d] = key_at(keys, key_kind, (size_t)c * head_dim + d);
        for (int h = 0; h < 32 * n_warps; ++h) {
            float partial = 0.0f;
            if (h < n_head) {
                const float *qh = q + (size_t)h * head_dim;
                float dot = 0.0f;
                for (int d = 0; d < head_dim; ++d) dot = std::fmaf(qh[d], k[d], dot);
                if (dot < 0.0f) dot = 0.0f;
                partial = dot * w[h];
            }
            lane[h] = partial;
        }
        float warp_sums[8];
        for (int wv = 0; wv < 8; ++wv)
            warp_sums[wv] = wv < n_warps ? xor_butterfly(&lane[(size_t)32 * wv], 32, 16) : 0.0f;
        scores[c] = xor_butterfly(warp_sums, 8, 4);
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
