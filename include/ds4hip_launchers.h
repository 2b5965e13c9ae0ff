/* ds4hip_launchers.h — the reference's C++ launcher surface over libds4hip.so.
 *
 * Header-only shims in namespace ds4cuda with the reference's names, parameter
 * order, default stream argument and void return, each forwarding to the
 * extern "C" entry point of ds4hip.h. As in the reference, errors do not
 * propagate through the return value: a failed call prints one line to stderr
 * and stores its status, which the caller reads with ds4hip_get_last_error()
 * (the reference's callers check cudaGetLastError() after each launch,
 * cuda/forward_layer.cu:81-89). The short-circuit launcher aborts on misuse
 * (n_comp > top_k) like the reference (cuda/indexer_allowed.cu:294-299)
 * unless ds4cuda::ds4hip_abort_on_misuse() is set to false.
 *
 * Link with -lds4hip; include after hip/hip_runtime.h or let this header
 * include it.
 */
#ifndef DS4HIP_LAUNCHERS_H
#define DS4HIP_LAUNCHERS_H

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "ds4hip.h"

namespace ds4cuda {

/* Same 34-byte record as the reference's block_q8_0 (cuda/common.cuh:29):
 * an f16 scale followed by 32 int8 quants. The layout is the on-disk GGUF
 * Q8_0 format, which is why it must be identical. */
struct __attribute__((aligned(2))) block_q8_0 {
    uint16_t d;
    int8_t qs[32];
};
static_assert(sizeof(block_q8_0) == 34, "block_q8_0 is 34 bytes");

inline bool &ds4hip_abort_on_misuse() {
    static bool v = true;
    return v;
}

inline void ds4hip_report(const char *name, int rc) {
    if (rc != 0) std::fprintf(stderr, "ds4hip: %s failed (%d)\n", name, rc);
}

/* cuda/flash_attn.cuh:73 */
inline void launch_flash_attn_decode_raw_f32(const float *Q, const float *K, const float *V,
                                             const float *sinks, float *out, int n_head, int n_kv,
                                             int head_dim, hipStream_t stream = 0) {
    ds4hip_report("launch_flash_attn_decode_raw_f32",
                  ds4hip_flash_attn_decode_raw_f32(Q, K, V, sinks, out, n_head, n_kv, head_dim,
                                                   stream));
}

/* cuda/flash_attn.cuh:142 */
inline void launch_flash_attn_decode_mixed_f32(const float *Q, const float *raw_kv,
                                               const float *comp_kv, const int32_t *comp_allowed,
                                               const float *sinks, float *out, int n_head,
                                               int n_raw, int n_comp, int head_dim,
                                               hipStream_t stream = 0) {
    ds4hip_report("launch_flash_attn_decode_mixed_f32",
                  ds4hip_flash_attn_decode_mixed_f32(Q, raw_kv, comp_kv, comp_allowed, sinks, out,
                                                     n_head, n_raw, n_comp, head_dim, stream));
}

/* cuda/flash_attn.cuh:73 and :142 with caller scratch, following the
 * reference's _prealloc convention (cuda/attn_out.cuh:94-98): the same
 * results as the launchers above, no allocation. workspace: at least
 * ds4hip_flash_attn_decode_f32_workspace_size(n_rows) bytes. */
inline void launch_flash_attn_decode_raw_f32_prealloc(const float *Q, const float *K,
                                                      const float *V, const float *sinks,
                                                      float *out, int n_head, int n_kv,
                                                      int head_dim, void *workspace,
                                                      size_t workspace_bytes,
                                                      hipStream_t stream = 0) {
    ds4hip_report("launch_flash_attn_decode_raw_f32_prealloc",
                  ds4hip_flash_attn_decode_raw_f32_prealloc(Q, K, V, sinks, out, n_head, n_kv,
                                                            head_dim, workspace, workspace_bytes,
                                                            stream));
}

inline void launch_flash_attn_decode_mixed_f32_prealloc(
        const float *Q, const float *raw_kv, const float *comp_kv, const int32_t *comp_allowed,
        const float *sinks, float *out, int n_head, int n_raw, int n_comp, int head_dim,
        void *workspace, size_t workspace_bytes, hipStream_t stream = 0) {
    ds4hip_report("launch_flash_attn_decode_mixed_f32_prealloc",
                  ds4hip_flash_attn_decode_mixed_f32_prealloc(Q, raw_kv, comp_kv, comp_allowed,
                                                              sinks, out, n_head, n_raw, n_comp,
                                                              head_dim, workspace,
                                                              workspace_bytes, stream));
}

/* cuda/fp8_kv.cuh:62 */
inline void launch_fp8_kv_quantize_round_trip_f32(const float *kv_in, float *kv_out, int n_rows,
                                                  int head_dim, int n_rot,
                                                  hipStream_t stream = 0) {
    ds4hip_report("launch_fp8_kv_quantize_round_trip_f32",
                  ds4hip_fp8_kv_quantize_round_trip_f32(kv_in, kv_out, n_rows, head_dim, n_rot,
                                                        stream));
}

/* cuda/indexer_allowed.cuh:33 */
inline void launch_indexer_allowed_short_circuit_i32(int32_t *out_i32, int n_comp, int top_k,
                                                     hipStream_t stream = 0) {
    const int rc = ds4hip_indexer_allowed_short_circuit_i32(out_i32, n_comp, top_k, stream);
    if (rc == -22 && ds4hip_abort_on_misuse() && n_comp > top_k) {
        std::fprintf(stderr, "ds4hip: short circuit with n_comp %d > top_k %d\n", n_comp, top_k);
        std::abort();
    }
    ds4hip_report("launch_indexer_allowed_short_circuit_i32", rc);
}

/* cuda/indexer_allowed.cuh:67 */
inline void launch_indexer_score_topk_i32(const float *q, const float *weights,
                                          const uint16_t *index_comp, int n_comp, int n_head,
                                          int head_dim, int top_k, int32_t *allowed_out,
                                          float *scratch_scores, hipStream_t stream = 0) {
    ds4hip_report("launch_indexer_score_topk_i32",
                  ds4hip_indexer_score_topk_i32(q, weights, index_comp, n_comp, n_head, head_dim,
                                                top_k, allowed_out, scratch_scores, stream));
}

/* cuda/indexer_allowed.cuh:83 */
inline void launch_indexer_score_topk_f32_i32(const float *q, const float *weights,
                                              const float *index_comp_f32, int n_comp, int n_head,
                                              int head_dim, int top_k, int32_t *allowed_out,
                                              float *scratch_scores, hipStream_t stream = 0) {
    ds4hip_report("launch_indexer_score_topk_f32_i32",
                  ds4hip_indexer_score_topk_f32_i32(q, weights, index_comp_f32, n_comp, n_head,
                                                    head_dim, top_k, allowed_out, scratch_scores,
                                                    stream));
}

/* cuda/indexer_allowed.cuh:97 */
inline void launch_scale_inplace_f32(float *y, int n, float scale, hipStream_t stream = 0) {
    ds4hip_report("launch_scale_inplace_f32", ds4hip_scale_inplace_f32(y, n, scale, stream));
}

/* cuda/compressor.cuh:78 */
inline void launch_compressor_decode_step_f32(bool is_attn, const float *x_f32,
                                              const uint16_t *w_kv_f16,
                                              const uint16_t *w_gate_f16,
                                              const uint16_t *w_ape_f16, const float *w_norm_f32,
                                              int in_dim, int head_dim_out, int compress_ratio,
                                              int pos, int il, float *state_kv,
                                              float *state_score, float *emit_out,
                                              int *emitted_out_host, hipStream_t stream = 0) {
    ds4hip_report("launch_compressor_decode_step_f32",
                  ds4hip_compressor_decode_step_f32(
                      is_attn ? 1 : 0, x_f32, w_kv_f16, w_gate_f16, w_ape_f16, w_norm_f32, in_dim,
                      head_dim_out, compress_ratio, pos, il, state_kv, state_score, emit_out,
                      emitted_out_host, stream));
}

/* cuda/compressor.cuh:102 */
inline void launch_compressor_decode_step_f32_prealloc(
    bool is_attn, const float *x_f32, const uint16_t *w_kv_f16, const uint16_t *w_gate_f16,
    const uint16_t *w_ape_f16, const float *w_norm_f32, int in_dim, int head_dim_out,
    int compress_ratio, int pos, int il, float *state_kv, float *state_score, float *emit_out,
    int *emitted_out_host, float *scratch_kv_cur, float *scratch_sc_cur,
    hipStream_t stream = 0) {
    ds4hip_report("launch_compressor_decode_step_f32_prealloc",
                  ds4hip_compressor_decode_step_f32_prealloc(
                      is_attn ? 1 : 0, x_f32, w_kv_f16, w_gate_f16, w_ape_f16, w_norm_f32, in_dim,
                      head_dim_out, compress_ratio, pos, il, state_kv, state_score, emit_out,
                      emitted_out_host, scratch_kv_cur, scratch_sc_cur, stream));
}

/* cuda/attn_out.cuh:52 */
inline void launch_tail_rope_yarn_inverse_f32(const float *x_in, float *x_out, int n_heads,
                                              int head_dim, int n_rot, int pos, int il,
                                              hipStream_t stream = 0) {
    ds4hip_report("launch_tail_rope_yarn_inverse_f32",
                  ds4hip_tail_rope_yarn_inverse_f32(x_in, x_out, n_heads, head_dim, n_rot, pos,
                                                    il, stream));
}

/* cuda/attn_out.cuh:86 */
inline void launch_mul_mv_q8_0_q8_0_grouped_f32(const block_q8_0 *W, const float *x, float *y,
                                                int n_groups, int group_dim, int rank,
                                                hipStream_t stream = 0) {
    ds4hip_report("launch_mul_mv_q8_0_q8_0_grouped_f32",
                  ds4hip_mul_mv_q8_0_q8_0_grouped_f32(W, x, y, n_groups, group_dim, rank,
                                                      stream));
}

/* cuda/attn_out.cuh:98 */
inline void launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(const block_q8_0 *W, const float *x,
                                                         float *y, int n_groups, int group_dim,
                                                         int rank, int8_t *scratch_xq,
                                                         float *scratch_xscale,
                                                         hipStream_t stream = 0) {
    ds4hip_report("launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc",
                  ds4hip_mul_mv_q8_0_q8_0_grouped_f32_prealloc(
                      W, x, y, n_groups, group_dim, rank, scratch_xq, scratch_xscale, stream));
}

/* cuda/dense_q8.cuh:62 */
inline void launch_mul_mv_q8_0_q8_0_f32_prealloc(const block_q8_0 *W_dev,
                                                 const float *x_fp32_dev, float *y_dev,
                                                 int n_rows, int n_cols, int8_t *scratch_xq_dev,
                                                 float *scratch_xscale_dev,
                                                 hipStream_t stream = 0) {
    ds4hip_report("launch_mul_mv_q8_0_q8_0_f32_prealloc",
                  ds4hip_mul_mv_q8_0_q8_0_f32_prealloc(W_dev, x_fp32_dev, y_dev, n_rows, n_cols,
                                                       scratch_xq_dev, scratch_xscale_dev,
                                                       stream));
}

/* cuda/norm.cuh:24 */
inline void launch_rms_norm_f32(const float *x, const float *w, float *y, int n, float eps,
                                hipStream_t stream = 0) {
    ds4hip_report("launch_rms_norm_f32", ds4hip_rms_norm_f32(x, w, y, n, eps, stream));
}

/* cuda/norm.cuh:40 */
inline void launch_rms_norm_batch_f32(const float *x, const float *w, int weight_dim, float *y,
                                      int n_rows, int n_per_row, float eps,
                                      hipStream_t stream = 0) {
    ds4hip_report("launch_rms_norm_batch_f32",
                  ds4hip_rms_norm_batch_f32(x, w, weight_dim, y, n_rows, n_per_row, eps, stream));
}

/* cuda/rope.cuh:51 */
inline void launch_tail_rope_yarn_f32(const float *x_in, float *x_out, int n_heads, int head_dim,
                                      int n_rot, int pos, int il, hipStream_t stream = 0) {
    ds4hip_report("launch_tail_rope_yarn_f32",
                  ds4hip_tail_rope_yarn_f32(x_in, x_out, n_heads, head_dim, n_rot, pos, il,
                                            stream));
}

/* cuda/router.cuh:62 */
inline void launch_mul_mv_f16_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32,
                                  int out_dim, int in_dim, hipStream_t stream = 0) {
    ds4hip_report("launch_mul_mv_f16_f32",
                  ds4hip_mul_mv_f16_f32(w_f16, x_f32, y_f32, out_dim, in_dim, stream));
}

}  // namespace ds4cuda

#endif /* DS4HIP_LAUNCHERS_H */
