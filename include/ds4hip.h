/* ds4hip.h — C-ABI of the gfx950 attention path (libds4hip.so).
 *
 * Every entry point returns 0 on success, -22 (EINVAL) for a rejected shape or
 * argument, or -1000 - hipError_t when the HIP runtime reports an error. All
 * pointers are caller-owned device memory unless a parameter says "host". All
 * launches are asynchronous on `stream` (a hipStream_t, NULL = default
 * stream) and nothing synchronizes internally. The C++ launchers with the
 * reference's exact names and parameter order live in ds4hip_launchers.h.
 *
 * Layout of the FP8 KV cache shared by the quantizer and the attention
 * kernels (one latent KV head of head_dim = 512, n_rot = 64):
 *   codes [row][448]   E4M3FN codes of dims [0,448) (sign bit 0x80)
 *   sexp  [row][8]     int8 power-of-two scale exponents of the seven 64-dim
 *                      blocks (slot 7 is zero padding)
 *   tail  [row][64]    the RoPE tail dims [448,512) as IEEE f16
 * 584 bytes per row. Element d < 448 of a row reads as
 * f16(value(code) * 2^sexp[d/64]); tail elements read as their f16 value.
 */
#ifndef DS4HIP_H
#define DS4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ---------------------------------------------------------------- */

/* Last non-zero status set by any entry point of this library (process-wide),
 * for the void-returning C++ shims. Reading it does not clear it. */
int ds4hip_get_last_error(void);
int ds4hip_set_last_error(int code);
/* Library version, (major << 16) | minor. */
int ds4hip_version(void);

/* ---- FP8 KV quantizer ---------------------------------------------------------- */

/* Replaces ds4cuda::launch_fp8_kv_quantize_round_trip_f32
 * (cuda/fp8_kv.cuh:62). Per row: dims [0, head_dim - n_rot) quantized to
 * E4M3FN in 64-element blocks with scale 2^ceil(log2(max(amax,1e-4)/448)) and
 * written back dequantized; the n_rot tail is copied through. In-place safe.
 * Requires head_dim <= 512, head_dim % 64 == 0, (head_dim - n_rot) % 64 == 0. */
int ds4hip_fp8_kv_quantize_round_trip_f32(const float *kv_in, float *kv_out, int n_rows,
                                          int head_dim, int n_rot, void *stream);

/* FP8-cache append (additive; the reference stores fp32 rows, so it has no
 * counterpart — it is the cache-writing form of the same quantizer,
 * cuda/fp8_kv.cu:144-195 + the f16 push of cuda/forward_layer.cu:182-190).
 * Row r of kv_in [n_rows][head_dim] fp32 is written to physical cache row
 * dst_rows[r] (device int64 array) or, when dst_rows is NULL, row0 + r. */
int ds4hip_fp8_kv_quantize_append(const float *kv_in, int n_rows, int head_dim, int n_rot,
                                  uint8_t *codes, int8_t *sexp, uint16_t *tail,
                                  long long row0, const long long *dst_rows, void *stream);

/* ---- decode attention ------------------------------------------------------------- */

/* Replaces ds4cuda::launch_flash_attn_decode_raw_f32 (cuda/flash_attn.cuh:73).
 * fp32 Q [n_head][head_dim], K == V rows [n_kv][head_dim] (MLA: the caller
 * passes the same buffer, cuda/forward_layer.cu:1167; K != V is rejected),
 * sinks [n_head], out [n_head][head_dim]. n_head = 64, head_dim = 512; the
 * reference's n_kv <= 128 cap is lifted. Partial-result scratch is
 * stream-ordered hipMallocAsync / hipFreeAsync. */
int ds4hip_flash_attn_decode_raw_f32(const float *Q, const float *K, const float *V,
                                     const float *sinks, float *out, int n_head, int n_kv,
                                     int head_dim, void *stream);

/* Replaces ds4cuda::launch_flash_attn_decode_mixed_f32 (cuda/flash_attn.cuh:142).
 * Rows are n_raw rows of raw_kv followed by n_comp rows of comp_kv; comp row c
 * is skipped when comp_allowed != NULL and comp_allowed[c] == 0. Same shape
 * rules as the raw launcher; no n_raw + n_comp cap. */
int ds4hip_flash_attn_decode_mixed_f32(const float *Q, const float *raw_kv,
                                       const float *comp_kv, const int32_t *comp_allowed,
                                       const float *sinks, float *out, int n_head, int n_raw,
                                       int n_comp, int head_dim, void *stream);

/* Workspace bytes needed by ds4hip_flash_attn_decode_fp8 for the given host
 * array of per-problem row counts. */
int ds4hip_flash_attn_decode_fp8_workspace_size(const long long *n_rows_per_prob, int n_prob,
                                                size_t *bytes);

/* Decode attention over the FP8 cache (additive: the FP8-cache form of
 * cuda/flash_attn.cuh:9-26,90-117, which take fp32 rows). Solves n_prob
 * independent single-query problems in one launch pair — layers of one token,
 * or sequences of a batch:
 *   q      problem p at q + p*q_stride elements, [64][512], bf16 bits
 *          (q_is_f32 = 0) or fp32 (q_is_f32 = 1)
 *   sinks  sinks + p*sinks_stride, [64] fp32
 *   out    out + p*out_stride, [64][512] fp32
 *   n_rows_per_prob  HOST array [n_prob] of row counts (n_prob <= 128)
 * Logical row r of problem p reads position pos = row_idx[p*row_idx_stride + r]
 * (or r when row_idx is NULL) and physical cache row
 *   page_table[p*page_table_stride + pos / page_rows] * page_rows + pos % page_rows
 * when page_table != NULL (page_rows a power of two), else
 *   (row_base ? row_base[p] : p*row_base_stride) + pos.
 * workspace must hold ds4hip_flash_attn_decode_fp8_workspace_size bytes.
 * phases: 3 runs both kernels; 1 launches only the split partial kernel and 2
 * only the merge, so a caller can place the merge next to its consumer (the
 * partials stay in the workspace between the two). */
int ds4hip_flash_attn_decode_fp8(const void *q, int q_is_f32, long long q_stride,
                                 const float *sinks, long long sinks_stride, float *out,
                                 long long out_stride, const uint8_t *codes, const int8_t *sexp,
                                 const uint16_t *tail, const long long *n_rows_per_prob,
                                 int n_prob, const long long *row_base,
                                 long long row_base_stride, const int32_t *row_idx,
                                 long long row_idx_stride, const int32_t *page_table,
                                 int page_table_stride, int page_rows, int n_head, int head_dim,
                                 int n_rot, void *workspace, size_t workspace_bytes,
                                 int phases, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DS4HIP_H */
