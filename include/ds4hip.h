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

/* Last non-zero status set by an entry point of this library on the calling
 * host thread (thread-local, like hipGetLastError), for the void-returning
 * C++ shims. Reading it does not clear it. */
int ds4hip_get_last_error(void);
int ds4hip_set_last_error(int code);
/* Returns the calling thread's last non-zero status and resets it to 0 (the
 * analogue of hipGetLastError for this library). */
int ds4hip_clear_last_error(void);
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

/* The row pushes of a batched step in one launch (no reference counterpart):
 * two FP8 appends (rows fp8_src[k] [fp8_n[k]][head_dim] fp32 to cache rows
 * fp8_dst[k][r], as ds4hip_fp8_kv_quantize_append) and one fp32 row scatter
 * (as ds4hip_rows_scatter_f32: f32_src row r to f32_dst row f32_dst_rows[r],
 * f32_width floats). A set with n = 0 is skipped. The results equal the
 * three separate calls. */
typedef struct ds4hip_rows_push {
    const float *fp8_src[2];
    int fp8_n[2];
    const long long *fp8_dst[2];
    const float *f32_src;
    int f32_n, f32_width;
    float *f32_dst;
    const long long *f32_dst_rows;
} ds4hip_rows_push;
int ds4hip_batch_rows_push_f32(const ds4hip_rows_push *p, uint8_t *codes, int8_t *sexp, uint16_t *tail,
                               int head_dim, int n_rot, void *stream);

/* ---- decode attention ------------------------------------------------------------- */

/* Replaces ds4cuda::launch_flash_attn_decode_raw_f32 (cuda/flash_attn.cuh:73).
 * fp32 Q [n_head][head_dim], K and V rows [n_kv][head_dim] (the same buffer in
 * the MLA layout, cuda/forward_layer.cu:1167, or two buffers), sinks
 * [n_head], out [n_head][head_dim]. n_head = 64, head_dim = 512; the
 * reference's n_kv <= 128 cap is lifted. The split-K partials need scratch:
 * this form takes it stream-ordered (hipMallocAsync / hipFreeAsync, freed
 * before the call returns); the _prealloc form below allocates nothing. */
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

/* Bytes of caller workspace the _prealloc fp32 launchers need for n_rows rows
 * (n_raw + n_comp). */
int ds4hip_flash_attn_decode_f32_workspace_size(long long n_rows, size_t *bytes);

/* ds4cuda::launch_flash_attn_decode_raw_f32 / _mixed_f32 with caller scratch
 * (the _prealloc convention of cuda/compressor.cuh:96-101 and
 * cuda/attn_out.cuh:94-97): the same results, no allocation. workspace holds
 * ds4hip_flash_attn_decode_f32_workspace_size(n_rows) bytes; calls that share
 * one workspace must be ordered on one stream. */
int ds4hip_flash_attn_decode_raw_f32_prealloc(const float *Q, const float *K, const float *V,
                                              const float *sinks, float *out, int n_head,
                                              int n_kv, int head_dim, void *workspace,
                                              size_t workspace_bytes, void *stream);
int ds4hip_flash_attn_decode_mixed_f32_prealloc(const float *Q, const float *raw_kv,
                                                const float *comp_kv,
                                                const int32_t *comp_allowed,
                                                const float *sinks, float *out, int n_head,
                                                int n_raw, int n_comp, int head_dim,
                                                void *workspace, size_t workspace_bytes,
                                                void *stream);

/* Allocation-free form of ds4hip_flash_attn_decode_mixed_f32 (no counterpart
 * in the reference): for callers that cannot call hipMalloc (code under graph
 * capture, tight serving loops, harnesses that forbid allocation). Same
 * arguments and results; the split-K partials live in a library-owned 8.5 MiB
 * device array per GPU (held until the process ends), so the call allocates
 * nothing and takes no workspace. n_raw + n_comp <= 4194304 (larger: -22).
 * Calls that overlap on one GPU (several streams or host threads) share that
 * array and race: order them on one stream. */
int ds4hip_flash_attn_decode_mixed_f32_noalloc(const float *Q, const float *raw_kv,
                                               const float *comp_kv,
                                               const int32_t *comp_allowed, const float *sinks,
                                               float *out, int n_head, int n_raw, int n_comp,
                                               int head_dim, void *stream);

/* Workspace bytes needed by ds4hip_flash_attn_decode_fp8 for the given host
 * array of per-problem row counts. */
int ds4hip_flash_attn_decode_fp8_workspace_size(const long long *n_rows_per_prob, int n_prob,
                                                size_t *bytes);

/* Per-call options of ds4hip_flash_attn_decode_fp8 (no counterpart in the
 * reference, whose scalar kernel keeps P in fp32, cuda/flash_attn.cu:70-85).
 * NULL selects the defaults (all fields 0). Nothing is process-wide: calls
 * with different options may run concurrently on different streams. */
typedef struct ds4hip_decode_opts {
    /* P . V precision of the bf16-Q decode: 0 (default) passes P as one f16
     * (max-abs error ~1e-3 x RMS(out), a third fewer MFMAs); 1 as f16 hi + lo
     * halves (~22 bits). The fp32-Q path always uses hi + lo. */
    int exact_p;
    /* DS4HIP_DECODE_KERNEL_AUTO (default): direct rows with one f16 P run the
     * flat-stage kernel, everything else the register-load kernel;
     * DS4HIP_DECODE_KERNEL_REGLOAD: the register-load kernel for direct rows too. */
    int kernel;
    /* What the merge writes. DS4HIP_DECODE_OUT_F32 (default): out.
     * DS4HIP_DECODE_OUT_ROPE_Q8: instead of out, each head's row after the
     * inverse tail RoPE (n_rot dims at position out_pos with layer out_il's
     * parameters, as ds4hip_tail_rope_yarn_inverse_f32) in Q8_0 form: int8
     * values at q8_out + p*n_head*head_dim and one fp32 scale per 32 values at
     * q8_scale + p*n_head*head_dim/32 (the quantization of
     * ds4hip_attn_out_decode_f32's first step, bit for bit) — the input of
     * ds4hip_attn_out_decode_q8_f32. DS4HIP_DECODE_OUT_ROPE_F32: out, each
     * head's row after that inverse tail RoPE (ds4hip_tail_rope_yarn_batch_f32
     * of out, bit for bit). out_pos_dev (device int32 [n_prob], may be NULL):
     * problem p's position, in place of out_pos. */
    int out_form;
    int out_pos, out_il;
    int8_t *q8_out;
    float *q8_scale;
    const int *out_pos_dev;
} ds4hip_decode_opts;
#define DS4HIP_DECODE_KERNEL_AUTO 0
#define DS4HIP_DECODE_KERNEL_REGLOAD 1
#define DS4HIP_DECODE_OUT_F32 0
#define DS4HIP_DECODE_OUT_ROPE_Q8 1
#define DS4HIP_DECODE_OUT_ROPE_F32 2

/* Decode attention over the FP8 cache (additive: the FP8-cache form of
 * cuda/flash_attn.cuh:9-26,90-117, which take fp32 rows). Solves n_prob
 * independent single-query problems in one launch pair — layers of one token,
 * or sequences of a batch:
 *   q      problem p at q + p*q_stride elements, [64][512], bf16 bits
 *          (q_is_f32 = 0) or fp32 (q_is_f32 = 1), or (q_is_f32 = 2) an fp32 Q
 *          as ds4hip_flash_attn_q_prep_f32 wrote it (q_stride in 32-bit
 *          words; same results as q_is_f32 = 1 on the unconverted Q, bit for
 *          bit; not with DS4HIP_DECODE_KERNEL_REGLOAD)
 *   sinks  sinks + p*sinks_stride, [64] fp32
 *   out    out + p*out_stride, [64][512] fp32
 *   n_rows_per_prob  HOST array [n_prob] of row counts (n_prob <= 128)
 *   row_base, row_idx, page_table  DEVICE arrays (the kernels read them)
 * Logical row r of problem p reads position pos = row_idx[p*row_idx_stride + r]
 * (or r when row_idx is NULL) and physical cache row
 *   page_table[p*page_table_stride + pos / page_rows] * page_rows + pos % page_rows
 * when page_table != NULL (page_rows a power of two), else
 *   (row_base ? row_base[p] : p*row_base_stride) + pos.
 * n_cache_rows (> 0) is the number of rows codes / sexp / tail hold. Direct
 * rows outside it are refused on the host (-22) where the host can see them
 * (row_base NULL); rows the host cannot see (row_base, row_idx, page_table
 * contents) are checked on the device: no row outside [0, n_cache_rows) is
 * ever read, and every output of a problem that named one is NaN.
 * opts: see ds4hip_decode_opts (NULL = defaults).
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
                                 int n_rot, long long n_cache_rows, const ds4hip_decode_opts *opts,
                                 void *workspace, size_t workspace_bytes, int phases, void *stream);

/* The fp32 queries of n_prob decode problems (q + p*q_stride floats,
 * [64][512]) converted to the form the FP8 decode's flat-stage kernel computes
 * from them at its start (three E4M3 parts with per-head E8M0 scales, f16 hi +
 * lo RoPE tail), written to out + p*out_stride 32-bit words
 * (ds4hip_flash_attn_q_prep_words() words each, 16-byte aligned). Decoding
 * with q_is_f32 = 2 then skips that work. Additive: no counterpart in the
 * reference, whose decode takes the fp32 Q (cuda/flash_attn.cuh:9-26). */
int ds4hip_flash_attn_q_prep_f32(const float *q, long long q_stride, int n_prob, void *out,
                                 long long out_stride, void *stream);
long long ds4hip_flash_attn_q_prep_words(void);

/* ---- chunked prefill ------------------------------------------------------------- */

/* Causal chunked-prefill attention over the FP8 cache (additive: the
 * reference runs prefill token by token through the decode launchers,
 * cuda/forward_batch.cu:264-284; this is the batched form of the same math,
 * cuda/flash_attn.cuh:9-26). Query t (0 <= t < n_q) of the chunk sits at
 * position n_cached + t and attends cache rows [0, n_cached + t]; the chunk's
 * own rows must already be in the cache (rows n_cached .. n_cached+n_q-1).
 * q [n_q][64][512] bf16 bits, sinks [64] fp32, out [n_q][64][512] fp32;
 * codes/sexp/tail point at the sequence's row 0. workspace holds
 * ds4hip_flash_attn_prefill_fp8_workspace_size(n_q) bytes (one flag per query
 * pair: pairs whose softmax range outgrows the fast kernel are redone by a
 * second, rescaling kernel in the same call). exact_p: 0 passes P to the P . V
 * MFMAs as one f16 (l sums the rounded values, so each output stays an exactly
 * normalized average), 1 as f16 hi + lo halves (~22 bits, twice the P . V
 * MFMAs). Per call; nothing is process-wide. */
size_t ds4hip_flash_attn_prefill_fp8_workspace_size(int n_q);
int ds4hip_flash_attn_prefill_fp8(const void *q, const float *sinks, float *out,
                                  const uint8_t *codes, const int8_t *sexp, const uint16_t *tail,
                                  int n_q, int n_cached, int n_head, int head_dim, int n_rot,
                                  void *workspace, size_t workspace_bytes, int exact_p, void *stream);

/* ---- tail RoPE YaRN --------------------------------------------------------------- */

/* Replaces ds4cuda::launch_tail_rope_yarn_f32 (cuda/rope.cuh:51): rotates the
 * last n_rot dims of each of n_heads rows of head_dim floats with the layer
 * il's YaRN parameters at position pos; the other dims are copied. In-place
 * safe. n_rot even, <= 128. */
int ds4hip_tail_rope_yarn_f32(const float *x_in, float *x_out, int n_heads, int head_dim,
                              int n_rot, int pos, int il, void *stream);

/* Replaces ds4cuda::launch_tail_rope_yarn_inverse_f32 (cuda/attn_out.cuh:52):
 * the same rotation with the sine negated. */
int ds4hip_tail_rope_yarn_inverse_f32(const float *x_in, float *x_out, int n_heads,
                                      int head_dim, int n_rot, int pos, int il, void *stream);

/* ---- matvecs ------------------------------------------------------------------------ */

/* Replaces ds4cuda::launch_mul_mv_f16_f32 (cuda/router.cuh:62): y[o] =
 * sum_i f16(w[o*in_dim + i]) * x[i], fp32 accumulation. in_dim <= 16384. */
int ds4hip_mul_mv_f16_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32, int out_dim,
                          int in_dim, void *stream);

/* Replaces ds4cuda::launch_mul_mv_q8_0_q8_0_grouped_f32 (cuda/attn_out.cuh:86).
 * W: n_groups*rank rows of group_dim/32 block_q8_0 records (34 bytes: f16 d,
 * 32 int8). x: n_groups*group_dim fp32, quantized per 32 elements
 * (d = amax/127, fp32 scale). Row r reads group r / rank. The activations
 * live in the library's per-stream scratch: nothing is allocated per call. */
int ds4hip_mul_mv_q8_0_q8_0_grouped_f32(const void *W, const float *x, float *y, int n_groups,
                                        int group_dim, int rank, void *stream);

/* Replaces ds4cuda::launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc
 * (cuda/attn_out.cuh:98): caller scratch int8 [n_groups*group_dim] and
 * fp32 [n_groups*group_dim/32]; allocates nothing. */
int ds4hip_mul_mv_q8_0_q8_0_grouped_f32_prealloc(const void *W, const float *x, float *y,
                                                 int n_groups, int group_dim, int rank,
                                                 int8_t *scratch_xq, float *scratch_xscale,
                                                 void *stream);

/* Replaces ds4cuda::launch_mul_mv_q8_0_q8_0_f32_prealloc (cuda/dense_q8.cuh:62):
 * dense Q8_0 x Q8_0, W n_rows x n_cols. */
int ds4hip_mul_mv_q8_0_q8_0_f32_prealloc(const void *W, const float *x, float *y, int n_rows,
                                         int n_cols, int8_t *scratch_xq, float *scratch_xscale,
                                         void *stream);

/* Fused launches (no reference counterpart: each replaces a pair of the
 * launchers above with the same arithmetic, so the results are bit-identical
 * to the pair; for callers that count launches, e.g. a per-token slice):
 *
 * ds4hip_mul_mv_f16_scaled_f32: ds4hip_mul_mv_f16_f32, then every output times
 * scale (the indexer head weights and their 1/sqrt(d * n_head) scale,
 * cuda/forward_layer.cu:1054-1060).
 *
 * ds4hip_mul_mv_f16_rope_f32: ds4hip_mul_mv_f16_f32 into n_heads rows of
 * head_dim, then ds4hip_tail_rope_yarn_f32 (the indexer query,
 * cuda/forward_layer.cu:1046-1053). head_dim and n_rot multiples of 4.
 *
 * ds4hip_attn_out_decode_q8_f32: ds4hip_attn_out_decode_f32 after its
 * first step, from the rotated Q8_0 attention output (a decode merge's
 * DS4HIP_DECODE_OUT_ROPE_Q8 form: xq [n_head*head_dim] int8, xscale
 * [n_head*head_dim/32]); the same results bit for bit.
 *
 * ds4hip_attn_out_decode_f32: Steps 14-16 (cuda/forward_layer.cu:1172-1210):
 * ds4hip_tail_rope_yarn_inverse_f32 of kqv [n_head][head_dim], the grouped
 * Q8_0 projection (n_groups groups, rank rows each) and the dense Q8_0
 * projection to out_dim, with the rotation and the first quantization in one
 * launch. Workspace: ds4hip_attn_out_decode_workspace_bytes. */
/* One layer step's independent launches of Steps 11-12c as one launch (no
 * reference counterpart; for a per-token slice that counts launches). Jobs:
 *   - the FP8 push: kv [head_dim] into cache row kv_row of codes / sexp / tail
 *     (as ds4hip_fp8_kv_quantize_append of one row);
 *   - n_comp (0..2) compressor projections over x [in_dim] with f16 weights
 *     (the projection half of ds4hip_compressor_decode_step_f32_prealloc at
 *     pos; the emit, on steps where (pos + 1) % ratio == 0, is
 *     ds4hip_compressor_emit_f32 afterwards);
 *   - if q_w: the indexer query, q_out = RoPE(q_w . q_x) (as
 *     ds4hip_mul_mv_f16_rope_f32 with n_rot 64);
 *   - if hw_w: the head weights, hw_out = (hw_w . x) * hw_scale (as
 *     ds4hip_mul_mv_f16_scaled_f32);
 *   - if qp_q: the layer's decode query qp_q [64][512] fp32 converted for
 *     the decode into qp_out (as ds4hip_flash_attn_q_prep_f32 of one problem).
 * head_dim 512 and n_rot 64 (the session's rows). The results are
 * bit-identical to those launches. in_dim, q_in <= 8192. */
typedef struct ds4hip_token_prologue {
    const float *kv;
    uint8_t *codes;
    int8_t *sexp;
    uint16_t *tail;
    long long kv_row;
    int head_dim, n_rot;
    const float *x;
    int in_dim, n_comp;
    const uint16_t *comp0_w_kv, *comp0_w_gate, *comp0_w_ape;
    float *comp0_state_kv, *comp0_state_score;
    int comp0_head_dim_out, comp0_ratio, comp0_pos;
    const uint16_t *comp1_w_kv, *comp1_w_gate, *comp1_w_ape;
    float *comp1_state_kv, *comp1_state_score;
    int comp1_head_dim_out, comp1_ratio, comp1_pos;
    const uint16_t *q_w;
    const float *q_x;
    float *q_out;
    int q_heads, q_head_dim, q_in, q_pos, q_il;
    const uint16_t *hw_w;
    float *hw_out;
    int hw_rows;
    float hw_scale;
    const float *qp_q;
    void *qp_out;
} ds4hip_token_prologue;
int ds4hip_token_prologue_f32(const ds4hip_token_prologue *a, void *stream);

/* The emit half of ds4hip_compressor_decode_step_f32_prealloc for a step whose
 * projection already ran (through ds4hip_token_prologue_f32): pool, RMSNorm,
 * tail RoPE at pos + 1 - ratio, FP8 round trip (is_attn) and the ratio-4 ring
 * shift, into emit_out [head_dim_out]. Only for (pos + 1) % ratio == 0. */
int ds4hip_compressor_emit_f32(int is_attn, const float *w_norm_f32, int head_dim_out, int compress_ratio,
                               int pos, int il, float *state_kv, float *state_score, float *emit_out,
                               void *stream);

int ds4hip_mul_mv_f16_scaled_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32, int out_dim,
                                 int in_dim, float scale, void *stream);
int ds4hip_mul_mv_f16_rope_f32(const uint16_t *w_f16, const float *x_f32, float *y_f32, int n_heads,
                               int head_dim, int n_rot, int pos, int il, int in_dim, void *stream);
size_t ds4hip_attn_out_decode_workspace_bytes(int n_head, int head_dim, int n_groups, int rank);
int ds4hip_attn_out_decode_f32(const float *kqv, const void *w_out_a, const void *w_out_b, float *out,
                               int n_head, int head_dim, int n_rot, int pos, int il, int n_groups, int rank,
                               int out_dim, void *workspace, size_t workspace_bytes, void *stream);
int ds4hip_attn_out_decode_q8_f32(const int8_t *xq, const float *xscale, const void *w_out_a, const void *w_out_b,
                                  float *out, int n_head, int head_dim, int n_groups, int rank, int out_dim,
                                  void *workspace, size_t workspace_bytes, void *stream);

/* Replaces ds4cuda::launch_rms_norm_f32 (cuda/norm.cuh:24): one row of n,
 * y = x * (1 / sqrtf(mean(x^2) + eps)) * w, fp32 accumulation. */
int ds4hip_rms_norm_f32(const float *x, const float *w, float *y, int n, float eps, void *stream);

/* Replaces ds4cuda::launch_rms_norm_batch_f32 (cuda/norm.cuh:40): n_rows rows
 * of n_per_row, each normalized on its own; weight_dim 0 (unit gain, w may be
 * NULL), n_per_row (w shared) or n_rows * n_per_row (a weight row each). */
int ds4hip_rms_norm_batch_f32(const float *x, const float *w, int weight_dim, float *y, int n_rows,
                              int n_per_row, float eps, void *stream);

/* Workspace bytes of ds4hip_attn_qkv_decode_f32. */
size_t ds4hip_attn_qkv_decode_workspace_bytes(void);

/* The decode Q / KV producer of one layer, Steps 3-10 of
 * cuda/forward_layer.cu:827-913 in one call (six launches, no allocation):
 *   q_lora      = Q8_0 matvec(w_q_a [1024 x 4096], attn_norm [4096])
 *   q_lora_norm = RMSNorm(q_lora, w_q_a_norm [1024])          -> q_lora_norm
 *   kv_raw      = Q8_0 matvec(w_kv_a [512 x 4096], attn_norm)
 *   kv_rope     = tail RoPE(RMSNorm(kv_raw, w_kv_a_norm [512]), pos, il) -> kv_rope
 *   q_raw       = Q8_0 matvec(w_q_b [32768 x 1024], q_lora_norm)
 *   q_cur       = tail RoPE(per-head RMSNorm(q_raw) [64 x 512], pos, il) -> q_cur
 * with eps 1e-6, weights as block_q8_0 rows. kv_rope is what
 * ds4hip_session_push_raw / ds4hip_fp8_kv_quantize_append take (Step 11) and
 * q_lora_norm is the indexer query's input. */
int ds4hip_attn_qkv_decode_f32(const float *attn_norm, const void *w_q_a, const float *w_q_a_norm,
                               const void *w_kv_a, const float *w_kv_a_norm, const void *w_q_b,
                               int pos, int il, float *q_lora_norm, float *q_cur, float *kv_rope,
                               void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes of ds4hip_mul_mm_bf16_f32 / ds4hip_mul_mm_f32_f32 for this
 * shape (0 when one column group covers every column). */
size_t ds4hip_mul_mm_workspace_bytes(int n_rows, int n_cols, int n_batch);

/* Batched bf16 projection (additive; the forward_batch form of the attention
 * output projection): Y[b][r] = sum_c W[r][c] X[b][c] for n_batch <= 16 rows
 * of X, W bf16 [n_rows][n_cols], n_cols % 32 == 0. Y is overwritten. The
 * column groups' partial sums go to workspace (ds4hip_mul_mm_workspace_bytes)
 * and are added in a fixed order: the result is the same on every run. */
int ds4hip_mul_mm_bf16_f32(const uint16_t *W, const float *X, float *Y, int n_rows, int n_cols,
                           int n_batch, void *workspace, size_t workspace_bytes, void *stream);

/* Batched fp32 projection (additive; the batched-decode compressor
 * projection): Y[b][r] = sum_c W[r][c] X[b][c], W fp32 [n_rows][n_cols],
 * n_batch <= 16, n_cols % 32 == 0. Y is overwritten; workspace as above. */
int ds4hip_mul_mm_f32_f32(const float *W, const float *X, float *Y, int n_rows, int n_cols,
                          int n_batch, void *workspace, size_t workspace_bytes, void *stream);

/* Tail RoPE for n_seq sequences at their own positions (additive; batched form
 * of ds4hip_tail_rope_yarn_f32 / _inverse_f32): x [n_seq][n_heads][head_dim],
 * pos_dev device int [n_seq]; inverse != 0 negates the sine. In-place safe. */
int ds4hip_tail_rope_yarn_batch_f32(const float *x_in, float *x_out, int n_seq, int n_heads,
                                    int head_dim, int n_rot, const int *pos_dev, int il,
                                    int inverse, void *stream);

/* ---- indexer --------------------------------------------------------------------------- */

/* Replaces ds4cuda::launch_indexer_allowed_short_circuit_i32
 * (cuda/indexer_allowed.cuh:33): out[0..n_comp) = 1. n_comp <= 0 is a no-op;
 * n_comp > top_k returns -22 (the reference aborts). */
int ds4hip_indexer_allowed_short_circuit_i32(int32_t *out_i32, int n_comp, int top_k,
                                             void *stream);

/* Replaces ds4cuda::launch_scale_inplace_f32 (cuda/indexer_allowed.cuh:97). */
int ds4hip_scale_inplace_f32(float *y, int n, float scale, void *stream);

/* Replaces ds4cuda::launch_indexer_score_topk_i32 (cuda/indexer_allowed.cuh:67):
 * scores score[c] = sum_h w[h] relu(q_h . k_c) over f16 keys into
 * scratch_scores, then allowed[c] = 1 for the top_k (score desc, index asc),
 * 0 otherwise; n_comp <= top_k -> all ones; top_k <= 0 -> all zeros;
 * n_comp <= 0 or n_head/head_dim <= 0 -> nothing. n_head <= 64, head_dim <= 128.
 * Scores use a fixed fma order (dot over d ascending, then heads ascending) so
 * the selection is reproducible exactly. Selection scratch is stream-ordered. */
int ds4hip_indexer_score_topk_i32(const float *q, const float *weights,
                                  const uint16_t *index_comp, int n_comp, int n_head,
                                  int head_dim, int top_k, int32_t *allowed_out,
                                  float *scratch_scores, void *stream);

/* Replaces ds4cuda::launch_indexer_score_topk_f32_i32 (cuda/indexer_allowed.cuh:83):
 * the same over fp32 keys. */
int ds4hip_indexer_score_topk_f32_i32(const float *q, const float *weights,
                                      const float *index_comp_f32, int n_comp, int n_head,
                                      int head_dim, int top_k, int32_t *allowed_out,
                                      float *scratch_scores, void *stream);

/* Bytes of selection scratch ds4hip_indexer_topk_positions needs for n_comp keys. */
size_t ds4hip_indexer_select_scratch_bytes(int n_comp);

/* Sparse-decode selection (additive; generalizes cuda/indexer_allowed.cu:200-279).
 * keys: key_kind 0 = fp32, 1 = f16, 2 = bf16, [n_comp][head_dim]. The last
 * n_recent positions are always selected; of the rest the best
 * top_k - n_recent by (score desc, index asc). allowed_mask [n_comp] (0/1)
 * and/or positions_out [min(top_k, n_comp)] (ascending) may be NULL. */
int ds4hip_indexer_topk_positions(const float *q, const float *weights, const void *keys,
                                  int key_kind, int n_comp, int n_head, int head_dim, int top_k,
                                  int n_recent, float *scratch_scores, void *scratch_select,
                                  int32_t *allowed_mask, int32_t *positions_out, void *stream);

/* Sparse-decode selection for up to 16 sequences in one launch pair
 * (additive). Sequence s scores its n_comp_host[s] key rows starting at key
 * row key_row0_host[s] of `keys` (key_kind as above, head_dim 128) with query
 * q[s] [n_head][128] and weights[s] [n_head], into scratch_scores (same row
 * indexing as keys), and writes its selected positions, ascending, to
 * positions_out + s * pos_stride: all n positions when n <= top_k, else the
 * last n_recent plus the best top_k - n_recent of the rest (score desc, index
 * asc). Candidates per sequence <= 16384. */
int ds4hip_indexer_topk_positions_batch(const float *q, const float *weights, const void *keys,
                                        int key_kind, const long long *key_row0_host,
                                        const int *n_comp_host, int n_seq, int n_head,
                                        int head_dim, int top_k, int n_recent,
                                        float *scratch_scores, int32_t *positions_out,
                                        int pos_stride, void *stream);

/* ---- compressor ------------------------------------------------------------------------ */

/* Replaces ds4cuda::launch_compressor_decode_step_f32_prealloc
 * (cuda/compressor.cuh:102): one streaming-compressor step for token pos of
 * layer il. is_attn != 0 FP8 round-trips the emitted row. *emitted_out_host
 * (host int, may be NULL) is set from pos: 1 when (pos + 1) % ratio == 0.
 * ratio 4 or 128; head_dim_out <= 512; in_dim <= 8192. */
int ds4hip_compressor_decode_step_f32_prealloc(int is_attn, const float *x_f32,
                                               const uint16_t *w_kv_f16,
                                               const uint16_t *w_gate_f16,
                                               const uint16_t *w_ape_f16,
                                               const float *w_norm_f32, int in_dim,
                                               int head_dim_out, int compress_ratio, int pos,
                                               int il, float *state_kv, float *state_score,
                                               float *emit_out, int *emitted_out_host,
                                               float *scratch_kv_cur, float *scratch_sc_cur,
                                               void *stream);

/* Replaces ds4cuda::launch_compressor_decode_step_f32 (cuda/compressor.cuh:78);
 * needs no scratch (the projections go straight into the state rows). */
int ds4hip_compressor_decode_step_f32(int is_attn, const float *x_f32, const uint16_t *w_kv_f16,
                                      const uint16_t *w_gate_f16, const uint16_t *w_ape_f16,
                                      const float *w_norm_f32, int in_dim, int head_dim_out,
                                      int compress_ratio, int pos, int il, float *state_kv,
                                      float *state_score, float *emit_out,
                                      int *emitted_out_host, void *stream);

/* The same step with fp32 projection weights (additive; the batched-decode
 * configuration states fp32 compressor weights). */
int ds4hip_compressor_decode_step_w32(int is_attn, const float *x_f32, const float *w_kv_f32,
                                      const float *w_gate_f32, const uint16_t *w_ape_f16,
                                      const float *w_norm_f32, int in_dim, int head_dim_out,
                                      int compress_ratio, int pos, int il, float *state_kv,
                                      float *state_score, float *emit_out,
                                      int *emitted_out_host, void *stream);

/* One compressor step for n_seq <= 16 sequences at once, fp32 weights read once
 * for all of them (additive; batched form of
 * ds4hip_compressor_decode_step_w32). x [n_seq][in_dim]; sequence b is at
 * position pos_host[b] (pos_dev: the same array in device memory) with state
 * at state_kv / state_score + b * state_stride floats; emit_out row b is
 * written when (pos + 1) % ratio == 0, and emitted_out_host[b] (host, may be
 * NULL) says so. scratch: ds4hip_compressor_batch_scratch_bytes(...) bytes
 * (the projections' column-group partials, added in a fixed order, so the
 * step is the same on every run). */
size_t ds4hip_compressor_batch_scratch_bytes(int n_seq, int in_dim, int head_dim_out,
                                             int compress_ratio);
int ds4hip_compressor_decode_step_batch_w32(int is_attn, int n_seq, const float *x_f32,
                                            const float *w_kv_f32, const float *w_gate_f32,
                                            const uint16_t *w_ape_f16, const float *w_norm_f32,
                                            int in_dim, int head_dim_out, int compress_ratio,
                                            const int *pos_host, const int *pos_dev, int il,
                                            float *state_kv, float *state_score,
                                            long long state_stride, float *emit_out,
                                            int *emitted_out_host, float *scratch,
                                            size_t scratch_bytes, void *stream);

/* One layer's two batched compressors at once (no reference counterpart; the
 * reference runs them one after the other, cuda/forward_layer.cu:1021-1072):
 * the attention compressor (is_attn = 1) and the indexer's (is_attn = 0),
 * same x, ratio and positions, in three launches instead of six (both
 * projections, both state updates, both emits). Each job's arguments mean
 * what they mean in ds4hip_compressor_decode_step_batch_w32, and the results
 * equal two calls of it bit for bit. scratch:
 * ds4hip_compressor_pair_batch_scratch_bytes(...) bytes. */
typedef struct ds4hip_compressor_batch_job {
    const float *w_kv_f32, *w_gate_f32;
    const uint16_t *w_ape_f16;
    const float *w_norm_f32;
    int head_dim_out;
    float *state_kv, *state_score;
    long long state_stride;
    float *emit_out;
} ds4hip_compressor_batch_job;
size_t ds4hip_compressor_pair_batch_scratch_bytes(int n_seq, int in_dim, int attn_head_dim_out,
                                                  int index_head_dim_out, int compress_ratio);
int ds4hip_compressor_pair_step_batch_w32(int n_seq, const float *x_f32, int in_dim, int compress_ratio,
                                          const int *pos_host, const int *pos_dev, int il,
                                          const ds4hip_compressor_batch_job *attn,
                                          const ds4hip_compressor_batch_job *index, int *emitted_out_host,
                                          float *scratch, size_t scratch_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DS4HIP_H */
