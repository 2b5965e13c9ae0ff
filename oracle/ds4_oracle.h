// ds4_oracle.h — CPU oracle for the ds4cuda attention path.
//
// TEST INFRASTRUCTURE ONLY. This library is a scalar C++ restatement of the
// reference kernels' math (Kwenai/ds4cuda, cuda/*.cu), written from the
// reference source as a specification. It is the checker for the HIP path:
// only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load it. The product library (ds4cuda_amd/libds4hip.so) never calls it.
//
// Every function cites the reference file:line it follows. The order of fp32
// operations inside ds4.c (the upstream CPU spec the reference kernels were
// aligned to, not vendored in the reference) cannot be observed here, so
// floating-point outputs are tolerance-checked; FP8 codes/scales and top-k
// selections are order-free and checked bit-exactly.

#ifndef DS4_ORACLE_H
#define DS4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- scalar helpers -------------------------------------------------------
// IEEE binary32 -> binary16 (round-to-nearest-even) and back. Restates the
// __float2half / __half2float pair used by f16_round (cuda/flash_attn.cu:113-115).
uint16_t orc_f32_to_f16(float x);
float    orc_f16_to_f32(uint16_t h);
float    orc_f16_round(float x);
// bf16 bits -> f32 (exact widening) and f32 -> bf16 (RNE).
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);

// ---- FP8 E4M3FN KV quantizer (cuda/fp8_kv.cuh:21-35, cuda/fp8_kv.cu:75-195) --
// Table value of E4M3FN magnitude index i in [0,127] (cuda/fp8_kv.cu:88-94).
float orc_e4m3fn_value(int i);
// Nearest table index for |v| <= 448, binary search + even-index tie
// (cuda/fp8_kv.cu:102-131). Returns the magnitude index (0..126).
int   orc_e4m3fn_nearest_index(float ax);
// Power-of-two exponent e with scale = 2^e for a block whose max |x| is amax
// (cuda/fp8_kv.cu:174-176): e = ceil(log2(max(amax,1e-4)/448)), with log2
// evaluated as a correctly rounded fp32 log2.
int   orc_fp8_scale_exp(float amax);
// Quantize one KV row: head_dim - n_rot leading dims in 64-blocks, n_rot tail
// dims passed through (cuda/fp8_kv.cu:144-195). Any output pointer may be NULL.
//   codes  [n_nope] E4M3FN codes (sign bit 0x80 | magnitude index)
//   sexp   [n_nope/64] scale exponents
//   tail   [n_rot] tail dims as f16 bits (the cache stores the tail as f16;
//          every reader f16-rounds it, cuda/forward_layer.cu:182-190)
//   deq    [head_dim] fake-quant fp32 row (the round-trip output)
void orc_fp8_quant_row(const float *x, int head_dim, int n_rot,
                       uint8_t *codes, int8_t *sexp, uint16_t *tail, float *deq);
void orc_fp8_quant_rows(const float *x, int n_rows, int head_dim, int n_rot,
                        uint8_t *codes, int8_t *sexp, uint16_t *tail, float *deq);
// Dequantized value of one cached element as the attention kernels read it:
// f16_round(value(code) * 2^e) (fp8_kv.cu:179 + flash_attn.cu:113-115).
float orc_fp8_deq(uint8_t code, int e);

// ---- decode attention (cuda/flash_attn.cuh:9-26,90-117) ------------------
// fp32 math, K/V rows f16-rounded on read, max seeded with the sink,
// masked comp rows contribute nothing. raw may be NULL when n_raw == 0.
void orc_attn_decode_mixed_f32(const float *Q, const float *raw_kv, int n_raw,
                               const float *comp_kv, int n_comp,
                               const int32_t *comp_allowed, const float *sinks,
                               float *out, int n_head, int head_dim);
// The raw launcher's math with K and V in separate buffers
// (cuda/flash_attn.cu:148-244 reads K[k] for the scores and V[k] for the sum).
void orc_attn_decode_kv_f32(const float *Q, const float *K, const float *V, int n_kv,
                            const float *sinks, float *out, int n_head, int head_dim);
// Same math over rows of the FP8 cache (codes [*,n_nope], sexp [*,8],
// tail [*,n_rot] f16), selected by physical row ids rows[0..n_rows).
// n_threads > 1 splits the heads over std::threads (CPU baseline mode).
void orc_attn_decode_fp8(const float *Q, const uint8_t *codes, const int8_t *sexp,
                         const uint16_t *tail, const int64_t *rows, int n_rows,
                         const float *sinks, float *out, int n_head, int head_dim,
                         int n_rot, int n_threads);

// Causal chunked prefill over the FP8 cache: query token t (0..n_q) sits at
// absolute position n_cached + t and attends rows [0, n_cached + t] with the
// same sink-seeded softmax per head. Q [n_q][n_head][head_dim].
void orc_attn_prefill_fp8(const float *Q, int n_q, const uint8_t *codes,
                          const int8_t *sexp, const uint16_t *tail, int n_cached,
                          const float *sinks, float *out, int n_head, int head_dim,
                          int n_rot, int n_threads);

// ---- indexer (cuda/indexer_allowed.cu:68-279) ----------------------------
// score[c] = sum_h w[h] * relu(q_h . k_c) in the reference kernel's own
// order (cuda/indexer_allowed.cu:68-171): per head an fma chain over d
// ascending from 0, relu, the rounded product dot * w[h], then the 32-lane
// xor butterfly (16, 8, 4, 2, 1) per warp of heads and warp 0's 8-lane xor
// butterfly (4, 2, 1) over the warp sums. key_kind: 0 = f32 keys, 1 = f16
// bits, 2 = bf16 bits (bf16 keys: the same arithmetic, keys widened exactly).
void orc_indexer_scores(const float *q, const float *w, const void *keys,
                        int key_kind, int n_comp, int n_head, int head_dim,
                        float *scores);
// Top-k mask by repeated argmax, ties to the lowest index
// (cuda/indexer_allowed.cu:200-279). n_comp <= top_k -> all ones.
void orc_topk_mask(const float *scores, int n_comp, int top_k, int32_t *mask);
// Allowed position list for sparse decode: the last n_recent positions plus
// the best (top_k - n_recent) of the rest by (score desc, index asc); output
// ascending. Returns the count written (min(top_k, n_comp)).
int  orc_topk_positions(const float *scores, int n_comp, int top_k, int n_recent,
                        int32_t *pos_out);

// ---- tail RoPE YaRN (cuda/rope.cu:114-259, cuda/attn_out.cu:54-107,207-251)
void orc_rope_tail(const float *x_in, float *x_out, int n_heads, int head_dim,
                   int n_rot, int pos, int il, int inverse);

// ---- matvecs -------------------------------------------------------------
// y[o] = sum_i f16(W[o,i]) * x[i] (cuda/router.cu:69-97), fp64 accumulate
// (the oracle's value is the exact sum rounded once).
void orc_mul_mv_f16_f32(const uint16_t *w, const float *x, float *y, int out_dim, int in_dim);
// Per-32 activation quantization (cuda/attn_out.cu:119-145, dense_q8.cu).
void orc_q8_quantize_act(const float *x, int n, int8_t *xq, float *xscale);
// Q8_0 x Q8_0 grouped matvec (cuda/attn_out.cu:159-197). W is n_groups*rank
// rows of group_dim/32 blocks of 34 bytes (f16 d + 32 int8).
void orc_q8_grouped_matvec(const uint8_t *W, const float *x, float *y,
                           int n_groups, int group_dim, int rank);
// Dense Q8_0 x Q8_0 matvec (cuda/dense_q8.cu launch_mul_mv_q8_0_q8_0_f32_prealloc).
void orc_q8_matvec(const uint8_t *W, const float *x, float *y, int n_rows, int n_cols);
// y = W x with W bf16 [n_rows][n_cols], fp64 accumulate.
void orc_bf16_matvec(const uint16_t *W, const float *x, float *y, int n_rows, int n_cols);

// ---- RMSNorm (cuda/norm.cu:4-7, cuda/norm.cuh:26-45) ------------------------
// ss = sum x^2 in fp64, scale = 1 / sqrtf((float)(ss / n) + eps),
// y = x * scale * w; w NULL is unit gain.
void orc_rms_norm_f32(const float *x, const float *w, float *y, int n, float eps);
// weight_dim: 0 (unit gain), n_per_row (shared row), n_rows * n_per_row (per row).
void orc_rms_norm_batch_f32(const float *x, const float *w, int weight_dim, float *y,
                            int n_rows, int n_per_row, float eps);

// ---- compressor decode step (cuda/compressor.cu:64-349) ------------------
// State layout and semantics exactly as the reference. Returns 1 on emit.
int orc_compressor_step(int is_attn, const float *x, const uint16_t *w_kv,
                        const uint16_t *w_gate, const uint16_t *w_ape,
                        const float *w_norm, int in_dim, int head_dim_out,
                        int ratio, int pos, int il, float *state_kv,
                        float *state_score, float *emit_out);
// The same step with fp32 projection weights (fp64 accumulation).
int orc_compressor_step_w32(int is_attn, const float *x, const float *w_kv,
                            const float *w_gate, const uint16_t *w_ape,
                            const float *w_norm, int in_dim, int head_dim_out,
                            int ratio, int pos, int il, float *state_kv,
                            float *state_score, float *emit_out);

#ifdef __cplusplus
}
#endif

#endif
