/* ds4hip_session.h — KV push / SWA eviction and the per-session KV arena.
 *
 * Same status convention as ds4hip.h (0, -22, -28 = cache full,
 * -1000 - hipError_t). Counters passed as host ints are updated only when the
 * call succeeds.
 */
#ifndef DS4HIP_SESSION_H
#define DS4HIP_SESSION_H

#include <stddef.h>
#include <stdint.h>

#include "ds4hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DS4HIP_N_LAYER 43
#define DS4HIP_N_SWA 128
#define DS4HIP_HEAD_DIM 512
#define DS4HIP_N_ROT 64
#define DS4HIP_INDEXER_HEAD_DIM 128
#define DS4HIP_FP8_CODES 448 /* bytes of E4M3 codes per cache row */
#define DS4HIP_FP8_SEXP 8    /* scale exponents per cache row (7 used) */
#define DS4HIP_FP8_TAIL 64   /* f16 tail elements per cache row */
#define DS4HIP_ENOSPC (-28)
#define DS4HIP_CHUNK_MAX 128 /* tokens per prefill chunk (staging rows in the arena) */

/* ---- reference fp32 row layout --------------------------------------------------- */

/* Raw sliding-window push (cuda/forward_layer.cu:941-972 with the kernels at
 * :159-190). raw_kv is [cap_raw][head_dim] fp32, rows [0, *n_raw_host) valid,
 * oldest first. If *n_raw_host < cap_raw the f16-rounded kv_cur goes to row
 * *n_raw_host and the count grows; otherwise rows 1..cap_raw-1 move down one
 * (f16-rounded, memmove order) and kv_cur goes to the last row. */
int ds4hip_swa_push_f32(float *raw_kv, int *n_raw_host, int cap_raw, const float *kv_cur,
                        int head_dim, void *stream);

/* Compressed-row append (cuda/forward_layer.cu:1021-1034): copies row to
 * comp_kv[*n_comp_host] and increments the count; -28 when the cache is full
 * (there is no eviction). */
int ds4hip_comp_push_f32(float *comp_kv, int *n_comp_host, int cap_comp, const float *row,
                         int head_dim, void *stream);

/* ---- FP8 session arena ------------------------------------------------------------ */

/* FP8 form of struct ds4_layer_state (include/ds4cuda.h:310-360): the KV rows
 * live in the session's FP8 cache (codes/sexp/tail, layout of ds4hip.h); the
 * layer owns rows [row_base, row_base + cap_comp + cap_raw): compressed rows
 * first, then the SWA ring. Compressor and indexer state stay fp32. */
typedef struct ds4hip_layer_state {
    int il;
    int compress_ratio; /* 0 (il < 2), 4 (even il >= 2), 128 (odd il >= 3) */
    int has_indexer;    /* compress_ratio == 4 */
    int cap_raw;        /* min(128, max_context) */
    int n_raw;          /* valid ring rows */
    int raw_head;       /* next ring slot to write (the oldest row once full) */
    int cap_comp;       /* max_context / ratio + 2 (cuda/session_state.cu:137) */
    int n_comp;
    int n_index_comp;
    long long row_base;
    /* device int32 [cap_raw + cap_comp]: cap_comp + cap_raw - 1 - k for the
     * ring part, then 0..cap_comp-1 (compressed rows in order, or the
     * indexer's selection written there); values are relative to row_base. */
    int32_t *row_list;
    float *attn_state_kv;     /* [coff*ratio][coff*512], coff = 2 for ratio 4 */
    float *attn_state_score;  /* same shape, -inf after reset */
    float *index_comp_kv;     /* [cap_comp][128] (ratio 4 only) */
    float *index_state_kv;    /* [8][256] */
    float *index_state_score; /* [8][256], -inf after reset */
} ds4hip_layer_state;

/* FP8 form of struct ds4_session_state (include/ds4cuda.h:392-425): one
 * device allocation carved into the FP8 cache, the row lists and the
 * compressor state. The hyper-connection residual and activation arena of the
 * reference belong to the rest of the layer and are not part of it. */
typedef struct ds4hip_session_state {
    int max_context;
    int pos;
    int n_tokens_processed;
    ds4hip_layer_state layers[DS4HIP_N_LAYER];
    uint8_t *codes;  /* [n_cache_rows][448] */
    int8_t *sexp;    /* [n_cache_rows][8] */
    uint16_t *tail;  /* [n_cache_rows][64] f16 */
    /* the layers' rows; rows [n_cache_rows, n_cache_rows + DS4HIP_CHUNK_MAX)
     * of codes / sexp / tail follow them: the staging rows of a prefill chunk */
    long long n_cache_rows;
    size_t codes_bytes; /* bytes of the cache region at the start of the arena */
    void *arena_base;
    size_t arena_bytes;
} ds4hip_session_state;

/* Device bytes ds4hip_session_state_alloc takes for max_context tokens (pure
 * size calculation; cuda/session_state.cu:147 for the fp32 form). */
size_t ds4hip_session_state_arena_bytes(int max_context);

/* The geometry ds4hip_session_state_alloc would give a session of
 * max_context tokens (capacities, row bases, n_cache_rows, arena_bytes), with
 * every pointer NULL and every counter 0: nothing is allocated. For planning
 * memory and for the host form of ds4hip_session_chunk_rows. */
int ds4hip_session_state_describe(ds4hip_session_state *out, int max_context);

/* One hipMalloc, carved; cache rows zeroed, compressor scores -inf, counters
 * 0 (cuda/session_state.cu:110-256). Synchronizes the null stream once. */
int ds4hip_session_state_alloc(ds4hip_session_state *out, int max_context);

/* Frees the arena and zeroes *s; a zeroed struct is a no-op. */
int ds4hip_session_state_free(ds4hip_session_state *s);

/* Re-initializes buffers and counters for a new sequence, on stream. */
int ds4hip_session_state_reset(ds4hip_session_state *s, void *stream);

/* Quantizes kv_cur [512] fp32 into layer il's SWA ring (overwriting the
 * oldest row once the ring is full). */
int ds4hip_session_push_raw(ds4hip_session_state *s, int il, const float *kv_cur, void *stream);

/* The ring bookkeeping of ds4hip_session_push_raw without the write: the
 * arena row (in codes / sexp / tail) the next raw row goes to, with the ring
 * counters advanced, for a caller that writes the row in a launch of its own
 * (ds4hip_token_prologue_f32). No counterpart in the reference. */
int ds4hip_session_claim_raw_row(ds4hip_session_state *s, int il, long long *row_out);

/* Quantizes an emitted compressed row [512] into the next compressed slot;
 * -28 when full, -22 on a layer without compression. */
int ds4hip_session_push_comp(ds4hip_session_state *s, int il, const float *row, void *stream);

/* Appends an indexer key row [128] fp32; -28 when full. */
int ds4hip_session_push_index_comp(ds4hip_session_state *s, int il, const float *row,
                                   void *stream);

/* Batched push of fp32 rows (additive; the batched-decode form of the
 * compressed-row D2D copies of cuda/forward_layer.cu:1021-1034 and the
 * indexer-key push): dst[dst_rows[r]][0..width) = src[r][0..width) for
 * r < n_rows, dst_rows a device int64 array. width % 4 == 0. */
int ds4hip_rows_scatter_f32(const float *src, int n_rows, int width, float *dst,
                            const long long *dst_rows, void *stream);

/* Writes n compressed-row numbers (device int32 sel[0..n)) where
 * ds4hip_session_layer_rows' *selected_out points: the selection the next
 * decode of layer il reads with n_selected = n (stream-ordered device copy).
 * The prefill chunk driver leaves its last token's indexer selection there,
 * as the token-by-token loop does (cuda/forward_layer.cu:1088-1137 keeps
 * the allowed mask of the last step in the session's scratch). */
int ds4hip_session_set_selection(ds4hip_session_state *s, int il, const int32_t *sel, int n,
                                 void *stream);

/* Rows for layer il's decode attention: *row_idx (device) and *n_rows are
 * the row_idx / n_rows arguments of ds4hip_flash_attn_decode_fp8 with
 * row_base = layers[il].row_base: the valid ring rows, then n_selected
 * compressed rows (n_selected < 0: all n_comp in order). *selected_out
 * (may be NULL) receives where a caller writes the n_selected compressed row
 * numbers (for example ds4hip_indexer_topk_positions' positions_out). */
int ds4hip_session_layer_rows(const ds4hip_session_state *s, int il, int n_selected,
                              const int32_t **row_idx, long long *n_rows, int32_t **selected_out);

/* Row lists of a prefill chunk of layer il (additive; the batched form of the
 * per-token loop of cuda/forward_batch.cu:264-284): tokens t < n_tok at
 * positions p0 + t whose KV rows have been written to the staging rows
 * n_cache_rows + t (not yet to the ring), while the ring still holds exactly
 * the positions < p0. Token t attends the window rows still in the ring
 * (positions max(0, p0 + t - 127) .. p0 - 1), staging rows 0..t, and of the
 * n_comp_tok[t] compressed rows either all (n_sel_tok[t] == n_comp_tok[t]) or
 * the n_sel_tok[t] listed at sel + t * sel_stride (device). Writes list t at
 * lists + t * list_stride (device int32, relative to layers[il].row_base: the
 * row_idx / row_base form of ds4hip_flash_attn_decode_fp8) and its length to
 * counts_out[t] (host). n_tok <= DS4HIP_CHUNK_MAX. */
int ds4hip_session_chunk_rows(const ds4hip_session_state *s, int il, int p0, int n_tok,
                              const int *n_comp_tok, const int *n_sel_tok, const int32_t *sel,
                              int sel_stride, int32_t *lists, int list_stride, long long *counts_out,
                              void *stream);

/* Host form of ds4hip_session_chunk_rows (same lists and checks): sel and
 * lists in host memory, no device access, so s may come from
 * ds4hip_session_state_describe with layer il's n_raw / raw_head set. For a
 * caller that stages the lists with its own copies. */
int ds4hip_session_chunk_rows_host(const ds4hip_session_state *s, int il, int p0, int n_tok,
                                   const int *n_comp_tok, const int *n_sel_tok, const int32_t *sel,
                                   int sel_stride, int32_t *lists, int list_stride,
                                   long long *counts_out);

/* ---- disk format of the FP8 session (cuda/kv_persist.cuh:6-37, adapted) ---------- */

/* One file holds the whole session: the header, then per layer its meta and
 * payload, then the trailer. Every buffer is written at full capacity, so a
 * load is a straight host-to-device copy and the restored arena is
 * byte-identical to the saved one:
 *
 *   [ ds4hip_kvc_header ]                           4096 B
 *   for il in 0..42:
 *     [ ds4hip_kvc_layer_meta ]                     64 B
 *     [ codes  (cap_comp + cap_raw) x 448 B ]       the layer's FP8 rows
 *     [ sexp   (cap_comp + cap_raw) x 8 B ]
 *     [ tail   (cap_comp + cap_raw) x 128 B ]       f16
 *     [ row_list (cap_raw + cap_comp) x 4 B ]
 *     if compress_ratio:  [ attn_state_kv ] [ attn_state_score ]   fp32 cells
 *     if has_indexer:     [ index_comp_kv cap_comp x 128 x 4 B ]
 *                         [ index_state_kv ] [ index_state_score ]
 *   [ trailer "DS4HIP01" ]
 *
 * The reference's file also carries the hyper-connection residual, which is
 * not part of this session (see ds4hip_session_state). */
#define DS4HIP_KVC_MAGIC "DS4HIPK8"   /* 8 bytes, no NUL */
#define DS4HIP_KVC_TRAILER "DS4HIP01" /* 8 bytes, no NUL */
#define DS4HIP_KVC_VERSION 1u
#define DS4HIP_KVC_MAX_TOKENS_HDR 64

typedef struct ds4hip_kvc_header {
    char magic[8];
    uint32_t version;
    uint32_t n_layer;
    uint32_t max_context;
    uint32_t pos;
    uint32_t n_tokens_processed;
    uint32_t n_prompt_tokens; /* valid entries of prompt_token_ids */
    uint32_t cap_raw;
    uint32_t row_codes;       /* 448 */
    uint32_t row_sexp;        /* 8 */
    uint32_t row_tail;        /* 64 (f16 elements) */
    uint64_t n_cache_rows;
    int32_t prompt_token_ids[DS4HIP_KVC_MAX_TOKENS_HDR];
    uint8_t pad[4096 - 56 - 4 * DS4HIP_KVC_MAX_TOKENS_HDR];
} ds4hip_kvc_header;

typedef struct ds4hip_kvc_layer_meta {
    int32_t il;
    int32_t compress_ratio;
    int32_t has_indexer;
    int32_t cap_raw;
    int32_t cap_comp;
    int32_t n_raw;
    int32_t raw_head;
    int32_t n_comp;
    int32_t n_index_comp;
    int32_t reserved0;
    int64_t row_base;
    uint64_t bytes_after; /* payload bytes of this layer (checked on load) */
    uint64_t reserved[1];
} ds4hip_kvc_layer_meta;

/* Writes the session to path (cuda/kv_persist.cuh:97-100): synchronizes the
 * device, then copies each buffer through one host bounce buffer. At most the
 * first 64 prompt token ids are stored (n_tokens may be 0 with NULL ids).
 * Returns 0, or -1 on any error (the reference's convention); the detailed
 * status (-22 arguments, -5 I/O, -1000 - hipError_t) is kept for
 * ds4hip_get_last_error. */
int ds4hip_session_save_to_disk(const ds4hip_session_state *s, const int32_t *prompt_token_ids,
                                int n_tokens, const char *path);

/* Restores a saved session into s_out, which must come from
 * ds4hip_session_state_alloc with the file's max_context
 * (cuda/kv_persist.cuh:102-127): header and every layer meta are checked
 * against s_out's geometry before its buffers are written; the counters, pos
 * and n_tokens_processed are set from the file. out_pos / out_n_tokens may be
 * NULL. Returns 0 or -1 as ds4hip_session_save_to_disk; after a failure past
 * the header check s_out is indeterminate (reset it before reuse). */
int ds4hip_session_load_from_disk(ds4hip_session_state *s_out, const char *path, int *out_pos,
                                  int *out_n_tokens);

/* ---- import of the reference's session files ---------------------------------------
 *
 * The reference saves its fp32 session as a "DS4CUDAK" file
 * (cuda/kv_persist.cuh:6-37,57-88): a header written as its struct (360
 * bytes: magic, version 1, n_layer 43, max_context, pos, n_tokens_processed,
 * n_prompt_tokens, cap_raw, a reserved word, 64 prompt token ids, 8 reserved
 * words), then per layer a 64-byte meta (il, compress_ratio, has_indexer,
 * cap_raw, cap_comp, n_raw, n_comp, n_index_comp, payload bytes) and the
 * layer's buffers at full capacity (raw_kv fp32 [cap_raw][512]; on compressed
 * layers comp_kv [cap_comp][512], attn_state_kv and attn_state_score; on
 * indexer layers index_comp_kv [cap_comp][128], index_state_kv and
 * index_state_score), then residual_hc (4 x 4096 fp32) and the trailer
 * "DS4CUDA1". */
typedef struct ds4hip_ds4cudak_info {
    int max_context;
    int pos;
    int n_tokens_processed;
    int cap_raw;
    int n_prompt_tokens;
    int32_t prompt_token_ids[DS4HIP_KVC_MAX_TOKENS_HDR];
    int n_raw[DS4HIP_N_LAYER];
    int n_comp[DS4HIP_N_LAYER];
    int n_index_comp[DS4HIP_N_LAYER];
    long long file_bytes;
} ds4hip_ds4cudak_info;

/* Reads and checks a reference session file on the host (no device work):
 * header, every layer meta against the geometry the header's max_context
 * gives, payload sizes, trailer and file length. Fills *info. Returns 0, or
 * -1 with -22 (format or geometry) / -5 (I/O, truncation) kept for
 * ds4hip_get_last_error. (No counterpart in the reference.) */
int ds4hip_ds4cudak_probe(const char *path, ds4hip_ds4cudak_info *info);

/* Loads a reference session file into an FP8 session of the same
 * max_context (no counterpart in the reference; the bridge from its fp32
 * files). The session is reset first. Window rows: raw_kv row i of a layer
 * holds position base + i, base = P - n_raw with P the header's pos, or
 * n_tokens_processed when pos is smaller than n_raw, or n_raw when both are;
 * it is quantized into ring slot (base + i) % cap_raw and raw_head becomes
 * (base + n_raw) % cap_raw. Compressed rows 0..n_comp-1 are quantized into
 * the layer's compressed rows; compressor states, indexer keys and indexer
 * states are copied as they are (the same layouts); residual_hc belongs to
 * the rest of the layer and is skipped. pos and n_tokens_processed come from
 * the header. Returns 0 or -1 as ds4hip_session_load_from_disk (the detail in
 * ds4hip_get_last_error); after a failure past the probe the session is
 * indeterminate (reset it). Synchronizes the device. */
int ds4hip_session_import_ds4cudak(ds4hip_session_state *s, const char *path, int *out_pos,
                                   int *out_n_tokens);

/* Writes the session as a reference session file that the reference's
 * ds4_session_save/load format describes (no counterpart in the reference;
 * the way back from the FP8 session). Window rows are written oldest first
 * (ring slot (raw_head - n_raw + i) % cap_raw as raw row i), dequantized and
 * f16-rounded as the reference's window holds them; compressed rows are
 * dequantized (their RoPE tail is the cache's f16 value); compressor and
 * indexer state are copied; residual_hc, which this session does not hold,
 * is written as zeros. At most the first 64 prompt token ids are stored.
 * Returns 0 or -1 as ds4hip_session_save_to_disk. Synchronizes the device. */
int ds4hip_session_export_ds4cudak(const ds4hip_session_state *s, const int32_t *prompt_token_ids,
                                   int n_tokens, const char *path);

#ifdef __cplusplus
}
#endif

#endif /* DS4HIP_SESSION_H */
