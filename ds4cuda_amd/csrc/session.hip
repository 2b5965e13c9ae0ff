// session.hip — KV push / SWA eviction and the per-session KV arena.
//
// Two forms:
//  * The reference's fp32 row layout (ds4hip_swa_push_f32 / ds4hip_comp_push_f32):
//    the raw sliding window is a linear array, oldest row first; when it is full
//    the rows move down by one and the new row goes last (memmove semantics,
//    cuda/forward_layer.cu:159-190,941-972); every stored element is
//    f16-rounded. Compressed rows append with no eviction; a full cache is an
//    error (cuda/forward_layer.cu:1021-1034).
//  * The FP8 session (ds4hip_session_state_*): every layer owns a range of FP8
//    cache rows, compressed rows first ([0, cap_comp)) then a 128-row SWA ring
//    ([cap_comp, cap_comp + 128)). The ring is a true ring: a push overwrites
//    the oldest slot, so eviction costs one row write instead of a 127-row move.
//    Attention is order-free over its rows, so the window's set of rows is all
//    that matters; a constant per-layer row list (ring slots in reverse, then
//    the compressed rows in order) makes "the n_raw valid ring rows followed by
//    the first n_comp compressed rows" one contiguous slice of that list, which
//    the decode kernel reads as its row-index array.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ds4hip_session.h"
#include "ds4hip_common.h"
#include "step_bodies.h"

using namespace ds4hip;

namespace {

constexpr int kShiftChunk = 16;

// f16 round trip of one fp32 value (round to nearest even), as stored rows are.
__device__ inline float f16_round(float v) { return __half2float(__float2half(v)); }

// Moves rows [1, n_rows) of a [n_rows][head_dim] fp32 array down by one, in
// place, f16-rounding on the way. One thread owns one column and walks it from
// low to high rows; each chunk of kShiftChunk rows is loaded before any of it
// is stored, and only rows at or below the last loaded one are stored.
__global__ __launch_bounds__(256) void swa_shift_kernel(float *__restrict__ base, int head_dim,
                                                        int n_rows) {
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= head_dim) return;
    float *p = base + col;
    for (int r0 = 0; r0 + 1 < n_rows; r0 += kShiftChunk) {
        float v[kShiftChunk];
#pragma unroll
        for (int i = 0; i < kShiftChunk; ++i)
            if (r0 + 1 + i < n_rows) v[i] = p[(size_t)(r0 + 1 + i) * head_dim];
#pragma unroll
        for (int i = 0; i < kShiftChunk; ++i)
            if (r0 + 1 + i < n_rows) p[(size_t)(r0 + i) * head_dim] = f16_round(v[i]);
    }
}

__global__ __launch_bounds__(256) void row_write_kernel(float *__restrict__ dst,
                                                        const float *__restrict__ src, int n,
                                                        int round_f16) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = round_f16 ? f16_round(src[i]) : src[i];
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float *__restrict__ p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *__restrict__ p, size_t n,
                                                       uint32_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Row list of one layer: [cap_raw - 1 - k + cap_comp for k < cap_raw] then
// [c for c < cap_comp] (row numbers relative to the layer's first row).
__global__ __launch_bounds__(256) void row_list_kernel(int32_t *__restrict__ list, int cap_raw,
                                                       int cap_comp) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < cap_raw) list[i] = cap_comp + cap_raw - 1 - i;
    else if (i < cap_raw + cap_comp) list[i] = i - cap_raw;
}

inline unsigned fill_grid(size_t n) {
    size_t g = (n + 255) / 256;
    return (unsigned)(g < 2048 ? (g ? g : 1) : 2048);
}

int layer_ratio(int il) { return il < 2 ? 0 : ((il & 1) == 0 ? 4 : 128); }

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

struct Plan {
    int cap_raw;
    int cap_comp[DS4HIP_N_LAYER];
    long long row_base[DS4HIP_N_LAYER];
    long long n_rows;
    size_t off_codes, off_sexp, off_tail, off_lists, off_state, bytes;
    size_t list_off[DS4HIP_N_LAYER];
    size_t state_off[DS4HIP_N_LAYER];  // attn kv, attn score, idx comp, idx kv, idx score
};

size_t attn_state_cells(int ratio) {
    const int coff = ratio == 4 ? 2 : 1;
    return (size_t)coff * ratio * coff * DS4HIP_HEAD_DIM;
}
size_t index_state_cells() { return (size_t)2 * 4 * 2 * DS4HIP_INDEXER_HEAD_DIM; }

size_t layer_state_bytes(int ratio, int cap_comp) {
    if (ratio == 0) return 0;
    size_t b = 2 * align256(attn_state_cells(ratio) * 4);
    if (ratio == 4)
        b += align256((size_t)cap_comp * DS4HIP_INDEXER_HEAD_DIM * 4) +
             2 * align256(index_state_cells() * 4);
    return b;
}

Plan make_plan(int max_context) {
    Plan P{};
    P.cap_raw = max_context < DS4HIP_N_SWA ? max_context : DS4HIP_N_SWA;
    long long rows = 0;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        const int r = layer_ratio(il);
        P.cap_comp[il] = r ? max_context / r + 2 : 0;  // cuda/session_state.cu:137
        P.row_base[il] = rows;
        rows += P.cap_comp[il] + P.cap_raw;
    }
    P.n_rows = rows;
    // the layers' rows, then DS4HIP_CHUNK_MAX staging rows for a prefill chunk
    const long long all_rows = rows + DS4HIP_CHUNK_MAX;
    size_t off = 0;
    P.off_codes = off;
    off += align256((size_t)all_rows * DS4HIP_FP8_CODES);
    P.off_sexp = off;
    off += align256((size_t)all_rows * DS4HIP_FP8_SEXP);
    P.off_tail = off;
    off += align256((size_t)all_rows * DS4HIP_FP8_TAIL * 2);
    P.off_lists = off;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        P.list_off[il] = off;
        off += align256((size_t)(P.cap_raw + P.cap_comp[il]) * 4);
    }
    P.off_state = off;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        P.state_off[il] = off;
        off += layer_state_bytes(layer_ratio(il), P.cap_comp[il]);
    }
    P.bytes = off;
    return P;
}

int fill(float *p, size_t n, float v, hipStream_t st) {
    if (!p || !n) return 0;
    hipLaunchKernelGGL(fill_f32_kernel, dim3(fill_grid(n)), dim3(256), 0, st, p, n, v);
    return hip_status(hipGetLastError());
}

int init_buffers(ds4hip_session_state *s, hipStream_t st) {
    s->pos = 0;
    s->n_tokens_processed = 0;
    int rc = 0;
    // Cache rows are zeroed so a stale row never holds NaN bit patterns.
    const size_t cache_words = (s->codes_bytes + 3) / 4;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(fill_grid(cache_words)), dim3(256), 0, st,
                       (uint32_t *)s->arena_base, cache_words, 0u);
    if ((rc = hip_status(hipGetLastError()))) return rc;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        ds4hip_layer_state *L = &s->layers[il];
        L->n_raw = L->raw_head = L->n_comp = L->n_index_comp = 0;
        // The compressed part may hold an indexer selection from the last sequence.
        const int nl = L->cap_raw + L->cap_comp;
        hipLaunchKernelGGL(row_list_kernel, dim3((nl + 255) / 256), dim3(256), 0, st, L->row_list,
                           L->cap_raw, L->cap_comp);
        if ((rc = hip_status(hipGetLastError()))) return rc;
        if (!L->compress_ratio) continue;
        const size_t cells = attn_state_cells(L->compress_ratio);
        if ((rc = fill(L->attn_state_kv, cells, 0.f, st))) return rc;
        if ((rc = fill(L->attn_state_score, cells, -INFINITY, st))) return rc;
        if (L->has_indexer) {
            if ((rc = fill(L->index_comp_kv, (size_t)L->cap_comp * DS4HIP_INDEXER_HEAD_DIM, 0.f,
                           st)))
                return rc;
            if ((rc = fill(L->index_state_kv, index_state_cells(), 0.f, st))) return rc;
            if ((rc = fill(L->index_state_score, index_state_cells(), -INFINITY, st))) return rc;
        }
    }
    return 0;
}

bool layer_ok(const ds4hip_session_state *s, int il) {
    return s && s->arena_base && il >= 0 && il < DS4HIP_N_LAYER;
}

}  // namespace

// ---- reference fp32 layout ------------------------------------------------------------------

extern "C" int ds4hip_swa_push_f32(float *raw_kv, int *n_raw_host, int cap_raw,
                                   const float *kv_cur, int head_dim, void *stream) {
    if (!raw_kv || !n_raw_host || !kv_cur || cap_raw <= 0 || head_dim <= 0 || *n_raw_host < 0 ||
        *n_raw_host > cap_raw)
        return ds4hip_set_last_error(kEINVAL);
    const hipStream_t st = (hipStream_t)stream;
    int slot = *n_raw_host;
    if (slot == cap_raw) {
        hipLaunchKernelGGL(swa_shift_kernel, dim3((head_dim + 255) / 256), dim3(256), 0, st,
                           raw_kv, head_dim, cap_raw);
        slot = cap_raw - 1;
    }
    hipLaunchKernelGGL(row_write_kernel, dim3((head_dim + 255) / 256), dim3(256), 0, st,
                       raw_kv + (size_t)slot * head_dim, kv_cur, head_dim, 1);
    const int rc = ds4hip_set_last_error(hip_status(hipGetLastError()));
    if (!rc) *n_raw_host = slot + 1;
    return rc;
}

extern "C" int ds4hip_comp_push_f32(float *comp_kv, int *n_comp_host, int cap_comp,
                                    const float *row, int head_dim, void *stream) {
    if (!comp_kv || !n_comp_host || !row || head_dim <= 0 || *n_comp_host < 0)
        return ds4hip_set_last_error(kEINVAL);
    if (*n_comp_host >= cap_comp) return ds4hip_set_last_error(DS4HIP_ENOSPC);
    hipLaunchKernelGGL(row_write_kernel, dim3((head_dim + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, comp_kv + (size_t)*n_comp_host * head_dim, row,
                       head_dim, 0);
    const int rc = ds4hip_set_last_error(hip_status(hipGetLastError()));
    if (!rc) ++*n_comp_host;
    return rc;
}

// ---- FP8 session --------------------------------------------------------------------------

extern "C" size_t ds4hip_session_state_arena_bytes(int max_context) {
    if (max_context <= 0) return 0;
    return make_plan(max_context).bytes;
}

extern "C" int ds4hip_session_state_describe(ds4hip_session_state *out, int max_context) {
    if (!out || max_context <= 0) return ds4hip_set_last_error(kEINVAL);
    std::memset(out, 0, sizeof(*out));
    const Plan P = make_plan(max_context);
    out->max_context = max_context;
    out->arena_bytes = P.bytes;
    out->n_cache_rows = P.n_rows;
    out->codes_bytes = P.off_lists;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        ds4hip_layer_state *L = &out->layers[il];
        const int r = layer_ratio(il);
        L->il = il;
        L->compress_ratio = r;
        L->has_indexer = r == 4;
        L->cap_raw = P.cap_raw;
        L->cap_comp = P.cap_comp[il];
        L->row_base = P.row_base[il];
    }
    return 0;
}

extern "C" int ds4hip_session_state_alloc(ds4hip_session_state *out, int max_context) {
    if (!out || max_context <= 0) return ds4hip_set_last_error(kEINVAL);
    std::memset(out, 0, sizeof(*out));
    const Plan P = make_plan(max_context);
    void *base = nullptr;
    int rc = hip_status(hipMalloc(&base, P.bytes));
    if (rc) return ds4hip_set_last_error(rc);
    uint8_t *b = (uint8_t *)base;
    out->max_context = max_context;
    out->arena_base = base;
    out->arena_bytes = P.bytes;
    out->codes = b + P.off_codes;
    out->sexp = (int8_t *)(b + P.off_sexp);
    out->tail = (uint16_t *)(b + P.off_tail);
    out->n_cache_rows = P.n_rows;
    out->codes_bytes = P.off_lists;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        ds4hip_layer_state *L = &out->layers[il];
        const int r = layer_ratio(il);
        L->il = il;
        L->compress_ratio = r;
        L->has_indexer = r == 4;
        L->cap_raw = P.cap_raw;
        L->cap_comp = P.cap_comp[il];
        L->row_base = P.row_base[il];
        L->row_list = (int32_t *)(b + P.list_off[il]);
        if (!r) continue;
        uint8_t *p = b + P.state_off[il];
        const size_t sb = align256(attn_state_cells(r) * 4);
        L->attn_state_kv = (float *)p;
        L->attn_state_score = (float *)(p + sb);
        p += 2 * sb;
        if (r == 4) {
            L->index_comp_kv = (float *)p;
            p += align256((size_t)L->cap_comp * DS4HIP_INDEXER_HEAD_DIM * 4);
            const size_t ib = align256(index_state_cells() * 4);
            L->index_state_kv = (float *)p;
            L->index_state_score = (float *)(p + ib);
        }
    }
    rc = hip_status(hipGetLastError());
    if (!rc) rc = init_buffers(out, 0);
    if (!rc) rc = hip_status(hipStreamSynchronize(0));
    if (rc) {
        (void)hipFree(base);
        std::memset(out, 0, sizeof(*out));
        return ds4hip_set_last_error(rc);
    }
    return 0;
}

extern "C" int ds4hip_session_state_free(ds4hip_session_state *s) {
    if (!s) return 0;
    int rc = 0;
    if (s->arena_base) rc = hip_status(hipFree(s->arena_base));
    std::memset(s, 0, sizeof(*s));
    return rc ? ds4hip_set_last_error(rc) : 0;
}

extern "C" int ds4hip_session_state_reset(ds4hip_session_state *s, void *stream) {
    if (!s || !s->arena_base) return ds4hip_set_last_error(kEINVAL);
    return ds4hip_set_last_error(init_buffers(s, (hipStream_t)stream));
}

namespace {
// the ring row of the next raw push, and the counters after it
long long raw_row(const ds4hip_layer_state *L) { return L->row_base + L->cap_comp + L->raw_head; }
void advance_raw(ds4hip_layer_state *L) {
    L->raw_head = (L->raw_head + 1) % L->cap_raw;
    if (L->n_raw < L->cap_raw) ++L->n_raw;
}
}  // namespace

extern "C" int ds4hip_session_push_raw(ds4hip_session_state *s, int il, const float *kv_cur,
                                       void *stream) {
    if (!layer_ok(s, il) || !kv_cur) return ds4hip_set_last_error(kEINVAL);
    ds4hip_layer_state *L = &s->layers[il];
    const int rc = ds4hip_fp8_kv_quantize_append(kv_cur, 1, DS4HIP_HEAD_DIM, DS4HIP_N_ROT, s->codes,
                                                 s->sexp, s->tail, raw_row(L), nullptr, stream);
    if (rc) return rc;
    advance_raw(L);
    return 0;
}

extern "C" int ds4hip_session_claim_raw_row(ds4hip_session_state *s, int il, long long *row_out) {
    if (!layer_ok(s, il) || !row_out) return ds4hip_set_last_error(kEINVAL);
    ds4hip_layer_state *L = &s->layers[il];
    *row_out = raw_row(L);
    advance_raw(L);
    return 0;
}

extern "C" int ds4hip_session_push_comp(ds4hip_session_state *s, int il, const float *row,
                                        void *stream) {
    if (!layer_ok(s, il) || !row) return ds4hip_set_last_error(kEINVAL);
    ds4hip_layer_state *L = &s->layers[il];
    if (!L->compress_ratio) return ds4hip_set_last_error(kEINVAL);
    if (L->n_comp >= L->cap_comp) return ds4hip_set_last_error(DS4HIP_ENOSPC);
    const int rc = ds4hip_fp8_kv_quantize_append(row, 1, DS4HIP_HEAD_DIM, DS4HIP_N_ROT, s->codes,
                                                 s->sexp, s->tail, L->row_base + L->n_comp,
                                                 nullptr, stream);
    if (!rc) ++L->n_comp;
    return rc;
}

extern "C" int ds4hip_session_push_index_comp(ds4hip_session_state *s, int il, const float *row,
                                              void *stream) {
    if (!layer_ok(s, il) || !row) return ds4hip_set_last_error(kEINVAL);
    ds4hip_layer_state *L = &s->layers[il];
    if (!L->has_indexer) return ds4hip_set_last_error(kEINVAL);
    return ds4hip_comp_push_f32(L->index_comp_kv, &L->n_index_comp, L->cap_comp, row,
                                DS4HIP_INDEXER_HEAD_DIM, stream);
}

extern "C" int ds4hip_session_layer_rows(const ds4hip_session_state *s, int il, int n_selected,
                                         const int32_t **row_idx, long long *n_rows,
                                         int32_t **selected_out) {
    if (!layer_ok(s, il) || !row_idx || !n_rows) return ds4hip_set_last_error(kEINVAL);
    const ds4hip_layer_state *L = &s->layers[il];
    const int n_sel = n_selected < 0 ? L->n_comp : n_selected;
    if (n_sel > L->cap_comp) return ds4hip_set_last_error(kEINVAL);
    *row_idx = L->row_list + (L->cap_raw - L->n_raw);
    *n_rows = (long long)L->n_raw + n_sel;
    if (selected_out) *selected_out = L->row_list + L->cap_raw;
    return 0;
}

extern "C" int ds4hip_session_set_selection(ds4hip_session_state *s, int il, const int32_t *sel, int n,
                                            void *stream) {
    if (!layer_ok(s, il) || n < 0 || (n && !sel)) return ds4hip_set_last_error(kEINVAL);
    const ds4hip_layer_state *L = &s->layers[il];
    if (n > L->cap_comp) return ds4hip_set_last_error(kEINVAL);
    if (!n) return 0;
    return ds4hip_set_last_error(hip_status(hipMemcpyAsync(L->row_list + L->cap_raw, sel, (size_t)n * 4,
                                                           hipMemcpyDeviceToDevice, (hipStream_t)stream)));
}

namespace {
// dst[dst_rows[r]][:] = src[r][:] for r < n_rows; one 64-lane wave per row,
// 16-byte moves (width % 4 == 0).
__global__ __launch_bounds__(256) void rows_scatter_kernel(const float *__restrict__ src,
                                                           int n_rows, int width,
                                                           float *__restrict__ dst,
                                                           const long long *__restrict__ dst_rows) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= n_rows) return;
    row_copy_body(src, r, width, dst, dst_rows, threadIdx.x & 63);
}
}  // namespace

extern "C" int ds4hip_rows_scatter_f32(const float *src, int n_rows, int width, float *dst,
                                       const long long *dst_rows, void *stream) {
    if (n_rows < 0 || width <= 0 || width % 4 != 0 || (n_rows && (!src || !dst || !dst_rows)))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    hipLaunchKernelGGL(rows_scatter_kernel, dim3((n_rows + 3) / 4), dim3(256), 0,
                       (hipStream_t)stream, src, n_rows, width, dst, dst_rows);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

// ---- disk persistence of the FP8 session (cuda/kv_persist.cu) ----------------------------
//
// Every layer's payload is a list of (device pointer, bytes) buffers, written
// and read in the same order through one host bounce buffer sized to the
// largest of them. The device is synchronized before a save (the copies must
// see the finished state) and after a load (the caller sees the buffers
// filled on return).

namespace {

static_assert(sizeof(ds4hip_kvc_header) == 4096, "header is 4 KiB");
static_assert(sizeof(ds4hip_kvc_layer_meta) == 64, "layer meta is 64 B");

constexpr int kEIO = -5;

struct Buf {
    void *p;
    size_t bytes;
};

// The buffers of layer L in file order; returns their count.
int layer_bufs(const ds4hip_session_state *s, const ds4hip_layer_state *L, Buf (&b)[9]) {
    const size_t rows = (size_t)L->cap_comp + L->cap_raw;
    int n = 0;
    b[n++] = {s->codes + (size_t)L->row_base * DS4HIP_FP8_CODES, rows * DS4HIP_FP8_CODES};
    b[n++] = {s->sexp + (size_t)L->row_base * DS4HIP_FP8_SEXP, rows * DS4HIP_FP8_SEXP};
    b[n++] = {s->tail + (size_t)L->row_base * DS4HIP_FP8_TAIL, rows * DS4HIP_FP8_TAIL * 2};
    b[n++] = {L->row_list, rows * 4};
    if (L->compress_ratio) {
        const size_t sb = attn_state_cells(L->compress_ratio) * 4;
        b[n++] = {L->attn_state_kv, sb};
        b[n++] = {L->attn_state_score, sb};
    }
    if (L->has_indexer) {
        b[n++] = {L->index_comp_kv, (size_t)L->cap_comp * DS4HIP_INDEXER_HEAD_DIM * 4};
        b[n++] = {L->index_state_kv, index_state_cells() * 4};
        b[n++] = {L->index_state_score, index_state_cells() * 4};
    }
    return n;
}

uint64_t layer_payload(const ds4hip_session_state *s, const ds4hip_layer_state *L, size_t *max_buf) {
    Buf b[9];
    const int n = layer_bufs(s, L, b);
    uint64_t t = 0;
    for (int i = 0; i < n; ++i) {
        t += b[i].bytes;
        if (max_buf && b[i].bytes > *max_buf) *max_buf = b[i].bytes;
    }
    return t;
}

// Geometry of an allocated session matches what ds4hip_session_state_alloc
// builds for its max_context (a struct edited by hand is refused).
bool session_ok(const ds4hip_session_state *s) {
    if (!s || !s->arena_base || s->max_context <= 0) return false;
    const Plan P = make_plan(s->max_context);
    if (s->n_cache_rows != P.n_rows) return false;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        const ds4hip_layer_state &L = s->layers[il];
        if (L.il != il || L.compress_ratio != layer_ratio(il) || L.cap_raw != P.cap_raw ||
            L.cap_comp != P.cap_comp[il] || L.row_base != P.row_base[il] || !L.row_list)
            return false;
    }
    return true;
}

struct File {
    FILE *f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

int fail(int code) {
    ds4hip_set_last_error(code);
    return -1;
}

}  // namespace

extern "C" int ds4hip_session_save_to_disk(const ds4hip_session_state *s, const int32_t *prompt_token_ids,
                                           int n_tokens, const char *path) {
    if (!path || !session_ok(s) || n_tokens < 0 || (n_tokens > 0 && !prompt_token_ids)) return fail(kEINVAL);
    int rc = hip_status(hipDeviceSynchronize());
    if (rc) return fail(rc);
    ds4hip_kvc_header h;
    std::memset(&h, 0, sizeof(h));
    std::memcpy(h.magic, DS4HIP_KVC_MAGIC, 8);
    h.version = DS4HIP_KVC_VERSION;
    h.n_layer = DS4HIP_N_LAYER;
    h.max_context = (uint32_t)s->max_context;
    h.pos = (uint32_t)s->pos;
    h.n_tokens_processed = (uint32_t)s->n_tokens_processed;
    h.n_prompt_tokens = (uint32_t)(n_tokens < DS4HIP_KVC_MAX_TOKENS_HDR ? n_tokens : DS4HIP_KVC_MAX_TOKENS_HDR);
    for (uint32_t i = 0; i < h.n_prompt_tokens; ++i) h.prompt_token_ids[i] = prompt_token_ids[i];
    h.cap_raw = (uint32_t)s->layers[0].cap_raw;
    h.row_codes = DS4HIP_FP8_CODES;
    h.row_sexp = DS4HIP_FP8_SEXP;
    h.row_tail = DS4HIP_FP8_TAIL;
    h.n_cache_rows = (uint64_t)s->n_cache_rows;
    size_t max_buf = 0;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) layer_payload(s, &s->layers[il], &max_buf);
    std::vector<uint8_t> bounce(max_buf);
    File out;
    out.f = std::fopen(path, "wb");   // truncates: a failed save leaves no stale payload behind
    if (!out.f) return fail(kEIO);
    if (std::fwrite(&h, sizeof(h), 1, out.f) != 1) return fail(kEIO);
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        const ds4hip_layer_state &L = s->layers[il];
        ds4hip_kvc_layer_meta m;
        std::memset(&m, 0, sizeof(m));
        m.il = il;
        m.compress_ratio = L.compress_ratio;
        m.has_indexer = L.has_indexer;
        m.cap_raw = L.cap_raw;
        m.cap_comp = L.cap_comp;
        m.n_raw = L.n_raw;
        m.raw_head = L.raw_head;
        m.n_comp = L.n_comp;
        m.n_index_comp = L.n_index_comp;
        m.row_base = L.row_base;
        m.bytes_after = layer_payload(s, &L, nullptr);
        if (std::fwrite(&m, sizeof(m), 1, out.f) != 1) return fail(kEIO);
        Buf b[9];
        const int nb = layer_bufs(s, &L, b);
        for (int i = 0; i < nb; ++i) {
            rc = hip_status(hipMemcpy(bounce.data(), b[i].p, b[i].bytes, hipMemcpyDeviceToHost));
            if (rc) return fail(rc);
            if (std::fwrite(bounce.data(), 1, b[i].bytes, out.f) != b[i].bytes) return fail(kEIO);
        }
    }
    if (std::fwrite(DS4HIP_KVC_TRAILER, 1, 8, out.f) != 8) return fail(kEIO);
    const int cr = std::fclose(out.f);
    out.f = nullptr;
    return cr == 0 ? 0 : fail(kEIO);
}

extern "C" int ds4hip_session_load_from_disk(ds4hip_session_state *s_out, const char *path, int *out_pos,
                                             int *out_n_tokens) {
    if (!path || !session_ok(s_out)) return fail(kEINVAL);
    File in;
    in.f = std::fopen(path, "rb");
    if (!in.f) return fail(kEIO);
    ds4hip_kvc_header h;
    if (std::fread(&h, sizeof(h), 1, in.f) != 1) return fail(kEIO);
    if (std::memcmp(h.magic, DS4HIP_KVC_MAGIC, 8) != 0 || h.version != DS4HIP_KVC_VERSION ||
        h.n_layer != DS4HIP_N_LAYER || h.max_context != (uint32_t)s_out->max_context ||
        h.cap_raw != (uint32_t)s_out->layers[0].cap_raw || h.row_codes != DS4HIP_FP8_CODES ||
        h.row_sexp != DS4HIP_FP8_SEXP || h.row_tail != DS4HIP_FP8_TAIL ||
        h.n_cache_rows != (uint64_t)s_out->n_cache_rows || h.pos > h.max_context ||
        h.n_prompt_tokens > DS4HIP_KVC_MAX_TOKENS_HDR)
        return fail(kEINVAL);
    size_t max_buf = 0;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) layer_payload(s_out, &s_out->layers[il], &max_buf);
    std::vector<uint8_t> bounce(max_buf);
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        ds4hip_layer_state &L = s_out->layers[il];
        ds4hip_kvc_layer_meta m;
        if (std::fread(&m, sizeof(m), 1, in.f) != 1) return fail(kEIO);
        if (m.il != il || m.compress_ratio != L.compress_ratio || m.has_indexer != L.has_indexer ||
            m.cap_raw != L.cap_raw || m.cap_comp != L.cap_comp || m.row_base != L.row_base ||
            m.bytes_after != layer_payload(s_out, &L, nullptr) || m.n_raw < 0 || m.n_raw > L.cap_raw ||
            m.raw_head < 0 || m.raw_head >= (L.cap_raw ? L.cap_raw : 1) || m.n_comp < 0 ||
            m.n_comp > L.cap_comp || m.n_index_comp < 0 || m.n_index_comp > L.cap_comp ||
            (!L.compress_ratio && m.n_comp) || (!L.has_indexer && m.n_index_comp))
            return fail(kEINVAL);
        Buf b[9];
        const int nb = layer_bufs(s_out, &L, b);
        for (int i = 0; i < nb; ++i) {
            if (std::fread(bounce.data(), 1, b[i].bytes, in.f) != b[i].bytes) return fail(kEIO);
            const int rc = hip_status(hipMemcpy(b[i].p, bounce.data(), b[i].bytes, hipMemcpyHostToDevice));
            if (rc) return fail(rc);
        }
        L.n_raw = m.n_raw;
        L.raw_head = m.raw_head;
        L.n_comp = m.n_comp;
        L.n_index_comp = m.n_index_comp;
    }
    char tr[8];
    if (std::fread(tr, 1, 8, in.f) != 8 || std::memcmp(tr, DS4HIP_KVC_TRAILER, 8) != 0) return fail(kEINVAL);
    const int rc = hip_status(hipDeviceSynchronize());
    if (rc) return fail(rc);
    s_out->pos = (int)h.pos;
    s_out->n_tokens_processed = (int)h.n_tokens_processed;
    if (out_pos) *out_pos = s_out->pos;
    if (out_n_tokens) *out_n_tokens = s_out->n_tokens_processed;
    return 0;
}

// ---- row lists of a prefill chunk -----------------------------------------------------------
namespace {
struct ChunkTok {   // per token: compressed rows visible, and how many of them it attends
    int n_comp[DS4HIP_CHUNK_MAX];
    int n_sel[DS4HIP_CHUNK_MAX];
};
struct ChunkGeom {
    int p0, cap_raw, cap_comp, stage_rel;
};

// Token t (position p0 + t) sees the window positions max(0, p0 + t -
// cap_raw + 1) .. p0 + t: those below p0 in the ring (position x in slot
// x % cap_raw, after the compressed rows), the others in the staging rows.
__host__ __device__ inline int chunk_first(const ChunkGeom &G, int t) {
    const int f = G.p0 + t - G.cap_raw + 1;
    return f > 0 ? f : 0;
}
__host__ __device__ inline int chunk_n_ring(const ChunkGeom &G, int t) {
    const int f = chunk_first(G, t);
    return G.p0 > f ? G.p0 - f : 0;
}
// Entry i < chunk_n_ring + t + 1 of token t's list (relative to row_base).
__host__ __device__ inline int32_t chunk_entry(const ChunkGeom &G, int t, int i) {
    const int nr = chunk_n_ring(G, t);
    return i < nr ? G.cap_comp + (chunk_first(G, t) + i) % G.cap_raw : G.stage_rel + (i - nr);
}

// One workgroup per token t: the window rows, then the token's compressed
// rows (its selection sel[t], or all of them).
__global__ __launch_bounds__(256) void chunk_rows_kernel(int32_t *__restrict__ lists, int stride, ChunkGeom G,
                                                         ChunkTok T, const int32_t *__restrict__ sel,
                                                         int sel_stride) {
    const int t = blockIdx.x;
    int32_t *out = lists + (size_t)t * stride;
    const int n_win = chunk_n_ring(G, t) + t + 1;
    const int n_sel = T.n_sel[t];
    const bool all = n_sel == T.n_comp[t];
    for (int i = threadIdx.x; i < n_win; i += 256) out[i] = chunk_entry(G, t, i);
    for (int i = threadIdx.x; i < n_sel; i += 256)
        out[n_win + i] = all ? i : sel[(size_t)t * sel_stride + i];
}

// Checks the arguments shared by the device and host forms and fills T,
// the geometry and the counts.
int chunk_plan(const ds4hip_session_state *s, int il, int p0, int n_tok, const int *n_comp_tok,
               const int *n_sel_tok, bool have_sel, int sel_stride, int list_stride, long long *counts_out,
               ChunkTok &T, ChunkGeom &G) {
    if (!s || il < 0 || il >= DS4HIP_N_LAYER || n_tok <= 0 || n_tok > DS4HIP_CHUNK_MAX || p0 < 0 ||
        !n_comp_tok || !n_sel_tok || !counts_out || list_stride <= 0)
        return kEINVAL;
    const ds4hip_layer_state *L = &s->layers[il];
    if (L->cap_raw <= 0) return kEINVAL;
    // the chunk stays inside the session's positions, and a token's window
    // (at most cap_raw rows) can hold the chunk's own rows up to it
    if ((long long)p0 + n_tok > s->max_context || n_tok > L->cap_raw) return kEINVAL;
    // the ring holds exactly the positions < p0 (one push per position)
    if (L->n_raw != (p0 < L->cap_raw ? p0 : L->cap_raw) || L->raw_head != p0 % L->cap_raw) return kEINVAL;
    G = ChunkGeom{p0, L->cap_raw, L->cap_comp, (int)(s->n_cache_rows - L->row_base)};
    for (int t = 0; t < n_tok; ++t) {
        const bool all = n_sel_tok[t] == n_comp_tok[t];
        if (n_comp_tok[t] < 0 || n_comp_tok[t] > L->cap_comp || n_sel_tok[t] < 0 ||
            n_sel_tok[t] > n_comp_tok[t] || (!all && (!have_sel || n_sel_tok[t] > sel_stride)))
            return kEINVAL;
        counts_out[t] = (long long)chunk_n_ring(G, t) + (t + 1) + n_sel_tok[t];
        if (counts_out[t] > list_stride) return kEINVAL;
        T.n_comp[t] = n_comp_tok[t];
        T.n_sel[t] = n_sel_tok[t];
    }
    return 0;
}
}  // namespace

extern "C" int ds4hip_session_chunk_rows(const ds4hip_session_state *s, int il, int p0, int n_tok,
                                         const int *n_comp_tok, const int *n_sel_tok,
                                         const int32_t *sel, int sel_stride, int32_t *lists,
                                         int list_stride, long long *counts_out, void *stream) {
    if (!layer_ok(s, il) || !lists) return ds4hip_set_last_error(kEINVAL);
    ChunkTok T;
    ChunkGeom G;
    const int rc = chunk_plan(s, il, p0, n_tok, n_comp_tok, n_sel_tok, sel != nullptr, sel_stride, list_stride,
                              counts_out, T, G);
    if (rc) return ds4hip_set_last_error(rc);
    hipLaunchKernelGGL(chunk_rows_kernel, dim3(n_tok), dim3(256), 0, (hipStream_t)stream, lists, list_stride, G,
                       T, sel, sel_stride);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_session_chunk_rows_host(const ds4hip_session_state *s, int il, int p0, int n_tok,
                                              const int *n_comp_tok, const int *n_sel_tok,
                                              const int32_t *sel, int sel_stride, int32_t *lists,
                                              int list_stride, long long *counts_out) {
    if (!lists) return ds4hip_set_last_error(kEINVAL);
    ChunkTok T;
    ChunkGeom G;
    const int rc = chunk_plan(s, il, p0, n_tok, n_comp_tok, n_sel_tok, sel != nullptr, sel_stride, list_stride,
                              counts_out, T, G);
    if (rc) return ds4hip_set_last_error(rc);
    for (int t = 0; t < n_tok; ++t) {
        int32_t *out = lists + (size_t)t * list_stride;
        const int n_win = chunk_n_ring(G, t) + t + 1;
        const bool all = T.n_sel[t] == T.n_comp[t];
        for (int i = 0; i < n_win; ++i) out[i] = chunk_entry(G, t, i);
        for (int i = 0; i < T.n_sel[t]; ++i) out[n_win + i] = all ? i : sel[(size_t)t * sel_stride + i];
    }
    return 0;
}

// ---- import of a reference session file ----------------------------------------------------
//
// The reference writes its header and layer metas as their structs
// (cuda/kv_persist.cu:206-236,246-262; layouts at cuda/kv_persist.cuh:57-88);
// the fields are read here at their byte offsets, little-endian.
namespace {

constexpr size_t kRefHdrBytes = 360;
constexpr size_t kRefMetaBytes = 64;
constexpr size_t kRefResidualBytes = (size_t)4 * 4096 * 4;   // N_HC x N_EMBD fp32

uint32_t rd_u32(const uint8_t *p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
int32_t rd_i32(const uint8_t *p) {
    int32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint64_t rd_u64(const uint8_t *p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}

// Payload bytes of one layer in the reference file.
uint64_t ref_layer_payload(int ratio, int cap_raw, int cap_comp) {
    uint64_t b = (uint64_t)cap_raw * DS4HIP_HEAD_DIM * 4;
    if (ratio) {
        b += (uint64_t)cap_comp * DS4HIP_HEAD_DIM * 4 + 2 * attn_state_cells(ratio) * 4;
        if (ratio == 4) b += (uint64_t)cap_comp * DS4HIP_INDEXER_HEAD_DIM * 4 + 2 * index_state_cells() * 4;
    }
    return b;
}

// Reads and checks the file; fills info and each layer's payload offset.
int ref_probe(FILE *f, ds4hip_ds4cudak_info *info, long long (&payload_off)[DS4HIP_N_LAYER]) {
    uint8_t h[kRefHdrBytes];
    if (std::fread(h, 1, kRefHdrBytes, f) != kRefHdrBytes) return kEIO;
    if (std::memcmp(h, "DS4CUDAK", 8) != 0 || rd_u32(h + 8) != 1u || rd_u32(h + 12) != DS4HIP_N_LAYER)
        return kEINVAL;
    const uint32_t max_ctx = rd_u32(h + 16);
    if (max_ctx == 0 || max_ctx > (1u << 24)) return kEINVAL;
    const Plan P = make_plan((int)max_ctx);
    std::memset(info, 0, sizeof(*info));
    info->max_context = (int)max_ctx;
    info->pos = (int)rd_u32(h + 20);
    info->n_tokens_processed = (int)rd_u32(h + 24);
    info->n_prompt_tokens = (int)rd_u32(h + 28);
    info->cap_raw = (int)rd_u32(h + 32);
    if (info->cap_raw != P.cap_raw || info->n_prompt_tokens < 0 ||
        info->n_prompt_tokens > DS4HIP_KVC_MAX_TOKENS_HDR || info->pos < 0 || info->n_tokens_processed < 0)
        return kEINVAL;
    for (int i = 0; i < DS4HIP_KVC_MAX_TOKENS_HDR; ++i) info->prompt_token_ids[i] = rd_i32(h + 40 + 4 * i);
    long long off = (long long)kRefHdrBytes;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        uint8_t m[kRefMetaBytes];
        if (std::fseek(f, off, SEEK_SET) != 0 || std::fread(m, 1, kRefMetaBytes, f) != kRefMetaBytes) return kEIO;
        const int ratio = layer_ratio(il);
        const int cap_comp = P.cap_comp[il];
        const int n_raw = rd_i32(m + 20), n_comp = rd_i32(m + 24), n_idx = rd_i32(m + 28);
        const uint64_t payload = ref_layer_payload(ratio, P.cap_raw, cap_comp);
        if (rd_i32(m) != il || rd_i32(m + 4) != ratio || rd_i32(m + 8) != (ratio == 4 ? 1 : 0) ||
            rd_i32(m + 12) != P.cap_raw || rd_i32(m + 16) != cap_comp || n_raw < 0 || n_raw > P.cap_raw ||
            n_comp < 0 || n_comp > cap_comp || n_idx < 0 || n_idx > cap_comp || (!ratio && n_comp) ||
            (ratio != 4 && n_idx) || rd_u64(m + 32) != payload)
            return kEINVAL;
        info->n_raw[il] = n_raw;
        info->n_comp[il] = n_comp;
        info->n_index_comp[il] = n_idx;
        payload_off[il] = off + (long long)kRefMetaBytes;
        off = payload_off[il] + (long long)payload;
    }
    off += (long long)kRefResidualBytes;
    char tr[8];
    if (std::fseek(f, off, SEEK_SET) != 0 || std::fread(tr, 1, 8, f) != 8) return kEIO;
    if (std::memcmp(tr, "DS4CUDA1", 8) != 0) return kEINVAL;
    if (std::fgetc(f) != EOF) return kEINVAL;   // nothing after the trailer
    info->file_bytes = off + 8;
    return 0;
}

int read_at(FILE *f, long long off, void *dst, size_t bytes) {
    if (std::fseek(f, off, SEEK_SET) != 0 || std::fread(dst, 1, bytes, f) != bytes) return kEIO;
    return 0;
}

}  // namespace

extern "C" int ds4hip_ds4cudak_probe(const char *path, ds4hip_ds4cudak_info *info) {
    if (!path || !info) return fail(kEINVAL);
    File in;
    in.f = std::fopen(path, "rb");
    if (!in.f) return fail(kEIO);
    long long off[DS4HIP_N_LAYER];
    const int rc = ref_probe(in.f, info, off);
    return rc ? fail(rc) : 0;
}

extern "C" int ds4hip_session_import_ds4cudak(ds4hip_session_state *s, const char *path, int *out_pos,
                                              int *out_n_tokens) {
    if (!path || !session_ok(s)) return fail(kEINVAL);
    File in;
    in.f = std::fopen(path, "rb");
    if (!in.f) return fail(kEIO);
    ds4hip_ds4cudak_info info;
    long long off[DS4HIP_N_LAYER];
    int rc = ref_probe(in.f, &info, off);
    if (rc) return fail(rc);
    if (info.max_context != s->max_context) return fail(kEINVAL);
    // device staging for one buffer of fp32 rows and their destination rows;
    // the host bounce buffer also receives whole compressor / indexer states,
    // which at small contexts are larger than the row buffers
    size_t max_rows = (size_t)s->layers[0].cap_raw;
    size_t host_floats = 0;
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        const ds4hip_layer_state &L = s->layers[il];
        max_rows = std::max(max_rows, (size_t)std::max(L.cap_comp, L.cap_raw));
        if (L.compress_ratio) host_floats = std::max(host_floats, attn_state_cells(L.compress_ratio));
        if (L.has_indexer)
            host_floats = std::max({host_floats, index_state_cells(),
                                    (size_t)L.cap_comp * DS4HIP_INDEXER_HEAD_DIM});
    }
    host_floats = std::max(host_floats, max_rows * DS4HIP_HEAD_DIM);
    std::vector<float> host(host_floats);
    std::vector<long long> dst(max_rows);
    float *d_rows = nullptr;
    long long *d_dst = nullptr;
    struct Free {
        void *a, *b;
        ~Free() {
            if (a) (void)hipFree(a);
            if (b) (void)hipFree(b);
        }
    } guard{nullptr, nullptr};
    if ((rc = hip_status(hipMalloc(&d_rows, max_rows * DS4HIP_HEAD_DIM * 4)))) return fail(rc);
    guard.a = d_rows;
    if ((rc = hip_status(hipMalloc(&d_dst, max_rows * 8)))) return fail(rc);
    guard.b = d_dst;
    if ((rc = init_buffers(s, 0))) return fail(rc);
    // From here on the session is being overwritten: any failure leaves it
    // reset (empty, counters 0), never a mix of old counters and new rows.
    auto fail_reset = [&](int code) {
        (void)init_buffers(s, 0);
        (void)hipDeviceSynchronize();
        return fail(code);
    };
    // rows [0, n) of the staged buffer into cache rows dst[0..n)
    auto put_rows = [&](int n) -> int {
        if (n == 0) return 0;
        int r = hip_status(hipMemcpy(d_rows, host.data(), (size_t)n * DS4HIP_HEAD_DIM * 4, hipMemcpyHostToDevice));
        if (!r) r = hip_status(hipMemcpy(d_dst, dst.data(), (size_t)n * 8, hipMemcpyHostToDevice));
        if (!r)
            r = ds4hip_fp8_kv_quantize_append(d_rows, n, DS4HIP_HEAD_DIM, DS4HIP_N_ROT, s->codes, s->sexp, s->tail,
                                              0, d_dst, nullptr);
        if (!r) r = hip_status(hipDeviceSynchronize());   // the staging buffers are reused
        return r;
    };
    auto copy_in = [&](long long at, void *d, size_t bytes) -> int {
        if (bytes > host.size() * sizeof(float)) return kEINVAL;
        int r = read_at(in.f, at, host.data(), bytes);
        if (!r) r = hip_status(hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice));
        return r;
    };
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        ds4hip_layer_state &L = s->layers[il];
        const int n_raw = info.n_raw[il];
        long long at = off[il];
        // window rows: raw row i holds position base + i
        const long long P = info.pos >= n_raw ? info.pos
                          : (info.n_tokens_processed >= n_raw ? info.n_tokens_processed : n_raw);
        const long long base = P - n_raw;
        if ((rc = read_at(in.f, at, host.data(), (size_t)L.cap_raw * DS4HIP_HEAD_DIM * 4))) return fail_reset(rc);
        for (int i = 0; i < n_raw; ++i) dst[i] = L.row_base + L.cap_comp + (base + i) % L.cap_raw;
        if ((rc = put_rows(n_raw))) return fail_reset(rc);
        at += (long long)L.cap_raw * DS4HIP_HEAD_DIM * 4;
        if (L.compress_ratio) {
            if ((rc = read_at(in.f, at, host.data(), (size_t)L.cap_comp * DS4HIP_HEAD_DIM * 4))) return fail_reset(rc);
            for (int i = 0; i < info.n_comp[il]; ++i) dst[i] = L.row_base + i;
            if ((rc = put_rows(info.n_comp[il]))) return fail_reset(rc);
            at += (long long)L.cap_comp * DS4HIP_HEAD_DIM * 4;
            const size_t sb = attn_state_cells(L.compress_ratio) * 4;
            if ((rc = copy_in(at, L.attn_state_kv, sb))) return fail_reset(rc);
            at += (long long)sb;
            if ((rc = copy_in(at, L.attn_state_score, sb))) return fail_reset(rc);
            at += (long long)sb;
            if (L.has_indexer) {
                const size_t kb = (size_t)L.cap_comp * DS4HIP_INDEXER_HEAD_DIM * 4;
                if ((rc = copy_in(at, L.index_comp_kv, kb))) return fail_reset(rc);
                at += (long long)kb;
                const size_t ib = index_state_cells() * 4;
                if ((rc = copy_in(at, L.index_state_kv, ib))) return fail_reset(rc);
                at += (long long)ib;
                if ((rc = copy_in(at, L.index_state_score, ib))) return fail_reset(rc);
            }
        }
        L.n_raw = n_raw;
        L.raw_head = (int)((base + n_raw) % L.cap_raw);
        L.n_comp = info.n_comp[il];
        L.n_index_comp = info.n_index_comp[il];
    }
    if ((rc = hip_status(hipDeviceSynchronize()))) return fail_reset(rc);
    s->pos = info.pos;
    s->n_tokens_processed = info.n_tokens_processed;
    if (out_pos) *out_pos = s->pos;
    if (out_n_tokens) *out_n_tokens = s->n_tokens_processed;
    return 0;
}

namespace {

void wr_u32(std::vector<uint8_t> &b, size_t at, uint32_t v) { std::memcpy(b.data() + at, &v, 4); }
void wr_u64(std::vector<uint8_t> &b, size_t at, uint64_t v) { std::memcpy(b.data() + at, &v, 8); }

// OCP E4M3FN value of code c (0x7F / 0xFF, the NaN codes, never occur in the cache)
float e4m3_value(uint8_t c) {
    const int e = (c >> 3) & 15, m = c & 7;
    const float mag = e == 0 ? std::ldexp((float)m, -9) : std::ldexp(1.0f + m / 8.0f, e - 7);
    return (c & 0x80) ? -mag : mag;
}

float f16_bits_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// One cache row as fp32: codes times 2^exponent per 64-dim block (rounded to
// f16 when f16_codes), then the f16 tail.
void dequant_row(const uint8_t *codes, const int8_t *sexp, const uint16_t *tail, bool f16_codes, float *out) {
    for (int d = 0; d < DS4HIP_FP8_CODES; ++d) {
        float v = std::ldexp(e4m3_value(codes[d]), sexp[d >> 6]);
        if (f16_codes) v = (float)(_Float16)v;
        out[d] = v;
    }
    for (int d = 0; d < DS4HIP_FP8_TAIL; ++d) out[DS4HIP_FP8_CODES + d] = f16_bits_to_float(tail[d]);
}

}  // namespace

extern "C" int ds4hip_session_export_ds4cudak(const ds4hip_session_state *s, const int32_t *prompt_token_ids,
                                              int n_tokens, const char *path) {
    if (!path || !session_ok(s) || n_tokens < 0 || (n_tokens > 0 && !prompt_token_ids)) return fail(kEINVAL);
    int rc = hip_status(hipDeviceSynchronize());
    if (rc) return fail(rc);
    File out;
    out.f = std::fopen(path, "wb");
    if (!out.f) return fail(kEIO);
    std::vector<uint8_t> h(kRefHdrBytes, 0);
    std::memcpy(h.data(), "DS4CUDAK", 8);
    wr_u32(h, 8, 1u);
    wr_u32(h, 12, DS4HIP_N_LAYER);
    wr_u32(h, 16, (uint32_t)s->max_context);
    wr_u32(h, 20, (uint32_t)s->pos);
    wr_u32(h, 24, (uint32_t)s->n_tokens_processed);
    const int n_ids = n_tokens < DS4HIP_KVC_MAX_TOKENS_HDR ? n_tokens : DS4HIP_KVC_MAX_TOKENS_HDR;
    wr_u32(h, 28, (uint32_t)n_ids);
    wr_u32(h, 32, (uint32_t)s->layers[0].cap_raw);
    for (int i = 0; i < n_ids; ++i) wr_u32(h, 40 + 4 * (size_t)i, (uint32_t)prompt_token_ids[i]);
    if (std::fwrite(h.data(), 1, h.size(), out.f) != h.size()) return fail(kEIO);
    std::vector<uint8_t> codes, sexp;
    std::vector<uint16_t> tail;
    std::vector<float> rows;
    auto get = [&](const void *d, void *hp, size_t bytes) {
        return hip_status(hipMemcpy(hp, d, bytes, hipMemcpyDeviceToHost));
    };
    auto put = [&](const void *p, size_t bytes) { return std::fwrite(p, 1, bytes, out.f) == bytes ? 0 : kEIO; };
    for (int il = 0; il < DS4HIP_N_LAYER; ++il) {
        const ds4hip_layer_state &L = s->layers[il];
        const size_t n_rows = (size_t)L.cap_comp + L.cap_raw;
        codes.resize(n_rows * DS4HIP_FP8_CODES);
        sexp.resize(n_rows * DS4HIP_FP8_SEXP);
        tail.resize(n_rows * DS4HIP_FP8_TAIL);
        if ((rc = get(s->codes + (size_t)L.row_base * DS4HIP_FP8_CODES, codes.data(), codes.size())) ||
            (rc = get(s->sexp + (size_t)L.row_base * DS4HIP_FP8_SEXP, sexp.data(), sexp.size())) ||
            (rc = get(s->tail + (size_t)L.row_base * DS4HIP_FP8_TAIL, tail.data(), tail.size() * 2)))
            return fail(rc);
        std::vector<uint8_t> m(kRefMetaBytes, 0);
        wr_u32(m, 0, (uint32_t)il);
        wr_u32(m, 4, (uint32_t)L.compress_ratio);
        wr_u32(m, 8, (uint32_t)L.has_indexer);
        wr_u32(m, 12, (uint32_t)L.cap_raw);
        wr_u32(m, 16, (uint32_t)L.cap_comp);
        wr_u32(m, 20, (uint32_t)L.n_raw);
        wr_u32(m, 24, (uint32_t)L.n_comp);
        wr_u32(m, 28, (uint32_t)L.n_index_comp);
        wr_u64(m, 32, ref_layer_payload(L.compress_ratio, L.cap_raw, L.cap_comp));
        if ((rc = put(m.data(), m.size()))) return fail(rc);
        auto row = [&](size_t r, bool f16_codes, float *o) {
            dequant_row(codes.data() + r * DS4HIP_FP8_CODES, (const int8_t *)sexp.data() + r * DS4HIP_FP8_SEXP,
                        tail.data() + r * DS4HIP_FP8_TAIL, f16_codes, o);
        };
        // window rows oldest first, the rest of the capacity zero
        rows.assign((size_t)L.cap_raw * DS4HIP_HEAD_DIM, 0.0f);
        for (int i = 0; i < L.n_raw; ++i) {
            const int slot = ((L.raw_head - L.n_raw + i) % L.cap_raw + L.cap_raw) % L.cap_raw;
            row((size_t)L.cap_comp + slot, true, rows.data() + (size_t)i * DS4HIP_HEAD_DIM);
        }
        if ((rc = put(rows.data(), rows.size() * 4))) return fail(rc);
        if (L.compress_ratio) {
            rows.assign((size_t)L.cap_comp * DS4HIP_HEAD_DIM, 0.0f);
            for (int i = 0; i < L.n_comp; ++i) row((size_t)i, false, rows.data() + (size_t)i * DS4HIP_HEAD_DIM);
            if ((rc = put(rows.data(), rows.size() * 4))) return fail(rc);
            std::vector<float> st(attn_state_cells(L.compress_ratio));
            if ((rc = get(L.attn_state_kv, st.data(), st.size() * 4)) || (rc = put(st.data(), st.size() * 4)) ||
                (rc = get(L.attn_state_score, st.data(), st.size() * 4)) || (rc = put(st.data(), st.size() * 4)))
                return fail(rc);
            if (L.has_indexer) {
                std::vector<float> kk((size_t)L.cap_comp * DS4HIP_INDEXER_HEAD_DIM), ist(index_state_cells());
                if ((rc = get(L.index_comp_kv, kk.data(), kk.size() * 4)) || (rc = put(kk.data(), kk.size() * 4)) ||
                    (rc = get(L.index_state_kv, ist.data(), ist.size() * 4)) ||
                    (rc = put(ist.data(), ist.size() * 4)) ||
                    (rc = get(L.index_state_score, ist.data(), ist.size() * 4)) ||
                    (rc = put(ist.data(), ist.size() * 4)))
                    return fail(rc);
            }
        }
    }
    std::vector<uint8_t> zeros(kRefResidualBytes, 0);
    if ((rc = put(zeros.data(), zeros.size())) || (rc = put("DS4CUDA1", 8))) return fail(rc);
    const int cr = std::fclose(out.f);
    out.f = nullptr;
    return cr == 0 ? 0 : fail(kEIO);
}
