// forward_layer_check.cpp — a forward_layer-shaped caller of the attention
// slice (Steps 11-16 of cuda/forward_layer.cu:915-1210), written against the
// ds4cuda:: launcher shims of ds4hip_launchers.h exactly as the reference's
// ds4_forward_layer calls its own launchers, with the reference's fp32 row
// layout (raw SWA ring with memmove eviction, compressed rows appended).
//
// Usage: forward_layer_check <dir> <il> <n_tokens> <top_k>
// Reads the token inputs and layer weights from <dir> (raw little-endian
// arrays written by tests/test_gpu_forward_layer.py), runs tokens
// pos = 0 .. n_tokens-1 through the slice on the GPU and writes, per token,
// the attention output, the allowed mask, the indexer query and weights, the
// compressed-row counts and the slice output to <dir>/out.bin.
#include "ds4hip_launchers.h"
#include "ds4hip_session.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

constexpr int kN_EMBD = 4096, kHEAD_DIM = 512, kN_HEAD = 64, kN_ROT = 64, kQ_DIM = 64 * 512;
constexpr int kQ_LORA_RANK = 1024, kN_INDEXER_HEAD = 64, kIDX_HEAD_DIM = 128;
constexpr int kIDX_Q_DIM = kN_INDEXER_HEAD * kIDX_HEAD_DIM;
constexpr int kN_OUT_GROUP = 8, kN_LORA_O = 1024, kATTN_LOW_OUT = kN_OUT_GROUP * kN_LORA_O;
constexpr int kN_SWA = 128;

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            std::exit(10);                                                             \
        }                                                                              \
    } while (0)

// ds4hip_get_last_error() after every launch, as cuda/forward_layer.cu:81-89
// checks cudaGetLastError().
#define FCK()                                                                          \
    do {                                                                               \
        const int rc_ = ds4hip_clear_last_error();                                     \
        if (rc_ != 0) {                                                                \
            std::fprintf(stderr, "%s:%d launcher failed %d\n", __FILE__, __LINE__, rc_); \
            std::exit(11);                                                             \
        }                                                                              \
    } while (0)

std::vector<char> read_file(const std::string &path, size_t expect) {
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) {
        std::fprintf(stderr, "missing %s\n", path.c_str());
        std::exit(12);
    }
    std::vector<char> b(expect);
    const size_t n = std::fread(b.data(), 1, expect, f);
    std::fclose(f);
    if (n != expect) {
        std::fprintf(stderr, "%s: %zu bytes, expected %zu\n", path.c_str(), n, expect);
        std::exit(13);
    }
    return b;
}

template <typename T>
T *upload(const std::string &dir, const char *name, size_t count) {
    const std::vector<char> h = read_file(dir + "/" + name, count * sizeof(T));
    T *d = nullptr;
    CK(hipMalloc(&d, count * sizeof(T)));
    CK(hipMemcpy(d, h.data(), count * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <typename T>
T *dalloc(size_t count, int fill_byte = 0) {
    T *d = nullptr;
    CK(hipMalloc(&d, count * sizeof(T)));
    CK(hipMemset(d, fill_byte, count * sizeof(T)));
    return d;
}

void fill_neg_inf(float *d, size_t n) {
    std::vector<float> h(n, -INFINITY);
    CK(hipMemcpy(d, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <dir> <il> <n_tokens> <top_k>\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const int il = std::atoi(argv[2]), T = std::atoi(argv[3]), top_k = std::atoi(argv[4]);
    const int ratio = il < 2 ? 0 : ((il & 1) == 0 ? 4 : 128);   // cuda/rope.cu:123-126
    const bool has_compressor = ratio != 0, has_indexer = ratio == 4;
    const int coff = ratio == 4 ? 2 : 1;
    const int cap_comp = T / (ratio ? ratio : 1) + 2;           // cuda/session_state.cu:137

    // token inputs
    float *kv_rope = upload<float>(dir, "kv_rope.bin", (size_t)T * kHEAD_DIM);
    float *attn_norm = upload<float>(dir, "attn_norm.bin", (size_t)T * kN_EMBD);
    float *q_cur = upload<float>(dir, "q_cur.bin", (size_t)T * kQ_DIM);
    float *q_lora = upload<float>(dir, "q_lora_norm.bin", (size_t)T * kQ_LORA_RANK);
    // weights
    float *sinks = upload<float>(dir, "sinks.bin", kN_HEAD);
    auto *w_out_a = upload<ds4cuda::block_q8_0>(dir, "attn_output_a.bin",
                                               (size_t)kATTN_LOW_OUT * (kN_LORA_O * 4 / 32));
    auto *w_out_b = upload<ds4cuda::block_q8_0>(dir, "attn_output_b.bin",
                                               (size_t)kN_EMBD * (kATTN_LOW_OUT / 32));
    const int aw = coff * kHEAD_DIM, iw = coff * kIDX_HEAD_DIM;
    uint16_t *c_kv = nullptr, *c_gate = nullptr, *c_ape = nullptr, *i_kv = nullptr,
             *i_gate = nullptr, *i_ape = nullptr, *i_qb = nullptr, *i_proj = nullptr;
    float *c_norm = nullptr, *i_norm = nullptr;
    if (has_compressor) {
        c_kv = upload<uint16_t>(dir, "comp_kv.bin", (size_t)aw * kN_EMBD);
        c_gate = upload<uint16_t>(dir, "comp_gate.bin", (size_t)aw * kN_EMBD);
        c_ape = upload<uint16_t>(dir, "comp_ape.bin", (size_t)ratio * aw);
        c_norm = upload<float>(dir, "comp_norm.bin", kHEAD_DIM);
    }
    if (has_indexer) {
        i_kv = upload<uint16_t>(dir, "idx_kv.bin", (size_t)iw * kN_EMBD);
        i_gate = upload<uint16_t>(dir, "idx_gate.bin", (size_t)iw * kN_EMBD);
        i_ape = upload<uint16_t>(dir, "idx_ape.bin", (size_t)ratio * iw);
        i_norm = upload<float>(dir, "idx_norm.bin", kIDX_HEAD_DIM);
        i_qb = upload<uint16_t>(dir, "idx_q_b.bin", (size_t)kIDX_Q_DIM * kQ_LORA_RANK);
        i_proj = upload<uint16_t>(dir, "idx_proj.bin", (size_t)kN_INDEXER_HEAD * kN_EMBD);
    }

    // layer state (the reference's fp32 ds4_layer_state, include/ds4cuda.h:310-360)
    float *raw_kv = dalloc<float>((size_t)kN_SWA * kHEAD_DIM);
    float *comp_kv = dalloc<float>((size_t)cap_comp * kHEAD_DIM);
    float *index_comp_kv = dalloc<float>((size_t)cap_comp * kIDX_HEAD_DIM);
    float *attn_state_kv = dalloc<float>((size_t)coff * (ratio ? ratio : 1) * aw);
    float *attn_state_score = dalloc<float>((size_t)coff * (ratio ? ratio : 1) * aw);
    float *index_state_kv = dalloc<float>((size_t)coff * 4 * iw);
    float *index_state_score = dalloc<float>((size_t)coff * 4 * iw);
    fill_neg_inf(attn_state_score, (size_t)coff * (ratio ? ratio : 1) * aw);
    fill_neg_inf(index_state_score, (size_t)coff * 4 * iw);
    int n_raw = 0, n_comp = 0, n_index_comp = 0;

    // activations / scratch
    float *kv_cur = dalloc<float>(kHEAD_DIM), *attn_emit = dalloc<float>(kHEAD_DIM);
    float *idx_emit = dalloc<float>(kIDX_HEAD_DIM);
    float *comp_kv_cur = dalloc<float>(2 * kHEAD_DIM), *comp_sc_cur = dalloc<float>(2 * kHEAD_DIM);
    int32_t *comp_allowed = dalloc<int32_t>(cap_comp);
    float *indexer_q = dalloc<float>(kIDX_Q_DIM), *indexer_w = dalloc<float>(kN_INDEXER_HEAD);
    float *indexer_scores = dalloc<float>(cap_comp);
    float *kqv_out = dalloc<float>(kQ_DIM), *kqv_back = dalloc<float>(kQ_DIM);
    float *attn_low = dalloc<float>(kATTN_LOW_OUT), *attn_out = dalloc<float>(kN_EMBD);
    int8_t *xq = dalloc<int8_t>(kQ_DIM);
    float *xscale = dalloc<float>(kQ_DIM / 32);

    hipStream_t stream;
    CK(hipStreamCreate(&stream));
    FILE *out = std::fopen((dir + "/out.bin").c_str(), "wb");
    std::vector<float> h_kqv(kQ_DIM), h_out(kN_EMBD), h_q(kIDX_Q_DIM), h_w(kN_INDEXER_HEAD);
    std::vector<int32_t> h_mask(cap_comp);

    for (int pos = 0; pos < T; ++pos) {
        const float *x = attn_norm + (size_t)pos * kN_EMBD;
        // Step 11: FP8 round trip of the roped KV row
        ds4cuda::launch_fp8_kv_quantize_round_trip_f32(kv_rope + (size_t)pos * kHEAD_DIM, kv_cur,
                                                       1, kHEAD_DIM, kN_ROT, stream);
        FCK();
        // Step 12: raw ring push (memmove eviction when full)
        if (ds4hip_swa_push_f32(raw_kv, &n_raw, kN_SWA, kv_cur, kHEAD_DIM, stream)) return 20;
        // Step 12a / 12b: compressors, row pushes, indexer_allowed
        int attn_emit_host = 0, idx_emit_host = 0;
        if (has_compressor) {
            ds4cuda::launch_compressor_decode_step_f32_prealloc(
                true, x, c_kv, c_gate, c_ape, c_norm, kN_EMBD, kHEAD_DIM, ratio, pos, il,
                attn_state_kv, attn_state_score, attn_emit, &attn_emit_host, comp_kv_cur,
                comp_sc_cur, stream);
            FCK();
            if (attn_emit_host &&
                ds4hip_comp_push_f32(comp_kv, &n_comp, cap_comp, attn_emit, kHEAD_DIM, stream))
                return 21;
        }
        if (has_indexer) {
            ds4cuda::launch_compressor_decode_step_f32_prealloc(
                false, x, i_kv, i_gate, i_ape, i_norm, kN_EMBD, kIDX_HEAD_DIM, ratio, pos, il,
                index_state_kv, index_state_score, idx_emit, &idx_emit_host, comp_kv_cur,
                comp_sc_cur, stream);
            FCK();
            if (idx_emit_host && ds4hip_comp_push_f32(index_comp_kv, &n_index_comp, cap_comp,
                                                      idx_emit, kIDX_HEAD_DIM, stream))
                return 22;
            if (n_index_comp > 0) {
                if (n_index_comp <= top_k) {
                    ds4cuda::launch_indexer_allowed_short_circuit_i32(comp_allowed, n_index_comp,
                                                                      top_k, stream);
                } else {
                    ds4cuda::launch_mul_mv_f16_f32(i_qb, q_lora + (size_t)pos * kQ_LORA_RANK,
                                                   indexer_q, kIDX_Q_DIM, kQ_LORA_RANK, stream);
                    FCK();
                    ds4cuda::launch_tail_rope_yarn_f32(indexer_q, indexer_q, kN_INDEXER_HEAD,
                                                       kIDX_HEAD_DIM, kN_ROT, pos, il, stream);
                    FCK();
                    ds4cuda::launch_mul_mv_f16_f32(i_proj, x, indexer_w, kN_INDEXER_HEAD, kN_EMBD,
                                                   stream);
                    FCK();
                    ds4cuda::launch_scale_inplace_f32(
                        indexer_w, kN_INDEXER_HEAD,
                        1.0f / std::sqrt((float)(kIDX_HEAD_DIM * kN_INDEXER_HEAD)), stream);
                    FCK();
                    ds4cuda::launch_indexer_score_topk_f32_i32(
                        indexer_q, indexer_w, index_comp_kv, n_index_comp, kN_INDEXER_HEAD,
                        kIDX_HEAD_DIM, top_k, comp_allowed, indexer_scores, stream);
                }
                FCK();
            }
        }
        // Step 13: attention
        const float *q = q_cur + (size_t)pos * kQ_DIM;
        if (has_compressor)
            ds4cuda::launch_flash_attn_decode_mixed_f32(
                q, raw_kv, comp_kv, (has_indexer && n_index_comp > 0) ? comp_allowed : nullptr,
                sinks, kqv_out, kN_HEAD, n_raw, n_comp, kHEAD_DIM, stream);
        else
            ds4cuda::launch_flash_attn_decode_raw_f32(q, raw_kv, raw_kv, sinks, kqv_out, kN_HEAD,
                                                      n_raw, kHEAD_DIM, stream);
        FCK();
        // Step 14: inverse tail RoPE
        ds4cuda::launch_tail_rope_yarn_inverse_f32(kqv_out, kqv_back, kN_HEAD, kHEAD_DIM, kN_ROT,
                                                   pos, il, stream);
        FCK();
        // Step 15: grouped Q8_0 low-rank projection
        ds4cuda::launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(
            w_out_a, kqv_back, attn_low, kN_OUT_GROUP, kHEAD_DIM * (kN_HEAD / kN_OUT_GROUP),
            kN_LORA_O, xq, xscale, stream);
        FCK();
        // Step 16: dense Q8_0 output projection
        ds4cuda::launch_mul_mv_q8_0_q8_0_f32_prealloc(w_out_b, attn_low, attn_out, kN_EMBD,
                                                      kATTN_LOW_OUT, xq, xscale, stream);
        FCK();

        CK(hipStreamSynchronize(stream));
        CK(hipMemcpy(h_kqv.data(), kqv_out, kQ_DIM * 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(h_out.data(), attn_out, kN_EMBD * 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(h_mask.data(), comp_allowed, cap_comp * 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(h_q.data(), indexer_q, kIDX_Q_DIM * 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(h_w.data(), indexer_w, kN_INDEXER_HEAD * 4, hipMemcpyDeviceToHost));
        const int32_t counts[4] = {n_raw, n_comp, n_index_comp, attn_emit_host};
        std::fwrite(counts, 4, 4, out);
        std::fwrite(h_kqv.data(), 4, kQ_DIM, out);
        std::fwrite(h_out.data(), 4, kN_EMBD, out);
        std::fwrite(h_mask.data(), 4, cap_comp, out);
        std::fwrite(h_q.data(), 4, kIDX_Q_DIM, out);
        std::fwrite(h_w.data(), 4, kN_INDEXER_HEAD, out);
    }
    // the index keys the indexer scored (fp32 rows), for the selection check
    std::vector<float> h_keys((size_t)cap_comp * kIDX_HEAD_DIM);
    CK(hipMemcpy(h_keys.data(), index_comp_kv, h_keys.size() * 4, hipMemcpyDeviceToHost));
    std::fwrite(h_keys.data(), 4, h_keys.size(), out);
    std::fclose(out);
    std::printf("forward_layer_check ok: il %d, %d tokens, n_raw %d, n_comp %d, n_index_comp %d\n",
                il, T, n_raw, n_comp, n_index_comp);
    return 0;
}
