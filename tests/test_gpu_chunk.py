"""The prefill chunk driver (ds4cuda_amd.chunk.forward_chunk_attn) against the
token-by-token loop it replaces (cuda/forward_batch.cu:264-284 runs
ds4_forward_layer per token): from the same session state (a history built
token by token, cloned through save/load), a chunk of tokens through the
driver and the same tokens one at a time (push, compressors, indexer
selection, single-problem decode) give

  * attention outputs with exact_p within 1e-4 x RMS (the same rows and
    math; only the split of the rows over workgroups differs); the default
    path's token outputs within the 2e-3 x RMS decode bar of those, per token
    (an fp32 Q always passes P as f16 hi + lo, so today they agree to ~1e-5;
    a one-f16-P path, which rounds P against a running max that depends on
    the split, measured up to 2.4e-3 here), and on the window-only layer both
    within 2e-3 x RMS of the CPU oracle for the chunk's last token;
  * byte-identical sessions afterwards (ring rows, compressed rows, indexer
    keys, compressor states, counters), the staging rows aside.

Layers: il 0 (window only), il 2 (ratio 4 with the indexer; top-k 8 so that
the selection runs) and il 3 (ratio 128), history 150 tokens, chunk 41."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import session, synth
from ds4cuda_amd.chunk import ChunkLayer, forward_chunk_attn
from ds4cuda_amd.ops import _ptr, _stream
from ds4cuda_amd._lib import call

pytestmark = pytest.mark.gpu

EMBD, HD, IHD, NH = 4096, 512, 128, 64
TOPK = 8
HIST, CHUNK = 150, 41


def f16t(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16))).to(gpu).view(torch.int16)


def layer_weights(il, gpu):
    ratio = 0 if il < 2 else (4 if il % 2 == 0 else 128)
    if not ratio:
        return None
    coff = 2 if ratio == 4 else 1
    g = lambda s, n, std: synth.normal(200 + il, s, n, std)
    w = {"comp_kv": f16t(g(1, coff * HD * EMBD, 0.02), gpu), "comp_gate": f16t(g(2, coff * HD * EMBD, 0.02), gpu),
         "comp_ape": f16t(g(3, ratio * coff * HD, 0.1), gpu),
         "comp_norm": torch.from_numpy((1 + 0.1 * g(4, HD, 1.0)).astype(np.float32)).to(gpu)}
    if ratio == 4:
        w.update({"idx_kv": f16t(g(5, 2 * IHD * EMBD, 0.02), gpu), "idx_gate": f16t(g(6, 2 * IHD * EMBD, 0.02), gpu),
                  "idx_ape": f16t(g(7, 4 * 2 * IHD, 0.1), gpu),
                  "idx_norm": torch.from_numpy((1 + 0.1 * g(8, IHD, 1.0)).astype(np.float32)).to(gpu),
                  "idx_q_b": f16t(g(9, NH * IHD * 1024, 0.05), gpu),
                  "idx_proj": f16t(g(10, NH * EMBD, 0.02), gpu)})
    return ChunkLayer(w, top_k=TOPK)


def token_inputs(il, pos, gpu):
    g = lambda s, n: torch.from_numpy(synth.normal(300 + il, 10 * pos + s, n)).to(gpu)
    return g(1, EMBD), g(2, 1024), g(3, NH * HD), g(4, HD)   # attn_norm, q_lora_norm, q_cur, kv_rope


def one_token(s, il, pos, layer, sinks, out, gpu, out_fast=None):
    """The per-token loop's attention slice (Steps 11-13) on the session; out
    receives the decode with P as hi + lo (exact_p), out_fast (if given) the
    default one-f16-P decode of the same rows."""
    x, qln, q, kv = token_inputs(il, pos, gpu)
    s.push_raw(il, kv)
    L = s.layer(il)
    ratio = L.compress_ratio
    st = _stream(None)
    n_sel = -1
    if ratio:
        w = layer.w
        coff = 2 if ratio == 4 else 1
        emit = torch.empty(HD, device=gpu)
        sc = torch.empty(2 * coff * HD, device=gpu)
        e = C.c_int(0)
        call("ds4hip_compressor_decode_step_f32_prealloc", 1, _ptr(x), _ptr(w["comp_kv"]), _ptr(w["comp_gate"]),
             _ptr(w["comp_ape"]), _ptr(w["comp_norm"]), EMBD, HD, ratio, pos, il, C.c_void_p(L.attn_state_kv),
             C.c_void_p(L.attn_state_score), _ptr(emit), C.byref(e), _ptr(sc), _ptr(sc[coff * HD:]), st)
        if e.value:
            s.push_comp(il, emit)
        if ratio == 4:
            ei_row = torch.empty(IHD, device=gpu)
            sci = torch.empty(2 * coff * IHD, device=gpu)
            ei = C.c_int(0)
            call("ds4hip_compressor_decode_step_f32_prealloc", 0, _ptr(x), _ptr(w["idx_kv"]), _ptr(w["idx_gate"]),
                 _ptr(w["idx_ape"]), _ptr(w["idx_norm"]), EMBD, IHD, ratio, pos, il,
                 C.c_void_p(L.index_state_kv), C.c_void_p(L.index_state_score), _ptr(ei_row), C.byref(ei),
                 _ptr(sci), _ptr(sci[coff * IHD:]), st)
            if ei.value:
                s.push_index_comp(il, ei_row)
            L = s.layer(il)
            if L.n_index_comp > TOPK:
                q_idx = torch.empty(NH * IHD, device=gpu)
                w_idx = torch.empty(NH, device=gpu)
                call("ds4hip_mul_mv_f16_f32", _ptr(w["idx_q_b"]), _ptr(qln), _ptr(q_idx), NH * IHD, 1024, st)
                call("ds4hip_tail_rope_yarn_f32", _ptr(q_idx), _ptr(q_idx), NH, IHD, 64, pos, il, st)
                call("ds4hip_mul_mv_f16_f32", _ptr(w["idx_proj"]), _ptr(x), _ptr(w_idx), NH, EMBD, st)
                call("ds4hip_scale_inplace_f32", _ptr(w_idx), NH, C.c_float(1.0 / np.sqrt(IHD * NH)), st)
                _, _, sel = s.layer_rows(il, TOPK)
                scores = torch.empty(L.n_index_comp, device=gpu)
                from ds4cuda_amd import lib
                select = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(L.n_index_comp),
                                     dtype=torch.uint8, device=gpu)
                call("ds4hip_indexer_topk_positions", _ptr(q_idx), _ptr(w_idx), C.c_void_p(L.index_comp_kv), 0,
                     L.n_index_comp, NH, IHD, TOPK, 0, _ptr(scores), _ptr(select), None, C.c_void_p(sel), st)
                n_sel = TOPK
    s.decode(il, q, sinks, out, n_selected=n_sel, exact_p=True)
    if out_fast is not None:
        s.decode(il, q, sinks, out_fast, n_selected=n_sel)


def layer_bytes(s, il):
    """The layer's FP8 rows, row list, compressor / indexer state and counters."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    torch.cuda.synchronize()
    L = s.layer(il)
    rows = L.cap_comp + L.cap_raw
    parts = [(s.s.codes + L.row_base * 448, rows * 448), (s.s.sexp + L.row_base * 8, rows * 8),
             (s.s.tail + L.row_base * 128, rows * 128), (L.row_list, rows * 4)]
    if L.compress_ratio:
        coff = 2 if L.compress_ratio == 4 else 1
        cells = coff * L.compress_ratio * coff * HD * 4
        parts += [(L.attn_state_kv, cells), (L.attn_state_score, cells)]
    if L.has_indexer:
        parts += [(L.index_comp_kv, L.cap_comp * IHD * 4), (L.index_state_kv, 8 * 256 * 4),
                  (L.index_state_score, 8 * 256 * 4)]
    out = []
    for p, nb in parts:
        b = np.empty(nb, np.uint8)
        assert hip.hipMemcpy(b.ctypes.data, p, nb, 2) == 0
        out.append(b)
    return out, (L.n_raw, L.raw_head, L.n_comp, L.n_index_comp)


@pytest.mark.parametrize("il", [0, 2, 3])
def test_chunk_matches_token_loop(gpu, tmp_path, il):
    layer = layer_weights(il, gpu)
    sinks = torch.from_numpy(synth.normal(310, il, NH)).to(gpu)
    out1 = torch.empty(NH * HD, device=gpu)
    out_fast = torch.empty(NH * HD, device=gpu)
    a = session.Session(1024)
    b = session.Session(1024)
    c = session.Session(1024)
    try:
        for pos in range(HIST):
            one_token(a, il, pos, layer, sinks, out1, gpu)
        a.save(tmp_path / "h.kv")
        assert b.load(tmp_path / "h.kv")[0] == 0
        assert c.load(tmp_path / "h.kv")[0] == 0
        # the chunk through the driver (session a: hi + lo P; session c: default)
        ins = [token_inputs(il, HIST + t, gpu) for t in range(CHUNK)]
        stack = lambda k: torch.stack([x[k] for x in ins])
        attn_norm, qln, q_cur, kv = stack(0), stack(1), stack(2).reshape(CHUNK, NH, HD), stack(3)
        out_chunk = torch.empty((CHUNK, NH, HD), device=gpu)
        out_chunk_fast = torch.empty((CHUNK, NH, HD), device=gpu)
        forward_chunk_attn(a, il, HIST, attn_norm, qln, q_cur, kv, sinks, out_chunk, layer=layer, exact_p=True)
        forward_chunk_attn(c, il, HIST, attn_norm, qln, q_cur, kv, sinks, out_chunk_fast, layer=layer)
        # the same tokens one at a time (session b)
        ref, ref_fast = [], []
        for t in range(CHUNK):
            one_token(b, il, HIST + t, layer, sinks, out1, gpu, out_fast)
            ref.append(out1.clone())
            ref_fast.append(out_fast.clone())
        torch.cuda.synchronize()
        got = out_chunk.cpu().numpy().reshape(CHUNK, -1)
        got_fast = out_chunk_fast.cpu().numpy().reshape(CHUNK, -1)
        exp = torch.stack(ref).cpu().numpy()
        exp_fast = torch.stack(ref_fast).cpu().numpy()
        rms = np.sqrt(np.mean(exp.astype(np.float64) ** 2))
        err = np.abs(got - exp).max() / rms
        # the decode bar holds per problem (each token is one): max err / RMS of its output
        rms_t = np.sqrt(np.mean(exp.astype(np.float64) ** 2, axis=1))
        e_fast = [float((np.abs(x - exp).max(axis=1) / rms_t).max()) for x in (got_fast, exp_fast)]
        print(f"il {il}: default paths vs exact_p: chunk {e_fast[0]:.2e}, token loop {e_fast[1]:.2e}")
        assert err < 1e-4, err
        assert max(e_fast) < 2e-3, e_fast
        if il == 0:   # oracle: the chunk's last token over its window (dequantized rows)
            win = np.stack([token_inputs(il, p, gpu)[3].cpu().numpy()
                            for p in range(HIST + CHUNK - 128, HIST + CHUNK)])
            deq = O.fp8_quant_rows(win)[3]
            ref_o = O.attn_decode_mixed_f32(q_cur[-1].cpu().numpy(), deq, None, None, sinks.cpu().numpy())
            for g in (got, got_fast):
                e_o = np.abs(g[-1].reshape(NH, HD) - ref_o).max() / np.sqrt(np.mean(ref_o.astype(np.float64) ** 2))
                print(f"il 0: last token vs oracle {e_o:.2e}")
                assert e_o < 2e-3, e_o
        ra, ca = layer_bytes(a, il), layer_bytes(b, il)
        assert ra[1] == ca[1]
        for x, y in zip(ra[0], ca[0]):
            assert np.array_equal(x, y)
        print(f"il {il}: chunk of {CHUNK} after {HIST} tokens, max err/RMS vs token loop {err:.2e}; "
              f"sessions byte-identical")
    finally:
        a.close()
        b.close()
        c.close()
