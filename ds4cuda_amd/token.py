"""The per-token attention slice of all 43 layers: Steps 11-16 of
ds4_forward_layer (cuda/forward_layer.cu:915-1210) for every layer of one
token, as ds4_forward_token runs them layer after layer
(cuda/forward_token.cu:368-378), over the FP8 session.

Per layer il at position pos:
  11. the layer's KV row into the FP8 ring (quantize + push);
  12. the attention compressor (ratio 4 / 128 layers) and, on an emit step,
      its row appended; on ratio-4 layers the indexer compressor, its key row,
      and once there are more than top_k keys the indexer query / head weights
      and the top-k selection written into the layer's row list;
  13. decode attention over the ring rows and the (selected) compressed rows,
      fp32 Q, with the layer's sinks;
  14. inverse tail RoPE;
  15. the grouped Q8_0 low-rank projection (8 groups x 4096 -> 1024);
  16. the dense Q8_0 output projection (8192 -> 4096)
(Steps 14-16 through ds4hip_attn_out_decode_f32, the indexer query and head
weights through the fused matvec launches: the same values, fewer launches).

Every buffer is allocated up front, and step() neither allocates, nor
synchronizes the host, nor writes memory with hipMemsetAsync, so capture()
can record a whole token (about 400 kernels) into one HIP graph. The
host-side decisions of a step (whether a compressor emits, whether the
indexer selects) depend only on pos and the session's counters, which the
capture advances as an eager step would; a graph therefore replays the token
it was captured at.

Every kernel is a libds4hip.so entry point; torch provides device memory and
the stream only.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import Ds4HipError, call, lib
from .ops import _check, _ptr, _stream, decode_fp8_workspace_bytes, q_prep_words
from .session import N_LAYER, Session

N_HEAD, HEAD_DIM, N_ROT, IDX_DIM, IDX_HEAD, N_EMBD = 64, 512, 64, 128, 64, 4096
Q_LORA = 1024
N_OUT_GROUP, N_LORA_O = 8, 1024
Q8_BLOCK = 34


class TokenPrologue(C.Structure):
    """ds4hip_token_prologue (include/ds4hip.h): one layer step's independent
    launches of Steps 11-12c as one."""
    _vp_fields = lambda pre: [(pre + n, C.c_void_p) for n in ("w_kv", "w_gate", "w_ape", "state_kv", "state_score")] + \
        [(pre + n, C.c_int) for n in ("head_dim_out", "ratio", "pos")]
    _fields_ = [("kv", C.c_void_p), ("codes", C.c_void_p), ("sexp", C.c_void_p), ("tail", C.c_void_p),
                ("kv_row", C.c_longlong), ("head_dim", C.c_int), ("n_rot", C.c_int), ("x", C.c_void_p),
                ("in_dim", C.c_int), ("n_comp", C.c_int)] + _vp_fields("comp0_") + _vp_fields("comp1_") + \
               [("q_w", C.c_void_p), ("q_x", C.c_void_p), ("q_out", C.c_void_p), ("q_heads", C.c_int),
                ("q_head_dim", C.c_int), ("q_in", C.c_int), ("q_pos", C.c_int), ("q_il", C.c_int),
                ("hw_w", C.c_void_p), ("hw_out", C.c_void_p), ("hw_rows", C.c_int), ("hw_scale", C.c_float),
                ("qp_q", C.c_void_p), ("qp_out", C.c_void_p)]


def layer_ratio(il: int) -> int:
    """Compression ratio of layer il (cuda/rope.cu:123-126): 0 for il < 2,
    then 4 on even and 128 on odd layers."""
    return 0 if il < 2 else (4 if il % 2 == 0 else 128)


def _vp(x):
    return C.c_void_p(x)


def q8_weights(rows: int, cols: int, gen: torch.Generator, device, scale: float = 0.02):
    """A random Q8_0 matrix [rows, cols / 32 blocks] as uint8 [rows, cols/32, 34]
    (f16 d, then 32 int8), on the device."""
    nb = cols // 32
    d = (torch.rand((rows, nb), generator=gen, device=device) * (2 * scale / 127) + scale / 254)
    qs = torch.randint(-127, 128, (rows, nb, 32), generator=gen, device=device, dtype=torch.int8)
    w = torch.empty((rows, nb, Q8_BLOCK), dtype=torch.uint8, device=device)
    w[:, :, :2] = d.to(torch.float16).view(torch.uint8).view(rows, nb, 2)
    w[:, :, 2:] = qs.view(torch.uint8)
    return w


def f16_weights(shape, gen, device, std=0.02):
    return (torch.randn(shape, generator=gen, device=device) * std).to(torch.float16).view(torch.int16)


def synthetic_weights(device, seed: int = 90):
    """Random-init weights of the reference's architecture and dtypes for the 43
    layers' attention slice (f16 compressor / indexer weights, Q8_0 output
    projections, fp32 sinks and norms)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layers = []
    for il in range(N_LAYER):
        r = layer_ratio(il)
        w = {"sinks": torch.randn(N_HEAD, generator=gen, device=device),
             "out_a": q8_weights(N_OUT_GROUP * N_LORA_O, HEAD_DIM * N_HEAD // N_OUT_GROUP, gen, device),
             "out_b": q8_weights(N_EMBD, N_OUT_GROUP * N_LORA_O, gen, device)}
        if r:
            coff = 2 if r == 4 else 1
            w.update(comp_kv=f16_weights((coff * HEAD_DIM, N_EMBD), gen, device),
                     comp_gate=f16_weights((coff * HEAD_DIM, N_EMBD), gen, device),
                     comp_ape=f16_weights((r, coff * HEAD_DIM), gen, device, 0.1),
                     comp_norm=1 + 0.1 * torch.randn(HEAD_DIM, generator=gen, device=device))
        if r == 4:
            w.update(idx_kv=f16_weights((2 * IDX_DIM, N_EMBD), gen, device),
                     idx_gate=f16_weights((2 * IDX_DIM, N_EMBD), gen, device),
                     idx_ape=f16_weights((4, 2 * IDX_DIM), gen, device, 0.1),
                     idx_norm=1 + 0.1 * torch.randn(IDX_DIM, generator=gen, device=device),
                     idx_q_b=f16_weights((IDX_HEAD * IDX_DIM, Q_LORA), gen, device, 0.05),
                     idx_proj=f16_weights((IDX_HEAD, N_EMBD), gen, device))
        layers.append(w)
    return layers


def _hip():
    h = C.CDLL("libamdhip64.so")
    h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return h


def fill_history(session: Session, pos: int, seed: int = 91):
    """Puts session in the state of `pos` tokens of synthetic history: every
    layer's ring holds its last min(pos, 128) rows, ratio-r layers pos // r
    compressed rows (and, on ratio-4 layers, as many fp32 indexer keys), the
    compressor states finite values. Rows are random N(0, 1) through the FP8
    quantizer (the same rows an eager history would hold, up to their values).
    Synchronous."""
    dev = torch.device("cuda", torch.cuda.current_device())
    s = session.s
    if pos > s.max_context:
        raise Ds4HipError("history past the session's max_context", -22)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    hip = _hip()
    for il in range(N_LAYER):
        L = s.layers[il]
        r = L.compress_ratio
        n_raw = min(pos, L.cap_raw)
        rows = torch.randn((n_raw, HEAD_DIM), generator=gen, device=dev)
        dst = torch.tensor([L.row_base + L.cap_comp + x % L.cap_raw for x in range(pos - n_raw, pos)],
                           dtype=torch.int64, device=dev)
        if n_raw:
            call("ds4hip_fp8_kv_quantize_append", _ptr(rows), n_raw, HEAD_DIM, N_ROT, _vp(s.codes),
                 _vp(s.sexp), _vp(s.tail), C.c_longlong(0), _ptr(dst), _stream(None))
        L.n_raw, L.raw_head = n_raw, pos % L.cap_raw
        if r:
            n_comp = min(pos // r, L.cap_comp)
            if n_comp:
                crow = torch.randn((n_comp, HEAD_DIM), generator=gen, device=dev)
                call("ds4hip_fp8_kv_quantize_append", _ptr(crow), n_comp, HEAD_DIM, N_ROT, _vp(s.codes),
                     _vp(s.sexp), _vp(s.tail), C.c_longlong(L.row_base), None, _stream(None))
            L.n_comp = n_comp
            coff = 2 if r == 4 else 1
            cells = coff * r * coff * HEAD_DIM
            for ptr in (L.attn_state_kv, L.attn_state_score):
                v = torch.randn(cells, generator=gen, device=dev)
                torch.cuda.synchronize()
                assert hip.hipMemcpy(ptr, v.data_ptr(), cells * 4, 3) == 0
            if L.has_indexer:
                keys = torch.randn((max(n_comp, 1), IDX_DIM), generator=gen, device=dev)
                torch.cuda.synchronize()
                if n_comp:
                    assert hip.hipMemcpy(L.index_comp_kv, keys.data_ptr(), n_comp * IDX_DIM * 4, 3) == 0
                L.n_index_comp = n_comp
                icells = 2 * 4 * 2 * IDX_DIM
                for ptr in (L.index_state_kv, L.index_state_score):
                    v = torch.randn(icells, generator=gen, device=dev)
                    torch.cuda.synchronize()
                    assert hip.hipMemcpy(ptr, v.data_ptr(), icells * 4, 3) == 0
    s.pos = pos
    s.n_tokens_processed = pos
    torch.cuda.synchronize()


class TokenSlice:
    """Steps 11-16 of all 43 layers for one token over `session`, with the
    given per-layer weights (synthetic_weights' layout). top_k: the indexer's
    selection size (512 in the model)."""

    def __init__(self, session: Session, weights, top_k: int = 512, fused: bool = True):
        self.session = session
        self.w = weights
        self.top_k = top_k
        # fused: each layer's push, compressor projections and indexer query /
        # weights as one launch (ds4hip_token_prologue_f32); otherwise one
        # launch each (the same values)
        self.fused = fused
        s = session.s
        dev = weights[0]["sinks"].device
        cap = max(1, max(s.layers[il].cap_comp for il in range(N_LAYER)))
        f = lambda n: torch.empty(n, dtype=torch.float32, device=dev)
        self.emit, self.kv_sc = f(HEAD_DIM), f(2 * 2 * HEAD_DIM)
        self.emit_i, self.kvi_sc = f(IDX_DIM), f(2 * 2 * IDX_DIM)
        self.q_idx, self.w_idx, self.scores = f(IDX_HEAD * IDX_DIM), f(IDX_HEAD), f(cap)
        self.select = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(cap), dtype=torch.uint8,
                                  device=dev)
        self.kqv = f(N_HEAD * HEAD_DIM)
        self.q_pre = torch.empty(q_prep_words(), dtype=torch.int32, device=dev)   # fused: Step 13's query
        # fused: Step 13's output as the merge writes it (rotated, Q8_0)
        self.kq8 = torch.empty(N_HEAD * HEAD_DIM, dtype=torch.int8, device=dev)
        self.kq8s = f(N_HEAD * HEAD_DIM // 32)
        self.out_ws = torch.empty(lib().ds4hip_attn_out_decode_workspace_bytes(N_HEAD, HEAD_DIM, N_OUT_GROUP,
                                                                               N_LORA_O),
                                  dtype=torch.uint8, device=dev)
        # the largest decode of any layer: the whole ring and every compressed row
        n_max = s.layers[0].cap_raw + cap
        self.dec_ws = torch.empty(decode_fp8_workspace_bytes([n_max]), dtype=torch.uint8, device=dev)

    def step(self, pos, kv_rope, attn_norm, q_cur, q_lora, out, stream=None):
        """kv_rope [43, 512], attn_norm [43, 4096], q_cur [43, 64, 512],
        q_lora [43, 1024] fp32 (each layer's producer outputs for this token);
        out [43, 4096] receives each layer's attention-slice output."""
        for t, n, nm in ((kv_rope, N_LAYER * HEAD_DIM, "kv_rope"), (attn_norm, N_LAYER * N_EMBD, "attn_norm"),
                         (q_cur, N_LAYER * N_HEAD * HEAD_DIM, "q_cur"), (q_lora, N_LAYER * Q_LORA, "q_lora"),
                         (out, N_LAYER * N_EMBD, "out")):
            _check(t, torch.float32, n, nm)
        sess, s = self.session, self.session.s
        st = _stream(stream)
        for il in range(N_LAYER):
            if self.fused:
                self._layer_fused(il, pos, kv_rope, attn_norm, q_cur, q_lora, out, stream)
                continue
            w = self.w[il]
            L = s.layers[il]
            r = L.compress_ratio
            x = attn_norm[il]
            # Step 11
            sess.push_raw(il, kv_rope[il], stream=stream)
            n_sel = -1
            if r:
                # Step 12a
                coff = 2 if r == 4 else 1
                e = C.c_int(0)
                call("ds4hip_compressor_decode_step_f32_prealloc", 1, _ptr(x), _ptr(w["comp_kv"]),
                     _ptr(w["comp_gate"]), _ptr(w["comp_ape"]), _ptr(w["comp_norm"]), N_EMBD, HEAD_DIM, r,
                     pos, il, _vp(L.attn_state_kv), _vp(L.attn_state_score), _ptr(self.emit), C.byref(e),
                     _ptr(self.kv_sc), _ptr(self.kv_sc[coff * HEAD_DIM:]), st)
                if e.value:
                    sess.push_comp(il, self.emit, stream=stream)
            if r == 4:
                # Step 12b
                ei = C.c_int(0)
                call("ds4hip_compressor_decode_step_f32_prealloc", 0, _ptr(x), _ptr(w["idx_kv"]),
                     _ptr(w["idx_gate"]), _ptr(w["idx_ape"]), _ptr(w["idx_norm"]), N_EMBD, IDX_DIM, r, pos,
                     il, _vp(L.index_state_kv), _vp(L.index_state_score), _ptr(self.emit_i), C.byref(ei),
                     _ptr(self.kvi_sc), _ptr(self.kvi_sc[2 * IDX_DIM:]), st)
                if ei.value:
                    sess.push_index_comp(il, self.emit_i, stream=stream)
                L = s.layers[il]
                if L.n_index_comp > self.top_k:
                    # Step 12c: indexer query, head weights, top-k into the row list
                    # the query with its RoPE, and the scaled head weights: one
                    # launch each (the fused forms of the matvec + RoPE / scale pairs)
                    call("ds4hip_mul_mv_f16_rope_f32", _ptr(w["idx_q_b"]), _ptr(q_lora[il]), _ptr(self.q_idx),
                         IDX_HEAD, IDX_DIM, N_ROT, pos, il, Q_LORA, st)
                    call("ds4hip_mul_mv_f16_scaled_f32", _ptr(w["idx_proj"]), _ptr(x), _ptr(self.w_idx), IDX_HEAD,
                         N_EMBD, C.c_float(1.0 / np.sqrt(IDX_DIM * IDX_HEAD)), st)
                    _, _, sel = sess.layer_rows(il, self.top_k)
                    call("ds4hip_indexer_topk_positions", _ptr(self.q_idx), _ptr(self.w_idx),
                         _vp(L.index_comp_kv), 0, L.n_index_comp, IDX_HEAD, IDX_DIM, self.top_k, 0,
                         _ptr(self.scores), _ptr(self.select), None, _vp(sel), st)
                    n_sel = self.top_k
            # Step 13
            sess.decode(il, q_cur[il].reshape(-1), w["sinks"], self.kqv, n_selected=n_sel,
                        workspace=self.dec_ws, stream=stream)
            # Steps 14-16: inverse RoPE + quantization in one launch, then the
            # grouped and the dense Q8_0 projections
            call("ds4hip_attn_out_decode_f32", _ptr(self.kqv), _ptr(w["out_a"]), _ptr(w["out_b"]), _ptr(out[il]),
                 N_HEAD, HEAD_DIM, N_ROT, pos, il, N_OUT_GROUP, N_LORA_O, N_EMBD, _ptr(self.out_ws),
                 self.out_ws.numel(), st)
        s.pos = pos + 1
        s.n_tokens_processed = pos + 1

    def _layer_fused(self, il, pos, kv_rope, attn_norm, q_cur, q_lora, out, stream):
        """One layer of step() with Steps 11-12c's independent launches as one."""
        sess, s = self.session, self.session.s
        st = _stream(stream)
        w = self.w[il]
        L = s.layers[il]
        r = L.compress_ratio
        x = attn_norm[il]
        P = TokenPrologue()
        # Step 11: the FP8 push into the ring row the session hands out
        P.kv, P.codes, P.sexp, P.tail = _ptr(kv_rope[il]), s.codes, s.sexp, s.tail
        P.kv_row = sess.claim_raw_row(il)
        P.head_dim, P.n_rot = HEAD_DIM, N_ROT
        P.x, P.in_dim = _ptr(x), N_EMBD
        emit = bool(r) and (pos + 1) % r == 0
        if r:   # Step 12a (and 12b): the projections
            P.n_comp = 2 if r == 4 else 1
            P.comp0_w_kv, P.comp0_w_gate, P.comp0_w_ape = _ptr(w["comp_kv"]), _ptr(w["comp_gate"]), _ptr(w["comp_ape"])
            P.comp0_state_kv, P.comp0_state_score = L.attn_state_kv, L.attn_state_score
            P.comp0_head_dim_out, P.comp0_ratio, P.comp0_pos = HEAD_DIM, r, pos
            if r == 4:
                P.comp1_w_kv, P.comp1_w_gate, P.comp1_w_ape = _ptr(w["idx_kv"]), _ptr(w["idx_gate"]), _ptr(w["idx_ape"])
                P.comp1_state_kv, P.comp1_state_score = L.index_state_kv, L.index_state_score
                P.comp1_head_dim_out, P.comp1_ratio, P.comp1_pos = IDX_DIM, r, pos
        # Step 12c runs when the indexer holds more than top_k keys after this step
        select = r == 4 and L.n_index_comp + (1 if emit else 0) > self.top_k
        if select:
            P.q_w, P.q_x, P.q_out = _ptr(w["idx_q_b"]), _ptr(q_lora[il]), _ptr(self.q_idx)
            P.q_heads, P.q_head_dim, P.q_in, P.q_pos, P.q_il = IDX_HEAD, IDX_DIM, Q_LORA, pos, il
            P.hw_w, P.hw_out, P.hw_rows = _ptr(w["idx_proj"]), _ptr(self.w_idx), IDX_HEAD
            P.hw_scale = 1.0 / np.sqrt(IDX_DIM * IDX_HEAD)
        # the decode query, converted for Step 13's kernel
        P.qp_q, P.qp_out = _ptr(q_cur[il]), _ptr(self.q_pre)
        call("ds4hip_token_prologue_f32", C.byref(P), st)
        if emit:   # the emits and their row pushes
            call("ds4hip_compressor_emit_f32", 1, _ptr(w["comp_norm"]), HEAD_DIM, r, pos, il,
                 _vp(L.attn_state_kv), _vp(L.attn_state_score), _ptr(self.emit), st)
            sess.push_comp(il, self.emit, stream=stream)
            if r == 4:
                call("ds4hip_compressor_emit_f32", 0, _ptr(w["idx_norm"]), IDX_DIM, r, pos, il,
                     _vp(L.index_state_kv), _vp(L.index_state_score), _ptr(self.emit_i), st)
                sess.push_index_comp(il, self.emit_i, stream=stream)
        n_sel = -1
        L = s.layers[il]
        if select:
            _, _, sel = sess.layer_rows(il, self.top_k)
            call("ds4hip_indexer_topk_positions", _ptr(self.q_idx), _ptr(self.w_idx),
                 _vp(L.index_comp_kv), 0, L.n_index_comp, IDX_HEAD, IDX_DIM, self.top_k, 0,
                 _ptr(self.scores), _ptr(self.select), None, _vp(sel), st)
            n_sel = self.top_k
        # Step 13, its merge writing Step 14's inverse RoPE and the first Q8_0
        # quantization of Step 15
        sess.decode(il, self.q_pre, w["sinks"], self.kqv, n_selected=n_sel, workspace=self.dec_ws,
                    rope_q8=(self.kq8, self.kq8s, pos, il), stream=stream)
        # Steps 15-16
        call("ds4hip_attn_out_decode_q8_f32", _ptr(self.kq8), _ptr(self.kq8s), _ptr(w["out_a"]), _ptr(w["out_b"]),
             _ptr(out[il]), N_HEAD, HEAD_DIM, N_OUT_GROUP, N_LORA_O, N_EMBD, _ptr(self.out_ws),
             self.out_ws.numel(), st)

    def capture(self, pos, kv_rope, attn_norm, q_cur, q_lora, out):
        """Records step(pos, ...) into a HIP graph (torch.cuda.CUDAGraph) and
        returns it. The capture runs no kernel but advances the session's
        host-side counters as step() would, so the graph's first replay
        leaves the session exactly as an eager step(pos) does."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                self.step(pos, kv_rope, attn_norm, q_cur, q_lora, out, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        return g
