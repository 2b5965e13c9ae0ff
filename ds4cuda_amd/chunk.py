"""Prefill chunk driver: one layer's attention slice for N prompt tokens at once.

The reference prefills a chunk layer by layer and, inside a layer, token by
token (ds4_forward_chunk, cuda/forward_batch.cu:264-284: for il { for t {
ds4_forward_layer } }). Its header names the batched form as the next step
(cuda/forward_batch.cuh:27-35,52-55). This module is that form for the
attention slice of one layer over the FP8 session (Session):

  1. the chunk's KV rows (Step 11) are quantized into the session's staging
     rows (one launch), so every token of the chunk can see the rows of the
     earlier chunk tokens while the ring still holds the window before p0;
  2. per token, in position order, the steps whose state carries from one
     token to the next: the attention compressor (and on ratio-4 layers the
     indexer compressor) with their emitted rows appended to the session, and
     on ratio-4 layers the indexer selection of the token's compressed rows
     (Step 12, cuda/forward_layer.cu:997-1132);
  3. one multi-problem FP8 decode launch computes all N tokens' attention
     (Step 13): token t attends the window rows still in the ring, staging
     rows 0..t and its compressed rows (ds4hip_session_chunk_rows);
  4. the chunk's rows are pushed into the ring in order, which leaves the
     session exactly as N single-token steps would.

Every kernel is a libds4hip.so entry point; torch provides device memory and
the stream only.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import Ds4HipError, call, lib
from .ops import _ptr, _stream

N_HEAD, HEAD_DIM, N_ROT, IDX_DIM, N_EMBD = 64, 512, 64, 128, 4096
CHUNK_MAX = 128
INDEXER_TOP_K = 512


def _vp(x):
    return C.c_void_p(x)


class ChunkLayer:
    """Compressor / indexer weights of one layer (device tensors, the
    reference's dtypes): comp_kv, comp_gate [coff*512, 4096] f16 bits (int16),
    comp_ape [ratio, coff*512] f16 bits, comp_norm [512] fp32; on ratio-4
    layers also idx_kv, idx_gate [2*128, 4096], idx_ape [4, 256], idx_norm
    [128], and the indexer query / head-weight projections idx_q_b
    [64*128, 1024] and idx_proj [64, 4096] (f16 bits)."""

    def __init__(self, weights: dict, top_k: int = INDEXER_TOP_K):
        self.w = weights
        self.top_k = top_k


def forward_chunk_attn(session, il, p0, attn_norm, q_lora_norm, q_cur, kv_rope, sinks, out,
                       layer: ChunkLayer | None = None, workspace=None, exact_p=False, stream=None):
    """Attention slice of layer il for the n tokens at positions p0 .. p0+n-1
    of the session (n <= 128). attn_norm [n, 4096], q_lora_norm [n, 1024],
    q_cur [n, 64, 512], kv_rope [n, 512] fp32 (the producer's outputs, e.g.
    ops.attn_qkv_decode_f32 per token); sinks [64]; out [n, 64, 512] receives
    each token's attention output (Step 13's kqv). exact_p: the decode's P as
    f16 hi + lo (as Session.decode). Returns the workspace."""
    from .ops import _check, decode_fp8_workspace_bytes, decode_opts
    n = kv_rope.shape[0]
    if not 0 < n <= CHUNK_MAX:
        raise Ds4HipError("chunk of 1..128 tokens", -22)
    _check(kv_rope, torch.float32, n * HEAD_DIM, "kv_rope")
    _check(attn_norm, torch.float32, n * N_EMBD, "attn_norm")
    _check(q_lora_norm, torch.float32, n * 1024, "q_lora_norm")
    _check(q_cur, torch.float32, n * N_HEAD * HEAD_DIM, "q_cur")
    _check(sinks, torch.float32, N_HEAD, "sinks")
    _check(out, torch.float32, n * N_HEAD * HEAD_DIM, "out")
    s = session.s
    L = s.layers[il]
    ratio = L.compress_ratio
    if ratio and layer is None:
        raise Ds4HipError("compressed layer needs its compressor weights", -22)
    dev = kv_rope.device
    st = _stream(stream)
    # 1. the chunk's KV rows into the staging rows
    call("ds4hip_fp8_kv_quantize_append", _ptr(kv_rope), n, HEAD_DIM, N_ROT, _vp(s.codes), _vp(s.sexp),
         _vp(s.tail), C.c_longlong(s.n_cache_rows), None, st)
    # 2. per token: compressors, emitted rows, indexer selection
    n_comp = np.zeros(n, np.int32)
    n_sel = np.zeros(n, np.int32)
    sel = None
    if ratio:
        w = layer.w
        coff = 2 if ratio == 4 else 1
        emit = torch.empty(HEAD_DIM, device=dev)
        kv_sc = torch.empty(2 * coff * HEAD_DIM, device=dev)
        if ratio == 4:
            emit_i = torch.empty(IDX_DIM, device=dev)
            kvi_sc = torch.empty(2 * coff * IDX_DIM, device=dev)
            q_idx = torch.empty(N_HEAD * IDX_DIM, device=dev)
            w_idx = torch.empty(N_HEAD, device=dev)
            sel = torch.empty((n, layer.top_k), dtype=torch.int32, device=dev)
            scores = torch.empty(max(L.cap_comp, 1), device=dev)
            select = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(max(L.cap_comp, 1)),
                                 dtype=torch.uint8, device=dev)
        for t in range(n):
            pos = p0 + t
            x = attn_norm[t]
            e = C.c_int(0)
            call("ds4hip_compressor_decode_step_f32_prealloc", 1, _ptr(x), _ptr(w["comp_kv"]),
                 _ptr(w["comp_gate"]), _ptr(w["comp_ape"]), _ptr(w["comp_norm"]), N_EMBD, HEAD_DIM,
                 ratio, pos, il, _vp(L.attn_state_kv), _vp(L.attn_state_score), _ptr(emit),
                 C.byref(e), _ptr(kv_sc), _ptr(kv_sc[coff * HEAD_DIM:]), st)
            if e.value:
                session.push_comp(il, emit, stream=stream)
            if ratio == 4:
                ei = C.c_int(0)
                call("ds4hip_compressor_decode_step_f32_prealloc", 0, _ptr(x), _ptr(w["idx_kv"]),
                     _ptr(w["idx_gate"]), _ptr(w["idx_ape"]), _ptr(w["idx_norm"]), N_EMBD, IDX_DIM,
                     ratio, pos, il, _vp(L.index_state_kv), _vp(L.index_state_score), _ptr(emit_i),
                     C.byref(ei), _ptr(kvi_sc), _ptr(kvi_sc[coff * IDX_DIM:]), st)
                if ei.value:
                    session.push_index_comp(il, emit_i, stream=stream)
            L = s.layers[il]
            n_comp[t] = L.n_comp
            n_sel[t] = L.n_comp
            if ratio == 4 and L.n_index_comp > layer.top_k:
                # indexer query and head weights of the token (Step 12b)
                call("ds4hip_mul_mv_f16_f32", _ptr(w["idx_q_b"]), _ptr(q_lora_norm[t]), _ptr(q_idx),
                     N_HEAD * IDX_DIM, 1024, st)
                call("ds4hip_tail_rope_yarn_f32", _ptr(q_idx), _ptr(q_idx), N_HEAD, IDX_DIM, N_ROT, pos,
                     il, st)
                call("ds4hip_mul_mv_f16_f32", _ptr(w["idx_proj"]), _ptr(x), _ptr(w_idx), N_HEAD, N_EMBD,
                     st)
                call("ds4hip_scale_inplace_f32", _ptr(w_idx), N_HEAD,
                     C.c_float(1.0 / np.sqrt(IDX_DIM * N_HEAD)), st)
                call("ds4hip_indexer_topk_positions", _ptr(q_idx), _ptr(w_idx), _vp(L.index_comp_kv), 0,
                     L.n_index_comp, N_HEAD, IDX_DIM, layer.top_k, 0, _ptr(scores), _ptr(select), None,
                     _ptr(sel[t]), st)
                n_sel[t] = layer.top_k
    # 3. all tokens' attention in one decode launch
    # list stride: the longest token list (window rows still in the ring, the
    # chunk's own rows up to the token, its compressed rows), from the layer's
    # ring capacity; ds4hip_session_chunk_rows refuses a stride too short
    n_ring0 = min(p0, L.cap_raw - 1)
    stride = (n_ring0 + n + int(n_sel.max()) + 63) // 64 * 64
    lists = torch.empty((n, stride), dtype=torch.int32, device=dev)
    # the decode and the list kernel read these on the device
    _check(lists, torch.int32, n * stride, "lists")
    if sel is not None:
        _check(sel, torch.int32, n * layer.top_k, "sel")
    counts = (C.c_longlong * n)()
    call("ds4hip_session_chunk_rows", C.byref(s), il, p0, n, n_comp.ctypes.data_as(C.c_void_p),
         n_sel.ctypes.data_as(C.c_void_p), _ptr(sel), sel.shape[1] if sel is not None else 0, _ptr(lists),
         stride, C.cast(counts, C.c_void_p), st)
    cnt = [int(c) for c in counts]
    need = decode_fp8_workspace_bytes(cnt)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    # the list entries are relative to the layer's first row: the cache
    # pointers start there and every problem's base is 0 (row_base NULL,
    # stride 0), as in Session.decode
    rb = int(L.row_base)
    call("ds4hip_flash_attn_decode_fp8", _ptr(q_cur), 1, N_HEAD * HEAD_DIM, _ptr(sinks), 0, _ptr(out),
         N_HEAD * HEAD_DIM, _vp(s.codes + rb * 448), _vp(s.sexp + rb * 8), _vp(s.tail + rb * 128),
         C.cast(counts, C.c_void_p), n, None, 0, _ptr(lists), stride, None, 0, 256, N_HEAD, HEAD_DIM,
         N_ROT, C.c_longlong(session.rows_from(rb)), C.byref(decode_opts(exact_p)), _ptr(workspace),
         workspace.numel(), 3, st)
    # the last token's selection stays in the layer's row list, where the
    # token-by-token loop leaves it
    if sel is not None and n_sel[-1] < n_comp[-1]:
        call("ds4hip_session_set_selection", C.byref(s), il, _ptr(sel[n - 1]), int(n_sel[-1]), st)
    # 4. the chunk's rows into the ring, in position order
    for t in range(n):
        session.push_raw(il, kv_rope[t], stream=stream)
    return workspace
