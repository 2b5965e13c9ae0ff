"""KV push / SWA eviction and the FP8 session arena (include/ds4hip_session.h).

`swa_push_f32` / `comp_push_f32` keep the reference's fp32 row layout
(cuda/forward_layer.cu:159-190,941-972,1021-1034). `Session` owns the FP8
form of ds4_session_state (include/ds4cuda.h:310-443,
cuda/session_state.cu:110-256): one device arena, per-layer FP8 rows
(compressed rows, then a 128-row SWA ring), compressor and indexer state.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

from ._lib import Ds4HipError, call, lib
from .ops import _check, _ptr, _stream

N_LAYER = 43
N_SWA = 128
CHUNK_STAGING_ROWS = 128   # staging rows of a prefill chunk after the layers' rows
ENOSPC = -28


class LayerState(C.Structure):
    _fields_ = [("il", C.c_int), ("compress_ratio", C.c_int), ("has_indexer", C.c_int),
                ("cap_raw", C.c_int), ("n_raw", C.c_int), ("raw_head", C.c_int),
                ("cap_comp", C.c_int), ("n_comp", C.c_int), ("n_index_comp", C.c_int),
                ("row_base", C.c_longlong), ("row_list", C.c_void_p),
                ("attn_state_kv", C.c_void_p), ("attn_state_score", C.c_void_p),
                ("index_comp_kv", C.c_void_p), ("index_state_kv", C.c_void_p),
                ("index_state_score", C.c_void_p)]


class SessionState(C.Structure):
    _fields_ = [("max_context", C.c_int), ("pos", C.c_int), ("n_tokens_processed", C.c_int),
                ("layers", LayerState * N_LAYER), ("codes", C.c_void_p), ("sexp", C.c_void_p),
                ("tail", C.c_void_p), ("n_cache_rows", C.c_longlong),
                ("codes_bytes", C.c_size_t), ("arena_base", C.c_void_p),
                ("arena_bytes", C.c_size_t)]


class Ds4cudakInfo(C.Structure):
    """ds4hip_ds4cudak_info: what ds4hip_ds4cudak_probe reads from a
    reference session file."""
    _fields_ = [("max_context", C.c_int), ("pos", C.c_int), ("n_tokens_processed", C.c_int),
                ("cap_raw", C.c_int), ("n_prompt_tokens", C.c_int),
                ("prompt_token_ids", C.c_int32 * 64), ("n_raw", C.c_int * N_LAYER),
                ("n_comp", C.c_int * N_LAYER), ("n_index_comp", C.c_int * N_LAYER),
                ("file_bytes", C.c_longlong)]


def probe_ds4cudak(path) -> Ds4cudakInfo:
    """Checks a reference (fp32, "DS4CUDAK") session file on the host and
    returns its header fields and per-layer counts; raises Ds4HipError."""
    info = Ds4cudakInfo()
    lib().ds4hip_clear_last_error()
    if lib().ds4hip_ds4cudak_probe(os.fsencode(path), C.byref(info)) != 0:
        raise Ds4HipError("ds4hip_ds4cudak_probe", lib().ds4hip_get_last_error())
    return info


def swa_push_f32(raw_kv, n_raw, cap_raw, kv_cur, head_dim, stream=None) -> int:
    """Returns the new n_raw."""
    _check(raw_kv, torch.float32, cap_raw * head_dim, "raw_kv")
    _check(kv_cur, torch.float32, head_dim, "kv_cur")
    n = C.c_int(n_raw)
    call("ds4hip_swa_push_f32", _ptr(raw_kv), C.byref(n), cap_raw, _ptr(kv_cur), head_dim,
         _stream(stream))
    return n.value


def comp_push_f32(comp_kv, n_comp, cap_comp, row, head_dim, stream=None) -> int:
    """Returns the new n_comp; raises Ds4HipError(-28) when the cache is full."""
    _check(row, torch.float32, head_dim, "row")
    n = C.c_int(n_comp)
    call("ds4hip_comp_push_f32", _ptr(comp_kv), C.byref(n), cap_comp, _ptr(row), head_dim,
         _stream(stream))
    return n.value


def arena_bytes(max_context: int) -> int:
    return lib().ds4hip_session_state_arena_bytes(max_context)


class Session:
    """Owns one ds4hip_session_state. The FP8 cache is exposed as torch views
    (codes [rows,448] u8, sexp [rows,8] i8, tail [rows,64] int16) for the
    decode launcher."""

    def __init__(self, max_context: int):
        self.s = SessionState()
        call("ds4hip_session_state_alloc", C.byref(self.s), max_context)

    def close(self):
        if self.s.arena_base:
            call("ds4hip_session_state_free", C.byref(self.s))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def layer(self, il) -> LayerState:
        return self.s.layers[il]

    def reset(self, stream=None):
        call("ds4hip_session_state_reset", C.byref(self.s), _stream(stream))

    def push_raw(self, il, kv_cur, stream=None):
        _check(kv_cur, torch.float32, 512, "kv_cur")
        call("ds4hip_session_push_raw", C.byref(self.s), il, _ptr(kv_cur), _stream(stream))

    def claim_raw_row(self, il) -> int:
        """Arena row of the next raw push, with the ring counters advanced
        (for a push written by the caller's own launch)."""
        row = C.c_longlong()
        call("ds4hip_session_claim_raw_row", C.byref(self.s), il, C.byref(row))
        return row.value

    def push_comp(self, il, row, stream=None):
        _check(row, torch.float32, 512, "row")
        call("ds4hip_session_push_comp", C.byref(self.s), il, _ptr(row), _stream(stream))

    def push_index_comp(self, il, row, stream=None):
        _check(row, torch.float32, 128, "row")
        call("ds4hip_session_push_index_comp", C.byref(self.s), il, _ptr(row), _stream(stream))

    def save(self, path, prompt_token_ids=None):
        """Writes the session to path (format in include/ds4hip_session.h);
        at most the first 64 prompt token ids are stored."""
        ids = [] if prompt_token_ids is None else [int(t) for t in prompt_token_ids]
        arr = (C.c_int32 * max(len(ids), 1))(*ids)
        self._persist("ds4hip_session_save_to_disk", C.byref(self.s), arr if ids else None,
                      len(ids), os.fsencode(path))

    def load(self, path):
        """Restores a saved session (same max_context); returns (pos, n_tokens_processed)."""
        pos, n = C.c_int(), C.c_int()
        self._persist("ds4hip_session_load_from_disk", C.byref(self.s), os.fsencode(path),
                      C.byref(pos), C.byref(n))
        return pos.value, n.value

    def import_ds4cudak(self, path):
        """Loads a reference session file (fp32 rows) into this FP8 session
        (same max_context); returns (pos, n_tokens_processed)."""
        pos, n = C.c_int(), C.c_int()
        self._persist("ds4hip_session_import_ds4cudak", C.byref(self.s), os.fsencode(path),
                      C.byref(pos), C.byref(n))
        return pos.value, n.value

    def export_ds4cudak(self, path, prompt_token_ids=None):
        """Writes this session as a reference (fp32, "DS4CUDAK") session file."""
        ids = [] if prompt_token_ids is None else [int(t) for t in prompt_token_ids]
        arr = (C.c_int32 * max(len(ids), 1))(*ids)
        self._persist("ds4hip_session_export_ds4cudak", C.byref(self.s), arr if ids else None, len(ids),
                      os.fsencode(path))

    @staticmethod
    def _persist(name, *args):
        # these two return -1 on any error (the reference's convention); the
        # detailed status is the library's last error
        lib().ds4hip_clear_last_error()
        if getattr(lib(), name)(*args) != 0:
            raise Ds4HipError(name, lib().ds4hip_get_last_error())

    def rows_from(self, row):
        """Arena rows from cache row `row` on: the layers' rows and the prefill
        chunk's staging rows after them."""
        return self.s.n_cache_rows + CHUNK_STAGING_ROWS - row

    def layer_rows(self, il, n_selected=-1):
        """(row_idx device address, n_rows, selected device address)."""
        ri, n, sel = C.c_void_p(), C.c_longlong(), C.c_void_p()
        call("ds4hip_session_layer_rows", C.byref(self.s), il, n_selected, C.byref(ri),
             C.byref(n), C.byref(sel))
        return ri.value, n.value, sel.value

    def decode(self, il, q, sinks, out, n_selected=-1, workspace=None, exact_p=False, rope_q8=None,
               stream=None):
        """Decode attention of one query (q [64,512] bf16/fp32, or an fp32 one
        converted by ops.flash_attn_q_prep_f32 / the token prologue) over layer il's
        valid ring rows plus its first n_selected compressed rows (all n_comp
        when n_selected < 0; the selection written at layer_rows()' selected
        address otherwise). exact_p: P as f16 hi + lo (the register kernels)
        instead of one f16 (the flat-stage kernel). rope_q8: see
        ops.decode_opts (the merge writes the rotated Q8_0 rows instead of out)."""
        from .ops import HEAD_DIM, N_HEAD, _q_mode, decode_fp8_workspace_bytes, decode_opts, N_ROT
        ri, n, _ = self.layer_rows(il, n_selected)
        q_mode, q_stride = _q_mode(q)
        _check(q, q.dtype, q_stride, "q")
        _check(sinks, torch.float32, N_HEAD, "sinks")
        _check(out, torch.float32, N_HEAD * HEAD_DIM, "out")
        counts = (C.c_longlong * 1)(n)
        need = decode_fp8_workspace_bytes([n])
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        rb = self.layer(il).row_base      # the layer's rows start at its row_base
        call("ds4hip_flash_attn_decode_fp8", _ptr(q), q_mode, q_stride, _ptr(sinks), N_HEAD, _ptr(out), N_HEAD * HEAD_DIM,
             C.c_void_p(self.s.codes + rb * 448), C.c_void_p(self.s.sexp + rb * 8),
             C.c_void_p(self.s.tail + rb * 128), C.cast(counts, C.c_void_p), 1, None, 0,
             C.c_void_p(ri),
             0, None, 0, 256, N_HEAD, HEAD_DIM, N_ROT, C.c_longlong(self.rows_from(rb)),
             C.byref(decode_opts(exact_p, rope_q8=rope_q8)), _ptr(workspace), workspace.numel(), 3,
             _stream(stream))
        return workspace
