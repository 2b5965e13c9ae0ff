"""Python mirror of the ds4cuda attention-path launchers over libds4hip.so.

Names, argument order and meaning follow the reference launchers
(cuda/flash_attn.cuh, cuda/fp8_kv.cuh, cuda/indexer_allowed.cuh,
cuda/compressor.cuh, cuda/attn_out.cuh, cuda/rope.cuh, cuda/router.cuh).
Device buffers are torch tensors on the GPU (torch is used for memory and
streams only); every call goes through the C-ABI. Where the reference prints
and drops a launch on a bad shape, these wrappers raise Ds4HipError.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from ._lib import Ds4HipError, call

N_HEAD = 64
HEAD_DIM = 512
N_ROT = 64
N_NOPE = HEAD_DIM - N_ROT
FP8_ROW_BYTES = N_NOPE + 8 + 2 * N_ROT   # 584


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, torch.cuda.Stream):
        return C.c_void_p(stream.cuda_stream)
    return C.c_void_p(stream)


def _check(t, dtype, numel=None, name="tensor"):
    if t is None:
        return
    if t.dtype != dtype or not t.is_contiguous():
        raise Ds4HipError(f"{name}: expected contiguous {dtype}, got {t.dtype}", -22)
    if numel is not None and t.numel() < numel:
        raise Ds4HipError(f"{name}: needs {numel} elements, has {t.numel()}", -22)


# ---- fp8_kv (cuda/fp8_kv.cuh:62) ---------------------------------------------------

def launch_fp8_kv_quantize_round_trip_f32(kv_in, kv_out, n_rows, head_dim, n_rot, stream=None):
    _check(kv_in, torch.float32, n_rows * head_dim, "kv_in")
    _check(kv_out, torch.float32, n_rows * head_dim, "kv_out")
    call("ds4hip_fp8_kv_quantize_round_trip_f32", _ptr(kv_in), _ptr(kv_out), n_rows, head_dim,
         n_rot, _stream(stream))


@dataclass
class Fp8KVCache:
    """FP8 E4M3FN KV cache rows: codes [rows,448] u8, sexp [rows,8] i8,
    tail [rows,64] f16 bits (as int16). 584 bytes per row."""
    codes: torch.Tensor
    sexp: torch.Tensor
    tail: torch.Tensor

    @staticmethod
    def empty(n_rows: int, device="cuda"):
        return Fp8KVCache(
            codes=torch.zeros((n_rows, N_NOPE), dtype=torch.uint8, device=device),
            sexp=torch.zeros((n_rows, 8), dtype=torch.int8, device=device),
            tail=torch.zeros((n_rows, N_ROT), dtype=torch.int16, device=device))

    @property
    def n_rows(self) -> int:
        return self.codes.shape[0]

    def append(self, kv, row0=0, dst_rows=None, stream=None):
        """Quantize fp32 rows kv [n, 512] into rows row0.. (or dst_rows, int64)."""
        n = kv.shape[0]
        _check(kv, torch.float32, n * HEAD_DIM, "kv")
        if dst_rows is not None:
            _check(dst_rows, torch.int64, n, "dst_rows")
        elif row0 + n > self.n_rows:
            raise Ds4HipError("append past the end of the cache", -22)
        call("ds4hip_fp8_kv_quantize_append", _ptr(kv), n, HEAD_DIM, N_ROT, _ptr(self.codes),
             _ptr(self.sexp), _ptr(self.tail), int(row0), _ptr(dst_rows), _stream(stream))


# ---- flash_attn (cuda/flash_attn.cuh:73,142) ----------------------------------------

def launch_flash_attn_decode_raw_f32(Q, K, V, sinks, out, n_head, n_kv, head_dim, stream=None):
    for t, n, nm in ((Q, n_head * head_dim, "Q"), (K, n_kv * head_dim, "K"),
                     (sinks, n_head, "sinks"), (out, n_head * head_dim, "out")):
        _check(t, torch.float32, n, nm)
    call("ds4hip_flash_attn_decode_raw_f32", _ptr(Q), _ptr(K), _ptr(V), _ptr(sinks), _ptr(out),
         n_head, n_kv, head_dim, _stream(stream))


def launch_flash_attn_decode_mixed_f32(Q, raw_kv, comp_kv, comp_allowed, sinks, out, n_head,
                                       n_raw, n_comp, head_dim, stream=None):
    _check(Q, torch.float32, n_head * head_dim, "Q")
    _check(raw_kv, torch.float32, n_raw * head_dim, "raw_kv")
    _check(comp_kv, torch.float32, n_comp * head_dim, "comp_kv")
    _check(comp_allowed, torch.int32, n_comp, "comp_allowed")
    call("ds4hip_flash_attn_decode_mixed_f32", _ptr(Q), _ptr(raw_kv), _ptr(comp_kv),
         _ptr(comp_allowed), _ptr(sinks), _ptr(out), n_head, n_raw, n_comp, head_dim,
         _stream(stream))


def decode_fp8_workspace_bytes(n_rows_per_prob) -> int:
    arr = (C.c_longlong * len(n_rows_per_prob))(*[int(x) for x in n_rows_per_prob])
    out = C.c_size_t(0)
    call("ds4hip_flash_attn_decode_fp8_workspace_size", C.cast(arr, C.c_void_p),
         len(n_rows_per_prob), C.byref(out))
    return out.value


def flash_attn_decode_fp8(q, sinks, out, cache: Fp8KVCache, n_rows_per_prob, *, row_base=None,
                          row_base_stride=0, row_idx=None, page_table=None, page_rows=256,
                          workspace=None, phases=3, stream=None):
    """Decode attention of n_prob single-query problems over the FP8 cache.

    q [n_prob, 64, 512] bf16 or fp32; sinks [n_prob, 64] fp32; out
    [n_prob, 64, 512] fp32; n_rows_per_prob: host ints. Row r of problem p is
    position row_idx[p, r] (or r), mapped through page_table[p] (pages of
    page_rows rows) or offset by row_base[p] (int64 tensor) / p*row_base_stride.
    """
    n_prob = len(n_rows_per_prob)
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise Ds4HipError("q must be bf16 or fp32", -22)
    _check(q, q.dtype, n_prob * N_HEAD * HEAD_DIM, "q")
    _check(sinks, torch.float32, n_prob * N_HEAD, "sinks")
    _check(out, torch.float32, n_prob * N_HEAD * HEAD_DIM, "out")
    _check(row_base, torch.int64, n_prob, "row_base")
    _check(row_idx, torch.int32, None, "row_idx")
    _check(page_table, torch.int32, None, "page_table")
    counts = (C.c_longlong * n_prob)(*[int(x) for x in n_rows_per_prob])
    need = decode_fp8_workspace_bytes(n_rows_per_prob)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    call("ds4hip_flash_attn_decode_fp8", _ptr(q), int(q.dtype == torch.float32),
         N_HEAD * HEAD_DIM, _ptr(sinks), N_HEAD, _ptr(out), N_HEAD * HEAD_DIM,
         _ptr(cache.codes), _ptr(cache.sexp), _ptr(cache.tail), C.cast(counts, C.c_void_p),
         n_prob, _ptr(row_base), int(row_base_stride), _ptr(row_idx),
         row_idx.shape[-1] if row_idx is not None else 0, _ptr(page_table),
         page_table.shape[-1] if page_table is not None else 0, int(page_rows), N_HEAD,
         HEAD_DIM, N_ROT, _ptr(workspace), workspace.numel(), int(phases), _stream(stream))
    return workspace
