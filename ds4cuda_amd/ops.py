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

from ._lib import Ds4HipError, call, lib

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
    if t.device.type != "cuda":
        # the kernels read and write these buffers: host memory here would
        # fault the GPU instead of failing the call
        raise Ds4HipError(f"{name}: expected a GPU tensor, got one on {t.device}", -22)
    if t.dtype != dtype or not t.is_contiguous():
        raise Ds4HipError(f"{name}: expected contiguous {dtype}, got {t.dtype}", -22)
    if numel is not None and t.numel() < numel:
        raise Ds4HipError(f"{name}: needs {numel} elements, has {t.numel()}", -22)


def _dev(t, name, nbytes=None):
    """Device-memory check for a buffer the kernels use as raw bytes
    (workspaces, scratch): any dtype, but on the GPU and large enough."""
    if t is None:
        raise Ds4HipError(f"{name}: a GPU tensor is required", -22)
    if t.device.type != "cuda":
        raise Ds4HipError(f"{name}: expected a GPU tensor, got one on {t.device}", -22)
    if not t.is_contiguous():
        raise Ds4HipError(f"{name}: expected a contiguous tensor", -22)
    if nbytes is not None and t.numel() * t.element_size() < nbytes:
        raise Ds4HipError(f"{name}: needs {nbytes} bytes, has {t.numel() * t.element_size()}", -22)


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
                     (V, n_kv * head_dim, "V"), (sinks, n_head, "sinks"),
                     (out, n_head * head_dim, "out")):
        _check(t, torch.float32, n, nm)
    call("ds4hip_flash_attn_decode_raw_f32", _ptr(Q), _ptr(K), _ptr(V), _ptr(sinks), _ptr(out),
         n_head, n_kv, head_dim, _stream(stream))


def decode_f32_workspace(n_rows, device):
    """Workspace (uint8 tensor) of the _prealloc fp32 decode launchers."""
    out = C.c_size_t(0)
    call("ds4hip_flash_attn_decode_f32_workspace_size", int(n_rows), C.byref(out))
    return torch.empty(max(out.value, 1), dtype=torch.uint8, device=device)


def launch_flash_attn_decode_raw_f32_prealloc(Q, K, V, sinks, out, n_head, n_kv, head_dim,
                                              workspace, stream=None):
    for t, n, nm in ((Q, n_head * head_dim, "Q"), (K, n_kv * head_dim, "K"),
                     (V, n_kv * head_dim, "V"), (sinks, n_head, "sinks"),
                     (out, n_head * head_dim, "out")):
        _check(t, torch.float32, n, nm)
    _dev(workspace, "workspace")
    call("ds4hip_flash_attn_decode_raw_f32_prealloc", _ptr(Q), _ptr(K), _ptr(V), _ptr(sinks),
         _ptr(out), n_head, n_kv, head_dim, _ptr(workspace), workspace.numel(), _stream(stream))


def launch_flash_attn_decode_mixed_f32(Q, raw_kv, comp_kv, comp_allowed, sinks, out, n_head,
                                       n_raw, n_comp, head_dim, stream=None):
    _check(Q, torch.float32, n_head * head_dim, "Q")
    _check(raw_kv, torch.float32, n_raw * head_dim, "raw_kv")
    _check(comp_kv, torch.float32, n_comp * head_dim, "comp_kv")
    _check(comp_allowed, torch.int32, n_comp, "comp_allowed")
    _check(sinks, torch.float32, n_head, "sinks")
    _check(out, torch.float32, n_head * head_dim, "out")
    call("ds4hip_flash_attn_decode_mixed_f32", _ptr(Q), _ptr(raw_kv), _ptr(comp_kv),
         _ptr(comp_allowed), _ptr(sinks), _ptr(out), n_head, n_raw, n_comp, head_dim,
         _stream(stream))


def launch_flash_attn_decode_mixed_f32_prealloc(Q, raw_kv, comp_kv, comp_allowed, sinks, out,
                                                n_head, n_raw, n_comp, head_dim, workspace,
                                                stream=None):
    _check(Q, torch.float32, n_head * head_dim, "Q")
    _check(raw_kv, torch.float32, n_raw * head_dim, "raw_kv")
    _check(comp_kv, torch.float32, n_comp * head_dim, "comp_kv")
    _check(comp_allowed, torch.int32, n_comp, "comp_allowed")
    _check(sinks, torch.float32, n_head, "sinks")
    _check(out, torch.float32, n_head * head_dim, "out")
    _dev(workspace, "workspace")
    call("ds4hip_flash_attn_decode_mixed_f32_prealloc", _ptr(Q), _ptr(raw_kv), _ptr(comp_kv),
         _ptr(comp_allowed), _ptr(sinks), _ptr(out), n_head, n_raw, n_comp, head_dim,
         _ptr(workspace), workspace.numel(), _stream(stream))


class DecodeOpts(C.Structure):
    """ds4hip_decode_opts: per-call P precision, kernel choice and merge output form."""
    _fields_ = [("exact_p", C.c_int), ("kernel", C.c_int), ("out_form", C.c_int), ("out_pos", C.c_int),
                ("out_il", C.c_int), ("q8_out", C.c_void_p), ("q8_scale", C.c_void_p),
                ("out_pos_dev", C.c_void_p)]


_KERNELS = {"auto": 0, "regload": 1}


def decode_opts(exact_p=False, kernel="auto", rope_q8=None, rope_out=None):
    """rope_q8: None (the merge writes out) or (q8_out int8, q8_scale fp32,
    pos, il): the merge writes the inverse-RoPE'd rows in Q8_0 form instead
    (DS4HIP_DECODE_OUT_ROPE_Q8), the input of attn_out_decode_q8_f32.
    rope_out: (pos_dev int32 [n_prob], il): out holds the rows after the
    inverse tail RoPE at each problem's position (DS4HIP_DECODE_OUT_ROPE_F32)."""
    if kernel not in _KERNELS:
        raise Ds4HipError(f"kernel must be one of {sorted(_KERNELS)}", -22)
    if rope_out is not None:
        pos_dev, il = rope_out
        _check(pos_dev, torch.int32, None, "out_pos_dev")
        return DecodeOpts(int(bool(exact_p)), _KERNELS[kernel], 2, 0, int(il), None, None, _ptr(pos_dev))
    if rope_q8 is None:
        return DecodeOpts(int(bool(exact_p)), _KERNELS[kernel])
    xq, xs, pos, il = rope_q8
    _check(xq, torch.int8, None, "q8_out")
    _check(xs, torch.float32, None, "q8_scale")
    return DecodeOpts(int(bool(exact_p)), _KERNELS[kernel], 1, int(pos), int(il), _ptr(xq), _ptr(xs))


def decode_fp8_workspace_bytes(n_rows_per_prob) -> int:
    arr = (C.c_longlong * len(n_rows_per_prob))(*[int(x) for x in n_rows_per_prob])
    out = C.c_size_t(0)
    call("ds4hip_flash_attn_decode_fp8_workspace_size", C.cast(arr, C.c_void_p),
         len(n_rows_per_prob), C.byref(out))
    return out.value


def q_prep_words() -> int:
    """32-bit words of one problem's converted query (flash_attn_q_prep_f32)."""
    return lib().ds4hip_flash_attn_q_prep_words()


def flash_attn_q_prep_f32(q, out=None, stream=None):
    """q [n_prob, 64, 512] fp32 -> int32 [n_prob, q_prep_words()]: the form
    the FP8 decode's flat-stage kernel builds from an fp32 Q at its start;
    passing it as q to flash_attn_decode_fp8 (or Session.decode) gives the
    fp32-Q results bit for bit without that work."""
    n_prob = q.numel() // (N_HEAD * HEAD_DIM)
    _check(q, torch.float32, n_prob * N_HEAD * HEAD_DIM, "q")
    w = q_prep_words()
    if out is None:
        out = torch.empty((n_prob, w), dtype=torch.int32, device=q.device)
    _check(out, torch.int32, n_prob * w, "out")
    call("ds4hip_flash_attn_q_prep_f32", _ptr(q), N_HEAD * HEAD_DIM, n_prob, _ptr(out), w, _stream(stream))
    return out


def _q_mode(q):
    """(q_is_f32 argument, problem stride) of a decode query tensor."""
    if q.dtype == torch.int32:
        return 2, q_prep_words()
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise Ds4HipError("q must be bf16, fp32 or a converted fp32 query (int32)", -22)
    return int(q.dtype == torch.float32), N_HEAD * HEAD_DIM


def flash_attn_decode_fp8(q, sinks, out, cache: Fp8KVCache, n_rows_per_prob, *, row_base=None,
                          row_base_stride=0, row_idx=None, page_table=None, page_rows=256,
                          workspace=None, phases=3, exact_p=False, kernel="auto", rope_q8=None, rope_out=None,
                          stream=None):
    """Decode attention of n_prob single-query problems over the FP8 cache.

    q [n_prob, 64, 512] bf16 or fp32 (or int32 [n_prob, q_prep_words()], a
    converted fp32 Q from flash_attn_q_prep_f32); sinks [n_prob, 64] fp32; out
    [n_prob, 64, 512] fp32; n_rows_per_prob: host ints. Row r of problem p is
    position row_idx[p, r] (or r), mapped through page_table[p] (pages of
    page_rows rows) or offset by row_base[p] (int64 tensor) / p*row_base_stride.
    exact_p: P as f16 hi + lo instead of one f16; kernel: "auto" or "regload"
    (the register-load kernel for direct rows too); rope_q8, rope_out: see decode_opts.
    """
    n_prob = len(n_rows_per_prob)
    q_mode, q_stride = _q_mode(q)
    _check(q, q.dtype, n_prob * q_stride, "q")
    _check(sinks, torch.float32, n_prob * N_HEAD, "sinks")
    _check(out, torch.float32, n_prob * N_HEAD * HEAD_DIM, "out")
    _check(row_base, torch.int64, n_prob, "row_base")
    _check(row_idx, torch.int32, None, "row_idx")
    _check(page_table, torch.int32, None, "page_table")
    counts = (C.c_longlong * n_prob)(*[int(x) for x in n_rows_per_prob])
    need = decode_fp8_workspace_bytes(n_rows_per_prob)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _dev(workspace, "workspace", need)
    call("ds4hip_flash_attn_decode_fp8", _ptr(q), q_mode, q_stride, _ptr(sinks), N_HEAD, _ptr(out),
         N_HEAD * HEAD_DIM, _ptr(cache.codes), _ptr(cache.sexp), _ptr(cache.tail), C.cast(counts, C.c_void_p),
         n_prob, _ptr(row_base), int(row_base_stride), _ptr(row_idx),
         row_idx.shape[-1] if row_idx is not None else 0, _ptr(page_table),
         page_table.shape[-1] if page_table is not None else 0, int(page_rows), N_HEAD,
         HEAD_DIM, N_ROT, C.c_longlong(cache.n_rows), C.byref(decode_opts(exact_p, kernel, rope_q8, rope_out)),
         _ptr(workspace), workspace.numel(), int(phases), _stream(stream))
    return workspace


def flash_attn_prefill_fp8(q, sinks, out, cache: Fp8KVCache, n_q, n_cached, row0=0,
                           workspace=None, exact_p=False, stream=None):
    """Causal chunked prefill: q [n_q, 64, 512] bf16, out [n_q, 64, 512] fp32;
    the sequence's rows start at cache row row0 and the chunk's own rows
    (n_cached .. n_cached + n_q - 1) are already appended. exact_p: P as f16
    hi + lo in P . V (default: one f16)."""
    _check(q, torch.bfloat16, n_q * N_HEAD * HEAD_DIM, "q")
    _check(sinks, torch.float32, N_HEAD, "sinks")
    _check(out, torch.float32, n_q * N_HEAD * HEAD_DIM, "out")
    if row0 + n_cached + n_q > cache.n_rows:
        raise Ds4HipError("prefill rows past the end of the cache", -22)
    c = cache.codes[row0:]
    s = cache.sexp[row0:]
    t = cache.tail[row0:]
    from ._lib import lib
    need = lib().ds4hip_flash_attn_prefill_fp8_workspace_size(n_q)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    call("ds4hip_flash_attn_prefill_fp8", _ptr(q), _ptr(sinks), _ptr(out), _ptr(c), _ptr(s),
         _ptr(t), n_q, n_cached, N_HEAD, HEAD_DIM, N_ROT, _ptr(workspace), workspace.numel(),
         int(bool(exact_p)), _stream(stream))
    return workspace


# ---- tail RoPE (cuda/rope.cuh:51, cuda/attn_out.cuh:52) ----------------------------------

def launch_tail_rope_yarn_f32(x_in, x_out, n_heads, head_dim, n_rot, pos, il, stream=None):
    _check(x_in, torch.float32, n_heads * head_dim, "x_in")
    _check(x_out, torch.float32, n_heads * head_dim, "x_out")
    call("ds4hip_tail_rope_yarn_f32", _ptr(x_in), _ptr(x_out), n_heads, head_dim, n_rot, pos, il,
         _stream(stream))


def launch_tail_rope_yarn_inverse_f32(x_in, x_out, n_heads, head_dim, n_rot, pos, il,
                                      stream=None):
    _check(x_in, torch.float32, n_heads * head_dim, "x_in")
    _check(x_out, torch.float32, n_heads * head_dim, "x_out")
    call("ds4hip_tail_rope_yarn_inverse_f32", _ptr(x_in), _ptr(x_out), n_heads, head_dim, n_rot,
         pos, il, _stream(stream))


# ---- matvecs (cuda/router.cuh:62, cuda/attn_out.cuh:86,98, cuda/dense_q8.cuh:62) ----------

def launch_mul_mv_f16_f32(w_f16, x_f32, y_f32, out_dim, in_dim, stream=None):
    _check(w_f16, torch.int16, out_dim * in_dim, "w_f16")
    _check(x_f32, torch.float32, in_dim, "x")
    _check(y_f32, torch.float32, out_dim, "y")
    call("ds4hip_mul_mv_f16_f32", _ptr(w_f16), _ptr(x_f32), _ptr(y_f32), out_dim, in_dim,
         _stream(stream))


def mul_mv_f16_scaled_f32(w_f16, x_f32, y_f32, out_dim, in_dim, scale, stream=None):
    """launch_mul_mv_f16_f32 then every output times scale, in one launch."""
    _check(w_f16, torch.int16, out_dim * in_dim, "w_f16")
    _check(x_f32, torch.float32, in_dim, "x")
    _check(y_f32, torch.float32, out_dim, "y")
    call("ds4hip_mul_mv_f16_scaled_f32", _ptr(w_f16), _ptr(x_f32), _ptr(y_f32), out_dim, in_dim,
         C.c_float(scale), _stream(stream))


def mul_mv_f16_rope_f32(w_f16, x_f32, y_f32, n_heads, head_dim, n_rot, pos, il, in_dim, stream=None):
    """launch_mul_mv_f16_f32 into n_heads rows of head_dim, then the forward
    tail RoPE, in one launch."""
    _check(w_f16, torch.int16, n_heads * head_dim * in_dim, "w_f16")
    _check(x_f32, torch.float32, in_dim, "x")
    _check(y_f32, torch.float32, n_heads * head_dim, "y")
    call("ds4hip_mul_mv_f16_rope_f32", _ptr(w_f16), _ptr(x_f32), _ptr(y_f32), n_heads, head_dim, n_rot,
         pos, il, in_dim, _stream(stream))


def attn_out_decode_workspace(n_head, head_dim, n_groups, rank, device):
    from ._lib import lib
    nb = lib().ds4hip_attn_out_decode_workspace_bytes(n_head, head_dim, n_groups, rank)
    return torch.empty(max(nb, 1), dtype=torch.uint8, device=device)


def attn_out_decode_f32(kqv, w_out_a, w_out_b, out, n_head, head_dim, n_rot, pos, il, n_groups, rank,
                        out_dim, workspace=None, stream=None):
    """Steps 14-16: inverse tail RoPE of kqv [n_head, head_dim], the grouped
    Q8_0 projection (n_groups x rank rows) and the dense Q8_0 projection to
    out [out_dim]; the rotation and the first quantization in one launch."""
    from ._lib import lib
    group_dim = n_head * head_dim // n_groups
    _check(kqv, torch.float32, n_head * head_dim, "kqv")
    _check(w_out_a, torch.uint8, n_groups * rank * (group_dim // 32) * 34, "w_out_a")
    _check(w_out_b, torch.uint8, out_dim * (n_groups * rank // 32) * 34, "w_out_b")
    _check(out, torch.float32, out_dim, "out")
    need = lib().ds4hip_attn_out_decode_workspace_bytes(n_head, head_dim, n_groups, rank)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=kqv.device)
    _dev(workspace, "workspace", need)
    call("ds4hip_attn_out_decode_f32", _ptr(kqv), _ptr(w_out_a), _ptr(w_out_b), _ptr(out), n_head, head_dim,
         n_rot, pos, il, n_groups, rank, out_dim, _ptr(workspace), workspace.numel(), _stream(stream))
    return workspace


def attn_out_decode_q8_f32(xq, xscale, w_out_a, w_out_b, out, n_head, head_dim, n_groups, rank, out_dim,
                           workspace=None, stream=None):
    """attn_out_decode_f32 after its first step: from the rotated Q8_0
    attention output (xq int8 [n_head*head_dim], xscale fp32 [/32]) that a
    decode merge writes with decode_opts(rope_q8=...)."""
    group_dim = n_head * head_dim // n_groups
    _check(xq, torch.int8, n_head * head_dim, "xq")
    _check(xscale, torch.float32, n_head * head_dim // 32, "xscale")
    _check(w_out_a, torch.uint8, n_groups * rank * (group_dim // 32) * 34, "w_out_a")
    _check(w_out_b, torch.uint8, out_dim * (n_groups * rank // 32) * 34, "w_out_b")
    _check(out, torch.float32, out_dim, "out")
    need = lib().ds4hip_attn_out_decode_workspace_bytes(n_head, head_dim, n_groups, rank)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=xq.device)
    _dev(workspace, "workspace", need)
    call("ds4hip_attn_out_decode_q8_f32", _ptr(xq), _ptr(xscale), _ptr(w_out_a), _ptr(w_out_b), _ptr(out), n_head,
         head_dim, n_groups, rank, out_dim, _ptr(workspace), workspace.numel(), _stream(stream))
    return workspace


def launch_mul_mv_q8_0_q8_0_grouped_f32(W, x, y, n_groups, group_dim, rank, stream=None):
    _check(W, torch.uint8, n_groups * rank * (group_dim // 32) * 34, "W")
    _check(x, torch.float32, n_groups * group_dim, "x")
    _check(y, torch.float32, n_groups * rank, "y")
    call("ds4hip_mul_mv_q8_0_q8_0_grouped_f32", _ptr(W), _ptr(x), _ptr(y), n_groups, group_dim,
         rank, _stream(stream))


def launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(W, x, y, n_groups, group_dim, rank, scratch_xq,
                                                 scratch_xscale, stream=None):
    _check(W, torch.uint8, n_groups * rank * (group_dim // 32) * 34, "W")
    _check(x, torch.float32, n_groups * group_dim, "x")
    _check(y, torch.float32, n_groups * rank, "y")
    _check(scratch_xq, torch.int8, n_groups * group_dim, "scratch_xq")
    _check(scratch_xscale, torch.float32, n_groups * group_dim // 32, "scratch_xscale")
    call("ds4hip_mul_mv_q8_0_q8_0_grouped_f32_prealloc", _ptr(W), _ptr(x), _ptr(y), n_groups,
         group_dim, rank, _ptr(scratch_xq), _ptr(scratch_xscale), _stream(stream))


def launch_mul_mv_q8_0_q8_0_f32_prealloc(W, x, y, n_rows, n_cols, scratch_xq, scratch_xscale,
                                         stream=None):
    _check(W, torch.uint8, n_rows * (n_cols // 32) * 34, "W")
    _check(x, torch.float32, n_cols, "x")
    _check(y, torch.float32, n_rows, "y")
    _check(scratch_xq, torch.int8, n_cols, "scratch_xq")
    _check(scratch_xscale, torch.float32, n_cols // 32, "scratch_xscale")
    call("ds4hip_mul_mv_q8_0_q8_0_f32_prealloc", _ptr(W), _ptr(x), _ptr(y), n_rows, n_cols,
         _ptr(scratch_xq), _ptr(scratch_xscale), _stream(stream))


def mul_mm_workspace(n_rows, n_cols, n_batch, device):
    """Workspace tensor for mul_mm_bf16_f32 / mul_mm_f32_f32 of this shape."""
    from ._lib import lib
    nb = lib().ds4hip_mul_mm_workspace_bytes(n_rows, n_cols, n_batch)
    return torch.empty(max(nb, 1), dtype=torch.uint8, device=device)


def mul_mm_bf16_f32(W, X, Y, n_rows, n_cols, n_batch, workspace=None, stream=None):
    """Y [n_batch, n_rows] = X W^T, bf16 W; deterministic (fixed-order split-K)."""
    _check(W, torch.bfloat16, n_rows * n_cols, "W")
    _check(X, torch.float32, n_batch * n_cols, "X")
    _check(Y, torch.float32, n_batch * n_rows, "Y")
    if workspace is None:
        workspace = mul_mm_workspace(n_rows, n_cols, n_batch, X.device)
    call("ds4hip_mul_mm_bf16_f32", _ptr(W), _ptr(X), _ptr(Y), n_rows, n_cols, n_batch,
         _ptr(workspace), workspace.numel(), _stream(stream))
    return workspace


# ---- indexer (cuda/indexer_allowed.cuh:33,67,83,97) ----------------------------------------

def launch_indexer_allowed_short_circuit_i32(out_i32, n_comp, top_k, stream=None):
    _check(out_i32, torch.int32, max(n_comp, 0), "out_i32")
    call("ds4hip_indexer_allowed_short_circuit_i32", _ptr(out_i32), n_comp, top_k,
         _stream(stream))


def launch_scale_inplace_f32(y, n, scale, stream=None):
    _check(y, torch.float32, n, "y")
    call("ds4hip_scale_inplace_f32", _ptr(y), n, float(scale), _stream(stream))


def launch_indexer_score_topk_i32(q, weights, index_comp, n_comp, n_head, head_dim, top_k,
                                  allowed_out, scratch_scores, stream=None):
    _check(index_comp, torch.int16, n_comp * head_dim, "index_comp")
    _check(q, torch.float32, n_head * head_dim, "q")
    _check(weights, torch.float32, n_head, "weights")
    _check(allowed_out, torch.int32, n_comp, "allowed_out")
    _check(scratch_scores, torch.float32, n_comp, "scratch_scores")
    call("ds4hip_indexer_score_topk_i32", _ptr(q), _ptr(weights), _ptr(index_comp), n_comp,
         n_head, head_dim, top_k, _ptr(allowed_out), _ptr(scratch_scores), _stream(stream))


def launch_indexer_score_topk_f32_i32(q, weights, index_comp_f32, n_comp, n_head, head_dim,
                                      top_k, allowed_out, scratch_scores, stream=None):
    _check(index_comp_f32, torch.float32, n_comp * head_dim, "index_comp_f32")
    _check(q, torch.float32, n_head * head_dim, "q")
    _check(weights, torch.float32, n_head, "weights")
    _check(allowed_out, torch.int32, n_comp, "allowed_out")
    _check(scratch_scores, torch.float32, n_comp, "scratch_scores")
    call("ds4hip_indexer_score_topk_f32_i32", _ptr(q), _ptr(weights), _ptr(index_comp_f32),
         n_comp, n_head, head_dim, top_k, _ptr(allowed_out), _ptr(scratch_scores),
         _stream(stream))


_KEY_KIND = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def indexer_topk_positions(q, weights, keys, top_k, n_recent, *, scores=None, select=None,
                           mask=None, positions=None, stream=None):
    """keys [n_comp, head_dim] fp32/f16/bf16; returns (positions, mask, scores)."""
    n_comp, head_dim = keys.shape
    n_head = q.numel() // head_dim
    dev = keys.device
    if scores is None:
        scores = torch.empty(n_comp, dtype=torch.float32, device=dev)
    if select is None:
        from ._lib import lib
        nb = lib().ds4hip_indexer_select_scratch_bytes(n_comp)
        select = torch.empty(nb, dtype=torch.uint8, device=dev)
    if positions is None:
        positions = torch.empty(min(top_k, n_comp), dtype=torch.int32, device=dev)
    _check(q, torch.float32, n_head * head_dim, "q")
    _check(weights, torch.float32, n_head, "weights")
    _check(scores, torch.float32, n_comp, "scores")
    _check(mask, torch.int32, n_comp, "mask")
    _check(positions, torch.int32, min(top_k, n_comp), "positions")
    _dev(keys, "keys")
    _dev(select, "select")
    call("ds4hip_indexer_topk_positions", _ptr(q), _ptr(weights), _ptr(keys),
         _KEY_KIND[keys.dtype], n_comp, n_head, head_dim, top_k, n_recent, _ptr(scores),
         _ptr(select), _ptr(mask), _ptr(positions), _stream(stream))
    return positions, mask, scores


# ---- compressor (cuda/compressor.cuh:78,102) -------------------------------------------------

def launch_compressor_decode_step_f32_prealloc(is_attn, x_f32, w_kv_f16, w_gate_f16, w_ape_f16,
                                               w_norm_f32, in_dim, head_dim_out, compress_ratio,
                                               pos, il, state_kv, state_score, emit_out,
                                               scratch_kv_cur, scratch_sc_cur, stream=None):
    """Returns `emitted` (the reference's *emitted_out_host)."""
    coff = 2 if compress_ratio == 4 else 1
    for t, nm in ((x_f32, "x"), (w_kv_f16, "w_kv"), (w_gate_f16, "w_gate"), (w_ape_f16, "w_ape"),
                  (w_norm_f32, "w_norm"), (state_kv, "state_kv"), (state_score, "state_score"),
                  (emit_out, "emit_out")):
        _dev(t, nm)
    _check(scratch_kv_cur, torch.float32, coff * head_dim_out, "scratch_kv_cur")
    _check(scratch_sc_cur, torch.float32, coff * head_dim_out, "scratch_sc_cur")
    _dev(scratch_kv_cur, "scratch_kv_cur")
    _dev(scratch_sc_cur, "scratch_sc_cur")
    emitted = C.c_int(0)
    call("ds4hip_compressor_decode_step_f32_prealloc", int(bool(is_attn)), _ptr(x_f32),
         _ptr(w_kv_f16), _ptr(w_gate_f16), _ptr(w_ape_f16), _ptr(w_norm_f32), in_dim,
         head_dim_out, compress_ratio, pos, il, _ptr(state_kv), _ptr(state_score), _ptr(emit_out),
         C.byref(emitted), _ptr(scratch_kv_cur), _ptr(scratch_sc_cur), _stream(stream))
    return emitted.value


def launch_compressor_decode_step_f32(is_attn, x_f32, w_kv_f16, w_gate_f16, w_ape_f16,
                                      w_norm_f32, in_dim, head_dim_out, compress_ratio, pos, il,
                                      state_kv, state_score, emit_out, stream=None):
    for t, nm in ((x_f32, "x"), (w_kv_f16, "w_kv"), (w_gate_f16, "w_gate"), (w_ape_f16, "w_ape"),
                  (w_norm_f32, "w_norm"), (state_kv, "state_kv"), (state_score, "state_score"),
                  (emit_out, "emit_out")):
        _dev(t, nm)
    emitted = C.c_int(0)
    call("ds4hip_compressor_decode_step_f32", int(bool(is_attn)), _ptr(x_f32), _ptr(w_kv_f16),
         _ptr(w_gate_f16), _ptr(w_ape_f16), _ptr(w_norm_f32), in_dim, head_dim_out,
         compress_ratio, pos, il, _ptr(state_kv), _ptr(state_score), _ptr(emit_out),
         C.byref(emitted), _stream(stream))
    return emitted.value


def compressor_decode_step_w32(is_attn, x_f32, w_kv_f32, w_gate_f32, w_ape_f16, w_norm_f32,
                               in_dim, head_dim_out, compress_ratio, pos, il, state_kv,
                               state_score, emit_out, stream=None):
    emitted = C.c_int(0)
    call("ds4hip_compressor_decode_step_w32", int(bool(is_attn)), _ptr(x_f32), _ptr(w_kv_f32),
         _ptr(w_gate_f32), _ptr(w_ape_f16), _ptr(w_norm_f32), in_dim, head_dim_out,
         compress_ratio, pos, il, _ptr(state_kv), _ptr(state_score), _ptr(emit_out),
         C.byref(emitted), _stream(stream))
    return emitted.value


# ---- batched forms (the batched-decode attention block) ------------------------------------

def mul_mm_f32_f32(W, X, Y, n_rows, n_cols, n_batch, workspace=None, stream=None):
    _check(W, torch.float32, n_rows * n_cols, "W")
    _check(X, torch.float32, n_batch * n_cols, "X")
    _check(Y, torch.float32, n_batch * n_rows, "Y")
    if workspace is None:
        workspace = mul_mm_workspace(n_rows, n_cols, n_batch, X.device)
    call("ds4hip_mul_mm_f32_f32", _ptr(W), _ptr(X), _ptr(Y), n_rows, n_cols, n_batch,
         _ptr(workspace), workspace.numel(), _stream(stream))
    return workspace


def tail_rope_yarn_batch_f32(x_in, x_out, n_seq, n_heads, head_dim, n_rot, pos_dev, il,
                             inverse=False, stream=None):
    _check(x_in, torch.float32, n_seq * n_heads * head_dim, "x_in")
    _check(x_out, torch.float32, n_seq * n_heads * head_dim, "x_out")
    _check(pos_dev, torch.int32, n_seq, "pos")
    call("ds4hip_tail_rope_yarn_batch_f32", _ptr(x_in), _ptr(x_out), n_seq, n_heads, head_dim,
         n_rot, _ptr(pos_dev), il, int(inverse), _stream(stream))


def indexer_topk_positions_batch(q, weights, keys, key_row0, n_comp, top_k, n_recent, scores,
                                 positions, pos_offset=0, stream=None):
    """q [n_seq, n_head, 128] fp32, weights [n_seq, n_head], keys [rows, 128]
    (fp32 / f16 / bf16), key_row0 / n_comp host ints per sequence, scores
    [rows] fp32 scratch, positions [n_seq, stride] int32; sequence s writes at
    positions[s, pos_offset:]."""
    n_seq = len(n_comp)
    n_head = q.shape[1]
    r0 = (C.c_longlong * n_seq)(*[int(x) for x in key_row0])
    nc = (C.c_int * n_seq)(*[int(x) for x in n_comp])
    _check(positions, torch.int32, n_seq * positions.shape[-1], "positions")
    stride = positions.shape[-1]
    if pos_offset + top_k > stride:
        raise Ds4HipError("positions rows too short", -22)
    call("ds4hip_indexer_topk_positions_batch", _ptr(q), _ptr(weights), _ptr(keys),
         _KEY_KIND[keys.dtype], C.cast(r0, C.c_void_p), C.cast(nc, C.c_void_p), n_seq, n_head,
         keys.shape[-1], top_k, n_recent, _ptr(scores),
         C.c_void_p(positions.data_ptr() + 4 * pos_offset), stride, _stream(stream))


def compressor_batch_scratch(n_seq, in_dim, head_dim_out, ratio, device):
    """Scratch tensor (uint8) for compressor_decode_step_batch_w32."""
    from ._lib import lib
    nb = lib().ds4hip_compressor_batch_scratch_bytes(n_seq, in_dim, head_dim_out, ratio)
    return torch.empty(nb, dtype=torch.uint8, device=device)


def compressor_decode_step_batch_w32(is_attn, x, w_kv, w_gate, w_ape, w_norm, in_dim,
                                     head_dim_out, ratio, pos, pos_dev, il, state_kv,
                                     state_score, state_stride, emit_out, scratch, stream=None):
    """One compressor step for len(pos) sequences; returns the host emit flags.
    scratch: a tensor of compressor_batch_scratch(...) bytes."""
    n = len(pos)
    ph = (C.c_int * n)(*[int(p) for p in pos])
    em = (C.c_int * n)()
    _check(pos_dev, torch.int32, n, "pos_dev")
    call("ds4hip_compressor_decode_step_batch_w32", int(is_attn), n, _ptr(x), _ptr(w_kv),
         _ptr(w_gate), _ptr(w_ape), _ptr(w_norm), in_dim, head_dim_out, ratio,
         C.cast(ph, C.c_void_p), _ptr(pos_dev), il, _ptr(state_kv), _ptr(state_score),
         int(state_stride), _ptr(emit_out), C.cast(em, C.c_void_p), _ptr(scratch),
         scratch.numel() * scratch.element_size(), _stream(stream))
    return list(em)


class RowsPush(C.Structure):
    """ds4hip_rows_push: two FP8 appends and one fp32 row scatter in one launch."""
    _fields_ = [("fp8_src", C.c_void_p * 2), ("fp8_n", C.c_int * 2), ("fp8_dst", C.c_void_p * 2),
                ("f32_src", C.c_void_p), ("f32_n", C.c_int), ("f32_width", C.c_int), ("f32_dst", C.c_void_p),
                ("f32_dst_rows", C.c_void_p)]


def batch_rows_push_f32(cache, fp8_sets, f32_src, f32_dst, f32_dst_rows, stream=None):
    """fp8_sets: two (rows [n, 512] fp32, dst_rows int64 [n]) appended to the
    FP8 cache; f32_src [m, w] rows copied to f32_dst rows f32_dst_rows (int64 [m])."""
    p = RowsPush()
    for k, (rows, dst) in enumerate(fp8_sets):
        n = rows.shape[0]
        _check(rows, torch.float32, n * HEAD_DIM, "fp8 rows")
        _check(dst, torch.int64, n, "fp8 dst_rows")
        p.fp8_src[k], p.fp8_n[k], p.fp8_dst[k] = _ptr(rows), n, _ptr(dst)
    m, w = f32_src.shape
    _check(f32_src, torch.float32, m * w, "f32_src")
    _check(f32_dst, torch.float32, None, "f32_dst")
    _check(f32_dst_rows, torch.int64, m, "f32_dst_rows")
    p.f32_src, p.f32_n, p.f32_width, p.f32_dst, p.f32_dst_rows = _ptr(f32_src), m, w, _ptr(f32_dst), _ptr(f32_dst_rows)
    call("ds4hip_batch_rows_push_f32", C.byref(p), _ptr(cache.codes), _ptr(cache.sexp), _ptr(cache.tail), HEAD_DIM,
         N_ROT, _stream(stream))


class CompressorBatchJob(C.Structure):
    """ds4hip_compressor_batch_job: one compressor of compressor_pair_step_batch_w32."""
    _fields_ = [("w_kv_f32", C.c_void_p), ("w_gate_f32", C.c_void_p), ("w_ape_f16", C.c_void_p),
                ("w_norm_f32", C.c_void_p), ("head_dim_out", C.c_int), ("state_kv", C.c_void_p),
                ("state_score", C.c_void_p), ("state_stride", C.c_longlong), ("emit_out", C.c_void_p)]


def compressor_pair_scratch(n_seq, in_dim, attn_head_dim_out, index_head_dim_out, ratio, device):
    """Scratch tensor (uint8) for compressor_pair_step_batch_w32."""
    nb = lib().ds4hip_compressor_pair_batch_scratch_bytes(n_seq, in_dim, attn_head_dim_out, index_head_dim_out,
                                                          ratio)
    return torch.empty(nb, dtype=torch.uint8, device=device)


def compressor_pair_step_batch_w32(x, in_dim, ratio, pos, pos_dev, il, attn, index, scratch, stream=None):
    """A layer's attention and indexer compressors for len(pos) sequences in
    three launches; attn / index: dicts of w_kv, w_gate, w_ape, w_norm,
    head_dim_out, state_kv, state_score, state_stride, emit_out (the
    arguments of compressor_decode_step_batch_w32). Returns the host emit flags."""
    n = len(pos)
    ph = (C.c_int * n)(*[int(p) for p in pos])
    em = (C.c_int * n)()
    _check(pos_dev, torch.int32, n, "pos_dev")
    _check(x, torch.float32, n * in_dim, "x")
    jobs = []
    for j in (attn, index):
        for k in ("w_kv", "w_gate", "w_norm", "state_kv", "state_score", "emit_out"):
            _check(j[k], torch.float32, None, k)
        _check(j["w_ape"], j["w_ape"].dtype, None, "w_ape")
        jobs.append(CompressorBatchJob(_ptr(j["w_kv"]), _ptr(j["w_gate"]), _ptr(j["w_ape"]), _ptr(j["w_norm"]),
                                       int(j["head_dim_out"]), _ptr(j["state_kv"]), _ptr(j["state_score"]),
                                       int(j["state_stride"]), _ptr(j["emit_out"])))
    _check(scratch, torch.uint8, None, "scratch")
    call("ds4hip_compressor_pair_step_batch_w32", n, _ptr(x), in_dim, ratio, C.cast(ph, C.c_void_p), _ptr(pos_dev),
         il, C.byref(jobs[0]), C.byref(jobs[1]), C.cast(em, C.c_void_p), _ptr(scratch), scratch.numel(),
         _stream(stream))
    return list(em)


def launch_rms_norm_f32(x, w, y, n, eps=1e-6, stream=None):
    _check(x, torch.float32, n, "x")
    _check(w, torch.float32, n, "w")
    _check(y, torch.float32, n, "y")
    call("ds4hip_rms_norm_f32", _ptr(x), _ptr(w), _ptr(y), n, eps, _stream(stream))


def launch_rms_norm_batch_f32(x, w, weight_dim, y, n_rows, n_per_row, eps=1e-6, stream=None):
    _check(x, torch.float32, n_rows * n_per_row, "x")
    _check(y, torch.float32, n_rows * n_per_row, "y")
    if weight_dim:
        _check(w, torch.float32, weight_dim, "w")
    call("ds4hip_rms_norm_batch_f32", _ptr(x), _ptr(w) if weight_dim else None, weight_dim,
         _ptr(y), n_rows, n_per_row, eps, _stream(stream))


def attn_qkv_decode_f32(attn_norm, w_q_a, w_q_a_norm, w_kv_a, w_kv_a_norm, w_q_b, pos, il,
                        q_lora_norm, q_cur, kv_rope, workspace=None, stream=None):
    """Steps 3-10 of one decode layer (Q8_0 weights as uint8 block rows):
    fills q_lora_norm [1024], q_cur [64*512] and kv_rope [512]; returns the
    workspace (reusable)."""
    _check(attn_norm, torch.float32, 4096, "attn_norm")
    _check(w_q_a, torch.uint8, 1024 * 128 * 34, "w_q_a")
    _check(w_kv_a, torch.uint8, 512 * 128 * 34, "w_kv_a")
    _check(w_q_b, torch.uint8, 32768 * 32 * 34, "w_q_b")
    _check(w_q_a_norm, torch.float32, 1024, "w_q_a_norm")
    _check(w_kv_a_norm, torch.float32, 512, "w_kv_a_norm")
    _check(q_lora_norm, torch.float32, 1024, "q_lora_norm")
    _check(q_cur, torch.float32, 64 * 512, "q_cur")
    _check(kv_rope, torch.float32, 512, "kv_rope")
    from ._lib import lib
    need = lib().ds4hip_attn_qkv_decode_workspace_bytes()
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=attn_norm.device)
    call("ds4hip_attn_qkv_decode_f32", _ptr(attn_norm), _ptr(w_q_a), _ptr(w_q_a_norm),
         _ptr(w_kv_a), _ptr(w_kv_a_norm), _ptr(w_q_b), pos, il, _ptr(q_lora_norm), _ptr(q_cur),
         _ptr(kv_rope), _ptr(workspace), workspace.numel(), _stream(stream))
    return workspace
