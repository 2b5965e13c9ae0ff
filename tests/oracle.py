"""ctypes wrapper of the CPU oracle (oracle/libds4oracle.so) for the tests.

Test infrastructure only: the oracle is the checker, never the thing tested.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "libds4oracle.so"

_o = None


def lib():
    global _o
    if _o is None:
        if not ORACLE_SO.exists():
            import subprocess
            subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True,
                           capture_output=True)
        _o = C.CDLL(str(ORACLE_SO))
        _o.orc_e4m3fn_value.restype = C.c_float
        _o.orc_e4m3fn_value.argtypes = [C.c_int]
        _o.orc_e4m3fn_nearest_index.restype = C.c_int
        _o.orc_e4m3fn_nearest_index.argtypes = [C.c_float]
        _o.orc_fp8_scale_exp.restype = C.c_int
        _o.orc_fp8_scale_exp.argtypes = [C.c_float]
        _o.orc_f32_to_f16.restype = C.c_uint16
        _o.orc_f32_to_f16.argtypes = [C.c_float]
        _o.orc_f16_to_f32.restype = C.c_float
        _o.orc_f16_to_f32.argtypes = [C.c_uint16]
        _o.orc_fp8_deq.restype = C.c_float
        _o.orc_fp8_deq.argtypes = [C.c_uint8, C.c_int]
        _o.orc_topk_positions.restype = C.c_int
        _o.orc_compressor_step.restype = C.c_int
        _o.orc_compressor_step_w32.restype = C.c_int
    return _o


def P(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def fp8_quant_rows(x: np.ndarray, n_rot: int = 64):
    """-> codes [n, n_nope] u8, sexp [n, 8] i8, tail [n, n_rot] u16, deq [n, d] f32"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    codes = np.zeros((n, d - n_rot), np.uint8)
    sexp = np.zeros((n, 8), np.int8)
    tail = np.zeros((n, n_rot), np.uint16)
    deq = np.zeros((n, d), np.float32)
    lib().orc_fp8_quant_rows(P(x), C.c_int(n), C.c_int(d), C.c_int(n_rot), P(codes), P(sexp),
                             P(tail), P(deq))
    return codes, sexp, tail, deq


def attn_decode_mixed_f32(Q, raw, comp, allowed, sinks):
    Q = np.ascontiguousarray(Q, np.float32)
    n_head, d = Q.shape
    out = np.zeros((n_head, d), np.float32)
    n_raw = 0 if raw is None else raw.shape[0]
    n_comp = 0 if comp is None else comp.shape[0]
    f = lambda a, t: None if a is None else np.ascontiguousarray(a, t)
    raw, comp, allowed = f(raw, np.float32), f(comp, np.float32), f(allowed, np.int32)
    sinks = np.ascontiguousarray(sinks, np.float32)
    lib().orc_attn_decode_mixed_f32(P(Q), P(raw), C.c_int(n_raw), P(comp), C.c_int(n_comp),
                                    P(allowed), P(sinks), P(out), C.c_int(n_head), C.c_int(d))
    return out


def attn_decode_kv_f32(Q, K, V, sinks):
    """Separate K and V rows (the raw launcher with V != K)."""
    Q = np.ascontiguousarray(Q, np.float32)
    n_head, d = Q.shape
    out = np.zeros((n_head, d), np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    lib().orc_attn_decode_kv_f32(P(Q), P(K), P(V), C.c_int(K.shape[0]),
                                 P(np.ascontiguousarray(sinks, np.float32)), P(out),
                                 C.c_int(n_head), C.c_int(d))
    return out


def attn_decode_fp8(Q, codes, sexp, tail, rows, sinks, n_threads=1):
    Q = np.ascontiguousarray(Q, np.float32)
    n_head, d = Q.shape
    rows = np.ascontiguousarray(rows, np.int64)
    out = np.zeros((n_head, d), np.float32)
    lib().orc_attn_decode_fp8(P(Q), P(np.ascontiguousarray(codes)), P(np.ascontiguousarray(sexp)),
                              P(np.ascontiguousarray(tail)), P(rows), C.c_int(len(rows)),
                              P(np.ascontiguousarray(sinks, np.float32)), P(out),
                              C.c_int(n_head), C.c_int(d), C.c_int(tail.shape[-1]),
                              C.c_int(n_threads))
    return out
