"""The C-ABI library loads and exports every symbol include/*.h declares;
argument validation runs on the host (no GPU needed)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:int|size_t|void)\s+(ds4hip_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "ds4hip_flash_attn_decode_fp8" in syms
    assert "ds4hip_fp8_kv_quantize_round_trip_f32" in syms


def test_library_exports_every_declared_symbol():
    from ds4cuda_amd import lib
    from ds4cuda_amd._lib import SIGNATURES
    l = lib()
    for name in declared_symbols():
        assert hasattr(l, name), name
        assert name in SIGNATURES, f"{name} missing from the ctypes signature table"


def test_shape_validation_returns_einval():
    from ds4cuda_amd import lib
    l = lib()
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 1, 500, 64, None) == -22
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 1, 512, 60, None) == -22
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 0, 512, 64, None) == 0
    assert l.ds4hip_flash_attn_decode_raw_f32(None, None, None, None, None, 32, 4, 512, None) == -22
    assert l.ds4hip_flash_attn_decode_raw_f32(None, None, None, None, None, 64, 4, 256, None) == -22
    assert l.ds4hip_flash_attn_decode_mixed_f32(None, None, None, None, None, None, 64, -1, 0, 512,
                                                None) == -22
    assert l.ds4hip_get_last_error() == -22


def test_workspace_size_is_positive():
    from ds4cuda_amd.ops import decode_fp8_workspace_bytes
    assert decode_fp8_workspace_bytes([32768] * 43) > 0
    assert decode_fp8_workspace_bytes([0, 5, 0]) > 0


def test_newer_entry_points_refuse_bad_arguments_on_the_host():
    """Null pointers, unsupported shapes and out-of-range switches are refused
    with -22 before any device work (the persistence calls return -1, as the
    reference's do, and keep -22 for ds4hip_get_last_error)."""
    from ds4cuda_amd import lib
    l = lib()
    N = None
    assert l.ds4hip_attn_qkv_decode_f32(N, N, N, N, N, N, 0, 0, N, N, N, N, C.c_size_t(0), N) == -22
    assert l.ds4hip_rms_norm_f32(N, N, N, 16, C.c_float(1e-6), N) == -22
    assert l.ds4hip_rms_norm_batch_f32(N, N, 0, N, 4, 16, C.c_float(1e-6), N) == -22
    assert l.ds4hip_session_save_to_disk(N, N, 0, b"/nonexistent/kv") == -1
    assert l.ds4hip_get_last_error() == -22
    assert l.ds4hip_session_load_from_disk(N, b"/nonexistent/kv", N, N) == -1
    assert l.ds4hip_get_last_error() == -22
    assert l.ds4hip_session_chunk_rows(N, 0, 0, 1, N, N, N, 0, N, 0, N, N) == -22
    assert l.ds4hip_session_push_raw(N, 0, N, N) == -22
    assert l.ds4hip_session_state_describe(N, 16) == -22
    cnt = (C.c_longlong * 1)(10)
    # 32 heads: the decode serves 64
    assert l.ds4hip_flash_attn_decode_fp8(N, 0, C.c_longlong(0), N, C.c_longlong(0), N, C.c_longlong(0), N, N,
                                          N, cnt, 1, N, C.c_longlong(0), N, C.c_longlong(0), N, 0, 256, 32,
                                          512, 64, C.c_longlong(100), N, N, C.c_size_t(0), 3, N) == -22
    # the host-visible checks that come before any launch: stand-in pointers
    # (never dereferenced) and a workspace size large enough
    from ds4cuda_amd.ops import DecodeOpts
    X = C.c_void_p(16)
    ws_sz = C.c_size_t(1 << 30)

    def dec(counts, n_cache_rows, opts=None, stride=0, row_idx=N, q=X):
        c = (C.c_longlong * len(counts))(*counts)
        return l.ds4hip_flash_attn_decode_fp8(q, 0, C.c_longlong(0), X, C.c_longlong(0), X, C.c_longlong(0), X,
                                              X, X, c, len(counts), N, C.c_longlong(stride), row_idx,
                                              C.c_longlong(0), N, 0, 256, 64, 512, 64, C.c_longlong(n_cache_rows),
                                              None if opts is None else C.byref(opts), X, ws_sz, 3, N)
    assert dec([10], 0) == -22                         # no cache size
    assert dec([10], 9) == -22                         # direct rows past the cache
    assert dec([10, 10], 19, stride=10) == -22         # problem 1's rows past the cache
    assert dec([10], 100, DecodeOpts(2, 0)) == -22     # unknown P mode
    assert dec([10], 100, DecodeOpts(0, 7)) == -22     # unknown kernel
    assert dec([10], 100, row_idx=X, q=N) == -22       # (control: a null q is refused too)
    assert dec([10], 100, DecodeOpts(0, 0, 3)) == -22  # unknown merge output form
    assert dec([10], 100, DecodeOpts(0, 0, 1)) == -22  # Q8_0 output form without its buffers
    assert dec([10], 100, DecodeOpts(0, 0, 2, -1)) == -22   # rotated output at a negative position
    c1 = (C.c_longlong * 1)(10)
    # a converted Q (q_is_f32 = 2) is read by the flat kernel only
    assert l.ds4hip_flash_attn_decode_fp8(X, 2, C.c_longlong(0), X, C.c_longlong(0), X, C.c_longlong(0), X, X, X,
                                          c1, 1, N, C.c_longlong(0), N, C.c_longlong(0), N, 0, 256, 64, 512, 64,
                                          C.c_longlong(100), C.byref(DecodeOpts(0, 1)), X, ws_sz, 3, N) == -22
    # the fused entry points' argument checks
    assert l.ds4hip_flash_attn_q_prep_f32(N, C.c_longlong(0), 1, N, C.c_longlong(0), N) == -22
    assert l.ds4hip_token_prologue_f32(N, N) == -22
    assert l.ds4hip_compressor_emit_f32(1, X, 512, 4, 2, 0, X, X, X, N) == -22   # (pos + 1) % 4 != 0
    assert l.ds4hip_attn_out_decode_q8_f32(N, N, N, N, N, 64, 512, 8, 1024, 4096, N, C.c_size_t(0), N) == -22
    assert l.ds4hip_compressor_pair_step_batch_w32(1, N, 4096, 4, N, N, 0, N, N, N, N, C.c_size_t(0), N) == -22
    assert l.ds4hip_compressor_pair_batch_scratch_bytes(16, 4096, 512, 128, 3) == 0   # ratio 3
    assert l.ds4hip_batch_rows_push_f32(N, N, N, N, 512, 64, N) == -22
    assert l.ds4hip_session_claim_raw_row(N, 0, N) == -22
    assert l.ds4hip_flash_attn_prefill_fp8(N, N, N, N, N, N, 4, 8, 64, 512, 64, N, C.c_size_t(0), 0, N) == -22
    assert l.ds4hip_flash_attn_prefill_fp8(N, N, N, N, N, N, 0, 8, 64, 512, 64, N, C.c_size_t(0), 2, N) == -22
    assert l.ds4hip_flash_attn_decode_mixed_f32_noalloc(N, N, N, N, N, N, 64, -1, 0, 512, N) == -22
    assert l.ds4hip_mul_mm_f32_f32(N, N, N, 16, 32, 1, N, C.c_size_t(0), N) == -22


def test_bench_and_entry_points_compile():
    """bench.py and __graft_entry__.py parse (the GPU box runs them unbuilt)."""
    import py_compile
    for f in ("bench.py", "__graft_entry__.py"):
        py_compile.compile(str(ROOT / f), doraise=True)
