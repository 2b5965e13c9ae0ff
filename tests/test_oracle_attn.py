"""Pins the oracle's decode attention (oracle/attn.cpp) with textbook
softmax attention in fp64, the sink-as-extra-key identity, masking
equivalences and special cases."""
import numpy as np
import pytest

import oracle as O


def sdpa64(Q, K, sinks=None):
    """fp64 softmax attention, one query per head, K == V."""
    Q = Q.astype(np.float64)
    K = K.astype(np.float64)
    s = Q @ K.T / np.sqrt(Q.shape[1])
    if sinks is not None:
        s = np.concatenate([s, sinks.astype(np.float64)[:, None]], axis=1)
        K = np.concatenate([K, np.zeros((1, K.shape[1]))], axis=0)   # sink = key with value 0
    s = s - s.max(axis=1, keepdims=True)
    w = np.exp(s)
    return (w / w.sum(axis=1, keepdims=True)) @ K


def f16r(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.fixture
def data():
    rng = np.random.default_rng(10)
    Q = rng.standard_normal((64, 512)).astype(np.float32)
    K = (rng.standard_normal((96, 512)) * 1.3).astype(np.float32)
    sinks = rng.standard_normal(64).astype(np.float32)
    return Q, K, sinks


def test_no_sink_is_textbook_attention(data):
    Q, K, _ = data
    out = O.attn_decode_mixed_f32(Q, K, None, None, np.full(64, -np.inf, np.float32))
    ref = sdpa64(Q, f16r(K))
    assert np.abs(out - ref).max() < 1e-5 * max(1.0, np.abs(ref).max())


def test_sink_is_extra_key_with_zero_value(data):
    Q, K, sinks = data
    out = O.attn_decode_mixed_f32(Q, K, None, None, sinks)
    ref = sdpa64(Q, f16r(K), sinks)
    assert np.abs(out - ref).max() < 1e-5


def test_f16_rounding_on_read(data):
    Q, K, sinks = data
    K2 = K + np.float32(1e-4)                    # not f16 representable
    a = O.attn_decode_mixed_f32(Q, K2, None, None, sinks)
    b = O.attn_decode_mixed_f32(Q, f16r(K2), None, None, sinks)
    assert np.array_equal(a, b)


def test_mixed_all_allowed_equals_concat(data):
    Q, K, sinks = data
    a = O.attn_decode_mixed_f32(Q, K[:40], K[40:], np.ones(56, np.int32), sinks)
    b = O.attn_decode_mixed_f32(Q, K, None, None, sinks)
    c = O.attn_decode_mixed_f32(Q, K[:40], K[40:], None, sinks)
    assert np.abs(a - b).max() < 1e-6 and np.array_equal(a, c)


def test_masked_rows_have_no_effect(data):
    Q, K, sinks = data
    rng = np.random.default_rng(11)
    mask = (rng.uniform(size=56) < 0.4).astype(np.int32)
    a = O.attn_decode_mixed_f32(Q, K[:40], K[40:], mask, sinks)
    keep = np.concatenate([K[:40], K[40:][mask == 1]])
    b = sdpa64(Q, f16r(keep), sinks)
    assert np.abs(a - b).max() < 1e-5


def test_single_row_no_sink_returns_row(data):
    Q, K, _ = data
    out = O.attn_decode_mixed_f32(Q, K[:1], None, None, np.full(64, -np.inf, np.float32))
    assert np.abs(out - f16r(K[:1])).max() < 1e-6


def test_empty_returns_zero(data):
    Q, _, sinks = data
    out = O.attn_decode_mixed_f32(Q, None, None, None, sinks)
    assert (out == 0).all()


def test_row_permutation_invariance(data):
    Q, K, sinks = data
    perm = np.random.default_rng(12).permutation(K.shape[0])
    a = O.attn_decode_mixed_f32(Q, K, None, None, sinks)
    b = O.attn_decode_mixed_f32(Q, K[perm], None, None, sinks)
    assert np.abs(a - b).max() < 1e-5


def test_fp8_path_equals_f32_path_on_dequantized_rows(data):
    Q, K, sinks = data
    codes, sexp, tail, deq = O.fp8_quant_rows(K)
    rows = np.arange(K.shape[0])
    a = O.attn_decode_fp8(Q, codes, sexp, tail, rows, sinks)
    b = O.attn_decode_mixed_f32(Q, deq, None, None, sinks)
    assert np.array_equal(a, b)
    # gathered rows
    sel = np.array([5, 3, 90, 17, 17, 0])
    a = O.attn_decode_fp8(Q, codes, sexp, tail, sel, sinks, n_threads=4)
    b = O.attn_decode_mixed_f32(Q, deq[sel], None, None, sinks)
    assert np.array_equal(a, b)


def test_separate_v_rows(data):
    # K == V gives the MLA form; with V != K the output is the fp64 softmax of
    # Q.K applied to V (sink = extra key with value 0)
    Q, K, sinks = data
    assert np.array_equal(O.attn_decode_kv_f32(Q, K, K, sinks),
                          O.attn_decode_mixed_f32(Q, K, None, None, sinks))
    V = np.random.default_rng(13).standard_normal(K.shape).astype(np.float32)
    out = O.attn_decode_kv_f32(Q, K, V, sinks)
    Kr, Vr = f16r(K).astype(np.float64), f16r(V).astype(np.float64)
    s = Q.astype(np.float64) @ Kr.T / np.sqrt(512)
    s = np.concatenate([s, sinks.astype(np.float64)[:, None]], axis=1)
    w = np.exp(s - s.max(axis=1, keepdims=True))
    ref = (w[:, :-1] @ Vr) / w.sum(axis=1, keepdims=True)
    assert np.abs(out - ref).max() < 1e-5
