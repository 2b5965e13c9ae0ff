"""Pins of the RMSNorm oracle (orc_rms_norm_f32 / orc_rms_norm_batch_f32,
restating cuda/norm.cu:4-7 and cuda/norm.cuh:26-45) by what the definition
fixes independently of the formula's code: closed forms for a constant row
and a one-hot row, exact invariance under power-of-two scaling (eps = 0), and
the batch form's three weight modes against per-row single calls."""
import ctypes as C

import numpy as np

import oracle as O
from oracle import P


def norm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    O.lib().orc_rms_norm_f32(P(x), P(np.ascontiguousarray(w, np.float32)) if w is not None else None,
                             P(y), C.c_int(x.size), C.c_float(eps))
    return y


def test_constant_row_closed_form():
    n = 1024
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    for c in (0.25, 3.0, -7.5, 1e-3):
        y = norm(np.full(n, c, np.float32), w)
        ref = w.astype(np.float64) * c / np.sqrt(c * c + 1e-6)
        assert np.allclose(y, ref, rtol=3e-7, atol=0), c


def test_one_hot_row_closed_form():
    n, k, a = 512, 37, 5.0
    x = np.zeros(n, np.float32)
    x[k] = a
    y = norm(x, None)
    assert np.count_nonzero(y) == 1
    assert np.isclose(y[k], a / np.sqrt(a * a / n + 1e-6), rtol=3e-7)


def test_power_of_two_scaling_is_exact():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    y = norm(x, w, eps=0.0)
    for k in (-6, -1, 1, 5):
        assert np.array_equal(norm(x * np.float32(2.0 ** k), w, eps=0.0), y), k


def test_batch_weight_modes_match_single_rows():
    rng = np.random.default_rng(4)
    rows, n = 5, 512
    x = rng.standard_normal((rows, n)).astype(np.float32) * np.arange(1, rows + 1, dtype=np.float32)[:, None]
    w_shared = rng.standard_normal(n).astype(np.float32)
    w_rows = rng.standard_normal((rows, n)).astype(np.float32)
    for wd, w in ((0, None), (n, w_shared), (rows * n, w_rows)):
        y = np.zeros_like(x)
        O.lib().orc_rms_norm_batch_f32(P(x), P(w) if w is not None else None, C.c_int(wd), P(y),
                                       C.c_int(rows), C.c_int(n), C.c_float(1e-6))
        for r in range(rows):
            wr = None if wd == 0 else (w_shared if wd == n else w_rows[r])
            assert np.array_equal(y[r], norm(x[r], wr)), (wd, r)
