"""Pins the oracle's FP8 E4M3FN quantizer (oracle/fp8.cpp) against
independent statements of the same arithmetic: the OCP E4M3FN decoding,
torch's float8_e4m3fn cast, numpy's float16 cast and closed forms."""
import math

import numpy as np
import pytest
import torch

import oracle as O


def test_table_is_ocp_e4m3fn():
    # cuda/fp8_kv.cuh:21-26: value(1) = 2^-9, value(8) = 2^-6, value(126) = 448
    codes = torch.arange(127, dtype=torch.uint8)
    ocp = codes.view(torch.float8_e4m3fn).float().numpy()
    mine = np.array([O.lib().orc_e4m3fn_value(i) for i in range(127)], np.float32)
    assert np.array_equal(mine, ocp)
    assert mine[1] == 2.0 ** -9 and mine[8] == 2.0 ** -6 and mine[126] == 448.0


def _torch_code(v):
    return torch.tensor(v, dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_nearest_picker_matches_torch_cast():
    lib = O.lib()
    vals = np.array([O.lib().orc_e4m3fn_value(i) for i in range(127)], np.float64)
    # every code, every midpoint (ties -> even code), points just around midpoints
    mids = (vals[:-1] + vals[1:]) / 2
    probe = np.concatenate([vals, mids, np.nextafter(mids.astype(np.float32), 0),
                            np.nextafter(mids.astype(np.float32), 1000)]).astype(np.float32)
    rng = np.random.default_rng(0)
    probe = np.concatenate([probe, rng.uniform(0, 448, 20000).astype(np.float32),
                            (2.0 ** rng.uniform(-14, 8.8, 20000)).astype(np.float32)])
    probe = np.clip(probe, 0, 448)
    ref = _torch_code(probe) & 0x7F
    mine = np.array([lib.orc_e4m3fn_nearest_index(float(v)) for v in probe])
    assert np.array_equal(mine, ref)


def test_f16_conversion_matches_numpy():
    lib = O.lib()
    all_h = np.arange(65536, dtype=np.uint16)
    fin = all_h[(all_h & 0x7C00) != 0x7C00]
    f = fin.view(np.float16).astype(np.float32)
    # exact values, midpoints between neighbours, and random floats
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    rnd = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-9, 5, 50000)).astype(np.float32)
    probe = np.concatenate([f, mids, rnd, np.float32([70000.0, -1e-30, 6e-8, 3e-8])])
    mine = np.array([lib.orc_f32_to_f16(float(v)) for v in probe], np.uint16)
    with np.errstate(over="ignore"):
        ref = probe.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, ref)
    back = np.array([lib.orc_f16_to_f32(int(h)) for h in fin], np.float32)
    assert np.array_equal(back.view(np.uint32), f.view(np.uint32))


def test_scale_exp_closed_form():
    lib = O.lib()
    rng = np.random.default_rng(2)
    amax = np.concatenate([(2.0 ** rng.uniform(-14, 12, 20000)).astype(np.float32),
                           np.float32([448.0 * 2.0 ** k for k in range(-12, 8)]),
                           np.float32([0.0, 1e-5, 1e-4, 448.0, 449.0])])
    for a in amax:
        e = lib.orc_fp8_scale_exp(float(a))
        y = float(np.float32(max(float(a), float(np.float32(1e-4))) / np.float32(448.0)))
        m, k = math.frexp(y)           # y = m 2^k, m in [0.5, 1)
        exact = k - 1 if m == 0.5 else k
        # correctly rounded log2 may round k-1+t back to an integer only when
        # y is within 2^-18 (relative) above a power of two
        if e != exact:
            assert e == exact - 1 and (y / 2.0 ** e - 1.0) < 2.0 ** -18
        assert abs(y / 2.0 ** e) <= 1.0 + 2.0 ** -18     # v = x/scale stays within 448(1+eps)
        assert y / 2.0 ** e > 0.5
    assert lib.orc_fp8_scale_exp(0.0) == -22             # floor 1e-4 -> 2^-22


def test_quant_row_properties():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x[1] *= 0.0                                           # all-zero blocks
    x[2, :64] = 448.0                                     # exact max
    x[3, :64] = -1e-7                                     # negative tiny -> -0
    x[3, 0] = 100.0
    x[4] *= 1000.0
    x[5, 5] = -0.0
    codes, sexp, tail, deq = O.fp8_quant_rows(x)
    # decode codes with torch (independent table) and the scales
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    scale = np.repeat(2.0 ** sexp[:, :7].astype(np.float64), 64, axis=1)
    assert np.array_equal((dec * scale).astype(np.float32), deq[:, :448])
    assert np.array_equal(deq[:, 448:], x[:, 448:])
    assert np.array_equal(tail, x[:, 448:].astype(np.float16).view(np.uint16))
    assert (sexp[1, :7] == -22).all() and (codes[1] == 0).all()
    assert (codes[2, :64] == 126).all()
    assert (codes[3, 1:64] == 0x80).all() and np.signbit(deq[3, 1:64]).all()
    # rounding error bound: half a code step at the block's scale
    for r in range(x.shape[0]):
        for b in range(7):
            blk = x[r, 64 * b:64 * b + 64].astype(np.float64)
            s = 2.0 ** int(sexp[r, b])
            err = np.abs(deq[r, 64 * b:64 * b + 64] - blk)
            step = np.maximum(2.0 ** np.floor(np.log2(np.maximum(np.abs(blk) / s, 2 ** -6))) / 8,
                              2.0 ** -9) * s
            assert (err <= step / 2 + 1e-30).all()
    # brute force on one block: every code's value is at least as far
    vals = np.array([O.lib().orc_e4m3fn_value(i) for i in range(127)])
    blk = x[0, :64]
    s = 2.0 ** int(sexp[0, 0])
    for j in range(64):
        v = min(abs(blk[j]) / s, 448.0)
        assert abs(vals[codes[0, j] & 0x7F] - v) <= np.min(np.abs(vals - v)) + 1e-12
