"""Pins orc_indexer_scores to the reference kernel's arithmetic, bit for bit.

The reference (cuda/indexer_allowed.cu:68-115 for f16 keys, :120-171 for fp32
keys) runs one block per key and one thread per head:

  * dot_h: `dot += qh[d] * kv[d]` over d ascending from 0.0f (nvcc contracts
    it to one fma per step);
  * relu `if (dot < 0.0f) dot = 0.0f`, then the rounded product dot * w[h];
  * per 32-lane warp an xor butterfly with offsets 16, 8, 4, 2, 1;
  * warp 0 combines the warp sums (lanes past the last warp hold 0.0f) with an
    xor butterfly over 8 lanes, offsets 4, 2, 1; lane 0 is the score.

Here that tree is built explicitly in numpy float32, array by array, with a
correctly rounded fp32 fma emulated from fp64 (an exact product, a TwoSum and
a fix-up of the double-rounding midpoint case), and compared with the oracle
bit for bit on small inputs. The same inputs under two plausible mistakes (a
sequential fma head sum, as an earlier oracle had; a product fused into the
butterfly's first addition) give different bits on some keys, so the check
would catch either.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from ds4cuda_amd import synth

P = O.P


def fma32(a, b, c):
    """Correctly rounded float32 a*b + c for float32 arrays."""
    a64, b64, c64 = (np.asarray(x, np.float32).astype(np.float64) for x in (a, b, c))
    p = a64 * b64                        # exact: 24 + 24 bits
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)    # s + err == p + c exactly (TwoSum)
    r = s.astype(np.float32)
    # s rounded to float32 is wrong only when s is a float32 midpoint that the
    # exact sum p + c is not (err != 0): then round toward err's side.
    other = np.nextafter(r, np.where(s > r.astype(np.float64), np.float32(np.inf), np.float32(-np.inf)))
    mid = (r.astype(np.float64) + other.astype(np.float64)) / 2
    fix = (mid == s) & (err != 0) & (r.astype(np.float64) != s)
    hi = np.where(other > r, other, r)
    lo = np.where(other > r, r, other)
    r = np.where(fix & (err > 0), hi, r)
    r = np.where(fix & (err < 0), lo, r)
    return r


def test_fma32_emulation():
    # 1 + 2^-24 is a float32 midpoint: exactly on it -> even; the fp64 sum
    # lands on it while the exact sum lies 2^-70 above -> up
    one = np.float32(1.0)
    assert fma32(np.float32(2.0 ** -24), one, one) == one
    a, b = np.float32(1 + 2.0 ** -23), np.float32(1 - 2.0 ** -24)       # a*b = 1 + 2^-24 - 2^-47
    c = np.float32(2.0 ** -47 * (1 + 2.0 ** -23))                       # + 2^-47 + 2^-70
    assert np.float32(np.float64(a) * np.float64(b) + np.float64(c)) == one   # naive: double rounding
    assert fma32(a, b, c) == np.float32(1 + 2.0 ** -23)
    got = fma32(np.float32(1 + 2.0 ** -23), np.float32(1 - 2.0 ** -23), np.float32(-1.0))
    assert got == np.float32(-(2.0 ** -46))                              # exact small result
    rng = np.random.default_rng(0)
    a, b, c = (rng.standard_normal(20000).astype(np.float32) for _ in range(3))
    r = fma32(a, b, c)
    # against exact rational arithmetic on a sample
    from fractions import Fraction
    for i in range(0, 20000, 97):
        ex = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        lo = np.float32(float(ex))
        cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
        dist = [abs(Fraction(float(x)) - ex) for x in cands]
        best = min(dist)
        winners = [x for x, d in zip(cands, dist) if d == best]
        if len(winners) == 1:
            assert r[i] == winners[0], i
        else:   # a tie: the even mantissa
            assert r[i] in winners and (r[i].view(np.uint32) & 1) == 0, i


def keys_as_float(keys_bits, kind):
    if kind == 0:
        return keys_bits.astype(np.float32)
    if kind == 1:
        return keys_bits.view(np.float16).astype(np.float32)
    return synth.bf16_bits_to_f32(keys_bits)


def reference_tree(q, w, k):
    """scores [n] of keys k [n, hd] (float32), the reference's operations."""
    n_head, hd = q.shape
    n = k.shape[0]
    n_warps = min((n_head + 31) // 32, 8)
    lanes = np.zeros((n, 32 * n_warps), np.float32)        # lane h of each key's block
    for h in range(min(n_head, 32 * n_warps)):
        dot = np.zeros(n, np.float32)
        for d in range(hd):
            dot = fma32(np.full(n, q[h, d], np.float32), k[:, d], dot)
        dot = np.where(dot < np.float32(0), np.float32(0), dot)
        lanes[:, h] = dot * np.float32(w[h])                 # numpy float32: one rounding
    warp_sums = np.zeros((n, 8), np.float32)
    for wv in range(n_warps):
        v = lanes[:, 32 * wv:32 * wv + 32].copy()
        for off in (16, 8, 4, 2, 1):
            v = v + v[:, np.arange(32) ^ off]
        warp_sums[:, wv] = v[:, 0]
    v = warp_sums
    for off in (4, 2, 1):
        v = v + v[:, np.arange(8) ^ off]
    return v[:, 0]


def oracle_scores(q, w, keys_bits, kind):
    n, hd = keys_bits.shape
    s = np.zeros(n, np.float32)
    O.lib().orc_indexer_scores(P(np.ascontiguousarray(q)), P(np.ascontiguousarray(w)),
                               P(np.ascontiguousarray(keys_bits)), C.c_int(kind), C.c_int(n),
                               C.c_int(q.shape[0]), C.c_int(hd), P(s))
    return s


def inputs(seed, n_head, hd, n, kind):
    q = synth.normal(seed, 0, n_head * hd).reshape(n_head, hd).astype(np.float32)
    w = (synth.normal(seed, 1, n_head) / np.sqrt(hd * n_head)).astype(np.float32)
    kf = synth.normal(seed, 2, n * hd).reshape(n, hd).astype(np.float32)
    if kind == 0:
        kb = kf
    elif kind == 1:
        kb = kf.astype(np.float16).view(np.uint16)
    else:
        kb = synth.to_bf16_bits(kf)
    return q, w, kb


@pytest.mark.parametrize("n_head,hd,kind", [(64, 128, 0), (64, 128, 1), (64, 128, 2), (40, 16, 0),
                                            (1, 7, 2), (33, 32, 1), (96, 8, 0)])
def test_oracle_scores_equal_the_reference_tree(n_head, hd, kind):
    n = 96
    q, w, kb = inputs(700 + n_head + hd + kind, n_head, hd, n, kind)
    got = oracle_scores(q, w, kb, kind)
    ref = reference_tree(q, w, keys_as_float(kb, kind))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_plausible_mistakes_fail_the_pin():
    """A sequential fma head sum and a fused product each change some bits."""
    n_head, hd, n = 64, 128, 96
    q, w, kb = inputs(777, n_head, hd, n, 2)
    k = keys_as_float(kb, 2)
    ref = reference_tree(q, w, k)
    seq = np.zeros(n, np.float32)       # s = fma(w_h, relu(dot_h), s) over h
    fused = np.zeros((n, 64), np.float32)
    for h in range(n_head):
        dot = np.zeros(n, np.float32)
        for d in range(hd):
            dot = fma32(np.full(n, q[h, d], np.float32), k[:, d], dot)
        r = np.where(dot < 0, np.float32(0), dot)
        seq = fma32(np.full(n, w[h], np.float32), r, seq)
        fused[:, h] = r
    # fused: the first butterfly level as fma(dot_h, w_h, partial_{h^16})
    lanes = np.zeros((n, 64), np.float32)
    for wv in range(2):
        base = 32 * wv
        for i in range(32):
            h, g = base + i, base + (i ^ 16)
            lanes[:, h] = fma32(fused[:, h], np.full(n, w[h], np.float32), fused[:, g] * w[g])
    ws = np.zeros((n, 8), np.float32)
    for wv in range(2):
        v = lanes[:, 32 * wv:32 * wv + 32]
        for off in (8, 4, 2, 1):
            v = v + v[:, np.arange(32) ^ off]
        ws[:, wv] = v[:, 0]
    for off in (4, 2, 1):
        ws = ws + ws[:, np.arange(8) ^ off]
    fz = ws[:, 0]
    assert (seq.view(np.uint32) != ref.view(np.uint32)).sum() > 5
    assert (fz.view(np.uint32) != ref.view(np.uint32)).sum() > 5
    # and the oracle sides with the reference tree
    assert np.array_equal(oracle_scores(q, w, kb, 2).view(np.uint32), ref.view(np.uint32))
