"""Checks of an FP8-quantized emitted row (the attention compressor's output).

The emitted row is the FP8 E4M3FN round trip of a pre-quantization row
(pool -> RMSNorm -> tail RoPE). The device computes that row in a different
fp32 order than the oracle, so the two pre-quantization rows differ by a few
ulp, and an element whose value lies between the two of them and a rounding
midpoint (or a block whose absmax straddles a scale boundary) can land on the
neighbouring code. This module checks:

  1. the device's pre-quantization row against the oracle's at the attention
     tolerance (2e-3 x RMS);
  2. the device's FP8 row against the oracle's FP8 round trip of the DEVICE's
     own pre-quantization row: bit-exact (the quantizer itself is exact);
  3. the device's FP8 row against the oracle's FP8 row (the RoPE tail, which
     the round trip passes through in fp32, at the f16 the cache stores): bit-exact except at
     elements where a rounding midpoint of the pair of codes lies between the
     oracle's and the device's pre-quantization values — and those must be few.
"""
from __future__ import annotations

import numpy as np

import oracle as O


def check_fp8_emit(got_q, got_pre, ref_q, ref_pre, tol=2e-3, max_flips=4, n_rot=64):
    got_q = np.asarray(got_q, np.float32).reshape(-1)
    got_pre = np.asarray(got_pre, np.float32).reshape(-1)
    ref_q = np.asarray(ref_q, np.float32).reshape(-1)
    ref_pre = np.asarray(ref_pre, np.float32).reshape(-1)
    rms = float(np.sqrt(np.mean(ref_pre.astype(np.float64) ** 2))) + 1e-30
    err = float(np.abs(got_pre.astype(np.float64) - ref_pre).max())
    assert np.isfinite(got_pre).all() and err <= tol * rms, \
        f"pre-quantization row: err {err:.3e} > {tol} * rms {rms:.3e}"
    # 2. the device's quantizer on its own values is exact
    _, _, _, deq = O.fp8_quant_rows(got_pre[None, :])
    assert np.array_equal(got_q.view(np.uint32), deq[0].view(np.uint32)), \
        "device FP8 round trip differs from the oracle's on the same pre-quantization row"
    # 3. against the oracle's FP8 row: only midpoint flips between the two pre rows.
    # The round trip passes the RoPE tail through in fp32; the cache stores it
    # as f16, so the tail is compared at f16 (its own rounding midpoints).
    n_nope = got_q.size - n_rot
    f16 = lambda a: a.astype(np.float16).astype(np.float32)
    got_q = np.concatenate([got_q[:n_nope], f16(got_q[n_nope:])])
    ref_q = np.concatenate([ref_q[:n_nope], f16(ref_q[n_nope:])])
    flips = np.nonzero(got_q.view(np.uint32) != ref_q.view(np.uint32))[0]
    assert len(flips) <= max_flips, (
        f"{len(flips)} FP8 elements differ (> {max_flips}); pre-row err/RMS {err / rms:.2e}; "
        f"first {flips[:12].tolist()}: got {got_q[flips[:6]].tolist()} ref {ref_q[flips[:6]].tolist()} "
        f"got_pre {got_pre[flips[:6]].tolist()} ref_pre {ref_pre[flips[:6]].tolist()}")
    for e in flips:
        lo, hi = sorted((float(got_pre[e]), float(ref_pre[e])))
        mid = 0.5 * (float(got_q[e]) + float(ref_q[e]))
        assert lo <= mid <= hi, (f"element {e}: codes {got_q[e]} vs {ref_q[e]} differ but their "
                                 f"midpoint {mid} is not between {lo} and {hi}")
    return err / rms, len(flips)
