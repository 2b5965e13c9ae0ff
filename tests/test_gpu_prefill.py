"""Causal chunked prefill over the FP8 cache vs the oracle: every output
within max|gpu - oracle| <= 2e-3 * RMS(oracle output), with P passed to
P . V as one f16 (the default) and as f16 hi + lo."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import ops, synth
from test_gpu_decode import check, make_cache, q_bf16, sinks_for

pytestmark = pytest.mark.gpu


def oracle_prefill(qf, codes, sexp, tail, n_cached, sinks):
    n_q = qf.shape[0]
    out = np.zeros((n_q, 64, 512), np.float32)
    O.lib().orc_attn_prefill_fp8(O.P(np.ascontiguousarray(qf, np.float32)), C.c_int(n_q),
                                 O.P(codes), O.P(sexp), O.P(tail), C.c_int(n_cached),
                                 O.P(np.ascontiguousarray(sinks, np.float32)), O.P(out),
                                 C.c_int(64), C.c_int(512), C.c_int(64), C.c_int(8))
    return out


def run(gpu, cache, bits, sinks, n_q, n_cached, row0=0, exact_p=False):
    q = torch.from_numpy(bits.view(np.int16)).to(gpu).view(torch.bfloat16)
    s = torch.from_numpy(np.ascontiguousarray(sinks, np.float32)).to(gpu)
    out = torch.full((n_q, 64, 512), float("nan"), device=gpu)
    ops.flash_attn_prefill_fp8(q, s, out, cache, n_q, n_cached, row0=row0, exact_p=exact_p)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("exact_p", [False, True])
@pytest.mark.parametrize("n_cached,n_q", [(0, 1), (0, 2), (5, 37), (100, 64), (1000, 33)])
def test_prefill_small(gpu, n_cached, n_q, exact_p):
    cache, (codes, sexp, tail) = make_cache(n_cached + n_q, 21 + n_q, gpu)
    bits, qf = q_bf16(22, n_q)
    sinks = sinks_for(23, 1)[0]
    got = run(gpu, cache, bits, sinks, n_q, n_cached, exact_p=exact_p)
    ref = oracle_prefill(qf, codes, sexp, tail, n_cached, sinks)
    for t in range(n_q):
        check(got[t], ref[t])


@pytest.mark.parametrize("exact_p", [False, True])
def test_prefill_offset_rows_and_outliers(gpu, exact_p):
    # the sequence starts at cache row 300; 5% outlier rows force rescales
    n_cached, n_q, row0 = 700, 40, 300
    cache, (codes, sexp, tail) = make_cache(row0 + n_cached + n_q, 24, gpu, outlier=0.05)
    bits, qf = q_bf16(25, n_q)
    sinks = sinks_for(26, 1)[0]
    got = run(gpu, cache, bits, sinks, n_q, n_cached, row0=row0, exact_p=exact_p)
    ref = oracle_prefill(qf, codes[row0:], sexp[row0:], tail[row0:], n_cached, sinks)
    for t in range(n_q):
        check(got[t], ref[t])


@pytest.mark.parametrize("exact_p", [False, True])
def test_prefill_cfg4_sampled_queries(gpu, exact_p):
    # full chunked-prefill shape: 2048 queries over 8192 cached rows + self;
    # a sample of queries is checked against the oracle's decode of the same rows
    n_cached, n_q = 8192, 2048
    cache, (codes, sexp, tail) = make_cache(n_cached + n_q, 27, gpu)
    bits, qf = q_bf16(28, n_q)
    sinks = sinks_for(29, 1)[0]
    got = run(gpu, cache, bits, sinks, n_q, n_cached, exact_p=exact_p)
    for t in (0, 1, 2, 777, 1500, 2046, 2047):
        rows = np.arange(n_cached + t + 1)
        ref = O.attn_decode_fp8(qf[t], codes, sexp, tail, rows, sinks, n_threads=8)
        check(got[t], ref)
    assert np.isfinite(got).all()
