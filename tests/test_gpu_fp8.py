"""FP8 E4M3FN quantizer on the GPU vs the oracle: codes, scale exponents,
f16 tail and the fake-quant round trip must be bit-exact."""
import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import ops, synth

pytestmark = pytest.mark.gpu


def boundary_rows():
    """Rows whose blocks stress the scale rule and the encoder: block maxima at
    and just above 448*2^k, values on code midpoints, tiny and zero blocks."""
    rng = np.random.default_rng(7)
    vals = np.array([O.lib().orc_e4m3fn_value(i) for i in range(127)], np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    rows = []
    for k in range(-20, 12):
        for ulps in (0, 1, 2, 5, 11, 22, 23, 100):
            amax = np.float32(448.0 * 2.0 ** k)
            for _ in range(ulps):
                amax = np.nextafter(amax, np.float32(np.inf))
            blk = (rng.uniform(-1, 1, 512) * amax).astype(np.float32)
            blk[::64] = amax
            m = rng.choice(mids, 512) * (2.0 ** k) * rng.choice([-1, 1], 512)
            blk[1::7] = m[1::7].astype(np.float32)
            rows.append(blk)
    z = np.zeros(512, np.float32)
    rows.append(z)
    t = z.copy()
    t[:64] = -1e-7
    t[0] = 100.0
    rows.append(t)
    return np.stack(rows).astype(np.float32)


def inputs():
    a = synth.kv_rows(0, 1, 1000, outlier_frac=0.01)
    return np.concatenate([a, boundary_rows()])


def test_append_bit_exact(gpu):
    x = inputs()
    n = x.shape[0]
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    cache = ops.Fp8KVCache.empty(n + 5, device=gpu)
    cache.append(torch.from_numpy(x).to(gpu), row0=5)
    torch.cuda.synchronize()
    assert np.array_equal(cache.codes[5:].cpu().numpy(), codes)
    assert np.array_equal(cache.sexp[5:, :7].cpu().numpy(), sexp[:, :7])
    assert (cache.sexp[5:, 7].cpu().numpy() == 0).all()
    assert np.array_equal(cache.tail[5:].cpu().numpy().view(np.uint16), tail)


def test_append_scattered_rows(gpu):
    x = synth.kv_rows(1, 1, 64)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    dst = torch.randperm(300, generator=torch.Generator().manual_seed(0))[:64]
    cache = ops.Fp8KVCache.empty(300, device=gpu)
    cache.append(torch.from_numpy(x).to(gpu), dst_rows=dst.to(gpu))
    torch.cuda.synchronize()
    d = dst.numpy()
    assert np.array_equal(cache.codes.cpu().numpy()[d], codes)
    assert np.array_equal(cache.sexp.cpu().numpy()[d, :7], sexp[:, :7])


def test_round_trip_bit_exact_and_in_place(gpu):
    x = inputs()
    _, _, _, deq = O.fp8_quant_rows(x)
    xin = torch.from_numpy(x).to(gpu)
    out = torch.empty_like(xin)
    ops.launch_fp8_kv_quantize_round_trip_f32(xin, out, x.shape[0], 512, 64)
    ops.launch_fp8_kv_quantize_round_trip_f32(xin, xin, x.shape[0], 512, 64)   # in place
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), deq.view(np.uint32))
    assert np.array_equal(xin.cpu().numpy().view(np.uint32), deq.view(np.uint32))


def test_round_trip_small_head_dim(gpu):
    # indexer-sized rows (head_dim 128, n_rot 64: one 64-block)
    x = synth.kv_rows(2, 1, 33, head_dim=128)
    _, _, _, deq = O.fp8_quant_rows(x, n_rot=64)
    xin = torch.from_numpy(x).to(gpu)
    out = torch.empty_like(xin)
    ops.launch_fp8_kv_quantize_round_trip_f32(xin, out, 33, 128, 64)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), deq.view(np.uint32))
