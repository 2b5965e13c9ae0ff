"""The allocation-free fp32 decode entry point
(ds4hip_flash_attn_decode_mixed_f32_noalloc) through the C-ABI: two calls in
a row, the second with a smaller input, each checked against the allocating
entry point ds4hip_flash_attn_decode_mixed_f32 on the same inputs (max-abs
difference <= 2e-3 x RMS; the two plan their split-K chunks differently, so
the fp32 sums run in another order) and against the oracle (same bar)."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import lib, synth

pytestmark = pytest.mark.gpu


def ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.sqrt(np.mean(ref ** 2)))


@pytest.mark.parametrize("sizes", [((128, 3000), (100, 40))])
def test_noalloc_matches_allocating_entry_point(gpu, sizes):
    L = lib()
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for call, (n_raw, n_comp) in enumerate(sizes):
        raw = synth.kv_rows(60 + call, 1, n_raw)
        comp = synth.kv_rows(60 + call, 2, n_comp) * 0.8
        mask = (synth.uniform(60 + call, 3, n_comp) < 0.7).astype(np.int32)
        Q = synth.normal(60 + call, 4, 64 * 512).reshape(64, 512)
        sinks = synth.normal(60 + call, 5, 64)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
        gq, graw, gcomp, gmask, gs = t(Q), t(raw), t(comp), t(mask), t(sinks)
        out_na = torch.full((64, 512), 7.0, device=gpu)
        out_ref = torch.zeros((64, 512), device=gpu)
        rc = L.ds4hip_flash_attn_decode_mixed_f32_noalloc(ptr(gq), ptr(graw), ptr(gcomp),
                                                          ptr(gmask), ptr(gs), ptr(out_na), 64,
                                                          n_raw, n_comp, 512, st)
        assert rc == 0
        rc = L.ds4hip_flash_attn_decode_mixed_f32(ptr(gq), ptr(graw), ptr(gcomp), ptr(gmask),
                                                  ptr(gs), ptr(out_ref), 64, n_raw, n_comp, 512,
                                                  st)
        assert rc == 0
        torch.cuda.synchronize()
        got, ref = out_na.cpu().numpy(), out_ref.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel(got, ref) <= 2e-3, (call, rel(got, ref))
        orc = O.attn_decode_mixed_f32(Q, raw, comp, mask, sinks)
        assert rel(got, orc) <= 2e-3, (call, rel(got, orc))
        print(f"noalloc call {call} ({n_raw} + {n_comp} rows): vs allocating entry "
              f"{rel(got, ref):.2e}, vs oracle {rel(got, orc):.2e}")
    # beyond the maximum: a clear -22, nothing launched
    big = 1 << 22
    assert L.ds4hip_flash_attn_decode_mixed_f32_noalloc(ptr(gq), ptr(graw), ptr(gcomp), None,
                                                        ptr(gs), ptr(out_na), 64, 1, big, 512,
                                                        st) == -22
