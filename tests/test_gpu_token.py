"""One token's attention slice over all 43 layers (ds4cuda_amd.token:
Steps 11-16 of every layer, cuda/forward_token.cu:368-378) eager and as a
captured HIP graph: from identical sessions (300 tokens of synthetic
history, indexer top-k 8 so that the selection runs on every ratio-4 layer),
two consecutive tokens replayed from their graphs give the eager outputs bit
for bit and leave byte-identical session arenas. Eager work and host
synchronizations run between the replays."""
import ctypes as C

import numpy as np
import pytest
import torch

from ds4cuda_amd import session, token

pytestmark = pytest.mark.gpu

POS, CTX, TOPK = 300, 512, 8


def arena(s):
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    torch.cuda.synchronize()
    b = np.empty(s.s.arena_bytes, np.uint8)
    assert hip.hipMemcpy(b.ctypes.data, s.s.arena_base, b.nbytes, 2) == 0
    return b


def inputs(pos, gpu):
    g = torch.Generator(device=gpu)
    g.manual_seed(1000 + pos)
    r = lambda *shape: torch.randn(shape, generator=g, device=gpu)
    return r(43, 512), r(43, 4096), r(43, 64, 512), r(43, 1024)


def test_token_slice_graph_replay_matches_eager(gpu):
    w = token.synthetic_weights(gpu)
    a, b = session.Session(CTX), session.Session(CTX)
    try:
        token.fill_history(a, POS)
        token.fill_history(b, POS)
        assert np.array_equal(arena(a), arena(b))
        ta, tb = token.TokenSlice(a, w, top_k=TOPK), token.TokenSlice(b, w, top_k=TOPK)
        for pos in (POS, POS + 1):
            x = inputs(pos, gpu)
            out_e = torch.empty((43, 4096), device=gpu)
            ta.step(pos, *x, out_e)
            torch.cuda.synchronize()
            out_g = torch.full((43, 4096), float("nan"), device=gpu)
            g = tb.capture(pos, *x, out_g)
            torch.cuda.synchronize()
            assert torch.isnan(out_g).all()          # capturing ran nothing
            g.replay()
            torch.cuda.synchronize()
            e, r = out_e.cpu().numpy(), out_g.cpu().numpy()
            assert np.isfinite(e).all()
            assert np.array_equal(e.view(np.uint32), r.view(np.uint32)), pos
            assert np.array_equal(arena(a), arena(b)), pos
            for il in range(43):
                la, lb = a.layer(il), b.layer(il)
                assert (la.n_raw, la.raw_head, la.n_comp, la.n_index_comp) == \
                       (lb.n_raw, lb.raw_head, lb.n_comp, lb.n_index_comp)
        print(f"token slice: 2 tokens at pos {POS}, graph replay == eager bit for bit, arenas identical")
    finally:
        a.close()
        b.close()


def test_token_slice_fused_prologue_matches_separate_launches(gpu):
    """fused=True (each layer's FP8 push, compressor projections and indexer
    query / head weights as one launch) against fused=False (one launch
    each): bit-identical outputs and arenas over positions 380-383, where
    pos 383 emits on both the ratio-4 and the ratio-128 layers and, with
    top_k 95, the ratio-4 layers' indexer first holds more than top_k keys
    (95 before the emit, 96 after), so the selection starts on that step."""
    pos0, topk = 380, 95
    w = token.synthetic_weights(gpu)
    a, b = session.Session(CTX), session.Session(CTX)
    try:
        token.fill_history(a, pos0)
        token.fill_history(b, pos0)
        assert a.layer(2).n_index_comp == topk
        ta = token.TokenSlice(a, w, top_k=topk, fused=False)
        tb = token.TokenSlice(b, w, top_k=topk, fused=True)
        for pos in range(pos0, pos0 + 4):
            x = inputs(pos, gpu)
            oa, ob = torch.empty((43, 4096), device=gpu), torch.empty((43, 4096), device=gpu)
            ta.step(pos, *x, oa)
            tb.step(pos, *x, ob)
            torch.cuda.synchronize()
            e, r = oa.cpu().numpy(), ob.cpu().numpy()
            assert np.isfinite(e).all()
            assert np.array_equal(e.view(np.uint32), r.view(np.uint32)), pos
            assert np.array_equal(arena(a), arena(b)), pos
            for il in range(43):
                la, lb = a.layer(il), b.layer(il)
                assert (la.n_raw, la.raw_head, la.n_comp, la.n_index_comp) == \
                       (lb.n_raw, lb.raw_head, lb.n_comp, lb.n_index_comp), (pos, il)
        assert a.layer(2).n_index_comp == topk + 1
        print(f"token slice fused == separate launches bit for bit, pos {pos0}-{pos0 + 3}")
    finally:
        a.close()
        b.close()
