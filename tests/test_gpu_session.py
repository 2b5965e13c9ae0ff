"""KV push / SWA eviction (reference fp32 layout, bit-exact) and the FP8
session arena (decode over ring + compressed rows vs the oracle)."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import Ds4HipError, lib, session, synth

pytestmark = pytest.mark.gpu


def f16r(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def test_swa_push_f32_matches_memmove_model(gpu):
    cap, hd = 128, 512
    raw = torch.full((cap, hd), 7.0, device=gpu)
    model = np.zeros((cap, hd), np.float32)
    n = 0
    for t in range(300):
        row = synth.normal(11, t, hd) * np.float32(1 + t % 7)
        n_new = session.swa_push_f32(raw, n, cap, torch.from_numpy(row).to(gpu), hd)
        if n < cap:
            model[n] = f16r(row)
        else:
            model[:-1] = f16r(model[1:])
            model[-1] = f16r(row)
        n = n_new
        if t in (0, 5, 127, 128, 129, 200, 299):
            torch.cuda.synchronize()
            got = raw.cpu().numpy()
            assert n == min(t + 1, cap)
            assert np.array_equal(got[:n].view(np.uint32), model[:n].view(np.uint32)), t


def test_comp_push_f32_and_full(gpu):
    comp = torch.zeros((4, 512), device=gpu)
    n = 0
    rows = [torch.from_numpy(synth.normal(12, i, 512)).to(gpu) for i in range(5)]
    for i in range(4):
        n = session.comp_push_f32(comp, n, 4, rows[i], 512)
    assert n == 4
    with pytest.raises(Ds4HipError) as e:
        session.comp_push_f32(comp, n, 4, rows[4], 512)
    assert e.value.code == -28
    torch.cuda.synchronize()
    assert torch.equal(comp, torch.stack(rows[:4]))


def fp8_deq(rows):
    return O.fp8_quant_rows(np.asarray(rows, np.float32))[3]


def check(got, ref, tol=2e-3):
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert np.abs(got - ref).max() <= tol * rms


def test_session_ring_and_compressed_decode(gpu):
    s = session.Session(1024)
    try:
        L0, L2 = s.layer(0), s.layer(2)
        assert (L0.compress_ratio, L2.compress_ratio, s.layer(3).compress_ratio) == (0, 4, 128)
        assert L2.cap_comp == 1024 // 4 + 2 and L0.cap_raw == 128
        q = torch.from_numpy(synth.normal(13, 0, 64 * 512)).to(gpu)
        sinks = torch.from_numpy(synth.normal(13, 1, 64)).to(gpu)
        out = torch.empty(64 * 512, device=gpu)
        qn = q.cpu().numpy().reshape(64, 512)
        sn = sinks.cpu().numpy()
        pushed = []
        for t in range(200):               # wraps the ring (evicts 72 rows)
            r = synth.normal(14, t, 512)
            if t % 50 == 7:
                r *= 8                     # an outlier row, as in the bench data
            pushed.append(r)
            s.push_raw(0, torch.from_numpy(r).to(gpu))
            if t in (0, 50, 127, 128, 199):
                s.decode(0, q, sinks, out)
                torch.cuda.synchronize()
                win = np.stack(pushed[-128:])
                ref = O.attn_decode_mixed_f32(qn, fp8_deq(win), None, None, sn)
                check(out.cpu().numpy().reshape(64, 512), ref)
        assert s.layer(0).n_raw == 128 and s.layer(0).raw_head == 200 % 128
        # layer 2: 10 raw rows, 6 compressed rows, 6 indexer keys
        raw2 = [synth.normal(15, t, 512) for t in range(10)]
        comp2 = [synth.normal(16, t, 512) * 2 for t in range(6)]
        keys = [synth.normal(17, t, 128) for t in range(6)]
        for r in raw2:
            s.push_raw(2, torch.from_numpy(r).to(gpu))
        for c, k in zip(comp2, keys):
            s.push_comp(2, torch.from_numpy(c).to(gpu))
            s.push_index_comp(2, torch.from_numpy(k).to(gpu))
        s.decode(2, q, sinks, out)
        torch.cuda.synchronize()
        ref = O.attn_decode_mixed_f32(qn, fp8_deq(raw2), fp8_deq(comp2), None, sn)
        check(out.cpu().numpy().reshape(64, 512), ref)
        # sparse: indexer top-3 of the 6 keys written straight into the row list
        iq = synth.normal(18, 0, 64 * 128)
        iw = synth.normal(18, 1, 64) / np.float32(np.sqrt(128 * 64))
        iq_t, iw_t = torch.from_numpy(iq).to(gpu), torch.from_numpy(iw).to(gpu)
        _, _, sel = s.layer_rows(2, 3)
        scores = torch.empty(6, device=gpu)
        scratch = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(6), dtype=torch.uint8,
                              device=gpu)
        L2 = s.layer(2)
        rc = lib().ds4hip_indexer_topk_positions(
            C.c_void_p(iq_t.data_ptr()), C.c_void_p(iw_t.data_ptr()),
            C.c_void_p(L2.index_comp_kv), 0, 6, 64, 128, 3, 0, C.c_void_p(scores.data_ptr()),
            C.c_void_p(scratch.data_ptr()), None, C.c_void_p(sel),
            C.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
        s.decode(2, q, sinks, out, n_selected=3)
        torch.cuda.synchronize()
        sc = np.zeros(6, np.float32)
        O.lib().orc_indexer_scores(O.P(iq), O.P(iw), O.P(np.stack(keys)), C.c_int(0), C.c_int(6),
                                   C.c_int(64), C.c_int(128), O.P(sc))
        mask = np.zeros(6, np.int32)
        O.lib().orc_topk_mask(O.P(sc), C.c_int(6), C.c_int(3), O.P(mask))
        ref = O.attn_decode_mixed_f32(qn, fp8_deq(raw2), fp8_deq(comp2), mask, sn)
        check(out.cpu().numpy().reshape(64, 512), ref)
        # errors: no compressed rows on layer 0; full compressed cache
        with pytest.raises(Ds4HipError):
            s.push_comp(0, torch.from_numpy(comp2[0]).to(gpu))
        row = torch.from_numpy(comp2[0]).to(gpu)
        for _ in range(L2.cap_comp - 6):
            s.push_comp(2, row)
        with pytest.raises(Ds4HipError) as e:
            s.push_comp(2, row)
        assert e.value.code == -28
        # reset: counters cleared, the row list is whole again
        s.reset()
        torch.cuda.synchronize()
        assert all(s.layer(il).n_raw == 0 and s.layer(il).n_comp == 0 for il in range(43))
        for r in raw2[:3]:
            s.push_raw(2, torch.from_numpy(r).to(gpu))
        for c in comp2[:4]:
            s.push_comp(2, torch.from_numpy(c).to(gpu))
        s.decode(2, q, sinks, out)
        torch.cuda.synchronize()
        ref = O.attn_decode_mixed_f32(qn, fp8_deq(raw2[:3]), fp8_deq(comp2[:4]), None, sn)
        check(out.cpu().numpy().reshape(64, 512), ref)
    finally:
        s.close()
