"""The batched-decode attention block end to end on the
GPU, exactly as bench.py runs it: 16 sequences with contexts ~U[1024, 16384]
(seed 5), ratio-4 compressors with fp32 weights, FP8 append into 256-row
pages, the top-2048 indexer over fp32 keys, decode over the 128 window rows +
the selected rows, inverse tail RoPE and the bf16 output projection
64 x 512 -> 4096. Two consecutive steps, every sequence checked against the
oracle run one sequence at a time:

  * KV rows appended this step: FP8 codes / exponents / tail bit-exact;
  * emitted compressed row: bit-exact up to a few rounding-midpoint flips;
  * emitted indexer key: 2e-3 x RMS (fp32 projections in another order);
  * indexer scores (over the device's keys) and selected positions: bit-exact;
  * attention output after inverse RoPE, and the projection: 2e-3 x RMS.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from oracle import P
from ds4cuda_amd import synth
from ds4cuda_amd.batch_block import BatchedAttentionBlock
from test_gpu_ops import close, t

pytestmark = pytest.mark.gpu

B, IN, OUT, TOPK, SWA = 16, 4096, 4096, 2048, 128


def make_weights(dev):
    n = lambda s, k, shape, std: synth.normal_device(70, s, int(np.prod(shape)), dev, std).reshape(shape)
    w = {
        "w_kv": n(1, 0, (1024, IN), 0.02), "w_gate": n(2, 0, (1024, IN), 0.02),
        "wi_kv": n(3, 0, (256, IN), 0.02), "wi_gate": n(4, 0, (256, IN), 0.02),
        "ape": n(5, 0, (4, 1024), 0.02).half().view(torch.int16).contiguous(),
        "ape_i": n(6, 0, (4, 256), 0.02).half().view(torch.int16).contiguous(),
        "wn": (1.0 + n(7, 0, (512,), 0.1)).contiguous(),
        "wn_i": (1.0 + n(8, 0, (128,), 0.1)).contiguous(),
        "w_out": n(9, 0, (OUT, 64 * 512), 0.02).to(torch.bfloat16).contiguous(),
    }
    return w


def host(x):
    return np.ascontiguousarray(x.cpu().numpy())


def test_batched_block_two_steps(gpu):
    ctx = np.random.default_rng(5).integers(1024, 16385, size=B)
    pos0 = (ctx - 1).astype(np.int64)
    w = make_weights(gpu)
    blk = BatchedAttentionBlock(w, B, int(pos0.max()) + 2, device=gpu)
    # history: compressed rows emitted before pos0, the full window, indexer keys
    win_pos = [np.arange(p - SWA + 1, p + 1) for p in pos0]      # window incl. pos0 (re-written)
    for b in range(B):
        n = int(pos0[b]) // 4
        comp = torch.from_numpy(synth.kv_rows(71, b, n, outlier_frac=0.01)).to(gpu)
        win = torch.from_numpy(synth.kv_rows(72, b, SWA)).to(gpu)
        keys = torch.from_numpy(synth.normal(73, b, n * 128).reshape(n, 128)).to(gpu)
        blk.load_history(b, comp, win, win_pos[b], keys)
    # compressor states: finite random contents (a window in progress)
    st = {k: synth.normal(74, i, B * 8 * wd).reshape(B, 8, wd)
          for i, (k, wd) in enumerate((("kv", 1024), ("sc", 1024), ("ikv", 256), ("isc", 256)))}
    blk.st_kv.copy_(t(st["kv"], gpu)); blk.st_sc.copy_(t(st["sc"], gpu))
    blk.sti_kv.copy_(t(st["ikv"], gpu)); blk.sti_sc.copy_(t(st["isc"], gpu))
    ost = {k: v.copy() for k, v in st.items()}                   # oracle copies
    ost_pre = {k: st[k].copy() for k in ("kv", "sc")}            # is_attn = 0 twin (pre-FP8)
    wh = {k: host(v) for k, v in w.items() if k != "w_out"}
    w_out_bits = host(w["w_out"].view(torch.int16)).view(np.uint16)
    worst = {"out": 0.0, "y": 0.0, "key": 0.0}
    flips = 0
    for step in range(2):
        pos = pos0 + step
        x = synth.normal(75, step, B * IN).reshape(B, IN)
        kv_cur = synth.normal(76, step, B * 512).reshape(B, 512)
        qb = synth.to_bf16_bits(synth.normal(77, step, B * 64 * 512)).reshape(B, 64, 512)
        q_idx = synth.normal(78, step, B * 64 * 128).reshape(B, 64, 128)
        w_idx = synth.normal(79, step, B * 64).reshape(B, 64) / np.float32(np.sqrt(128 * 64))
        sinks = synth.normal(80, step, B * 64).reshape(B, 64)
        y = blk.step(pos, t(x, gpu), t(kv_cur, gpu),
                     t(qb.view(np.int16), gpu).view(torch.bfloat16), t(q_idx, gpu), t(w_idx, gpu),
                     t(sinks, gpu))
        torch.cuda.synchronize()
        plan = blk.plan(pos)
        codes, sexp, tail = host(blk.cache.codes), host(blk.cache.sexp), host(blk.cache.tail)
        keys, scores = host(blk.keys), host(blk.scores)
        rowlist, emit_g, out_g, y_g = host(blk.rowlist), host(blk.emit), host(blk.out), host(y)
        for b in range(B):
            p = int(pos[b])
            # 1. compressors (oracle state carried across the two steps)
            e_ref, e_pre, ei_ref = (np.zeros(512, np.float32), np.zeros(512, np.float32),
                                    np.zeros(128, np.float32))
            args = lambda wkv, wg, ape, wn, hd: (P(x[b]), P(wh[wkv]), P(wh[wg]), P(wh[ape]),
                                                 P(wh[wn]), C.c_int(IN), C.c_int(hd), C.c_int(4),
                                                 C.c_int(p), C.c_int(2))
            r = O.lib().orc_compressor_step_w32(C.c_int(1), *args("w_kv", "w_gate", "ape", "wn", 512),
                                                P(ost["kv"][b]), P(ost["sc"][b]), P(e_ref))
            O.lib().orc_compressor_step_w32(C.c_int(0), *args("w_kv", "w_gate", "ape", "wn", 512),
                                            P(ost_pre["kv"][b]), P(ost_pre["sc"][b]), P(e_pre))
            O.lib().orc_compressor_step_w32(C.c_int(0), *args("wi_kv", "wi_gate", "ape_i", "wn_i", 128),
                                            P(ost["ikv"][b]), P(ost["isc"][b]), P(ei_ref))
            assert r == int(plan["emits"][b])
            # 2. appended rows
            ref_c, ref_s, ref_t, _ = O.fp8_quant_rows(kv_cur[b][None, :])
            pr = blk.phys(b, blk.window_lrow(p))
            assert np.array_equal(codes[pr], ref_c[0]) and np.array_equal(sexp[pr], ref_s[0])
            assert np.array_equal(tail[pr].view(np.uint16), ref_t[0])
            n_before = p // 4
            if r:
                # codes bit-exact; the fp32 RoPE tail at the f16 the cache stores
                f16 = lambda a: np.concatenate([a[:448], a[448:].astype(np.float16).astype(np.float32)])
                eg, er = f16(emit_g[b]), f16(e_ref)
                diff = np.nonzero(eg.view(np.uint32) != er.view(np.uint32))[0]
                assert len(diff) <= 4, f"seq {b}: {len(diff)} FP8 elements of the emit differ"
                rms = np.sqrt(np.mean(e_pre.astype(np.float64) ** 2))
                for e in diff:   # each a neighbouring code across a midpoint of the pre row
                    mid = 0.5 * (float(eg[e]) + float(er[e]))
                    assert abs(float(e_pre[e]) - mid) <= 1e-4 * rms, (b, e)
                flips += len(diff)
                pc = blk.phys(b, n_before)
                gc, gs, gt, _ = O.fp8_quant_rows(emit_g[b][None, :])
                assert np.array_equal(codes[pc], gc[0]) and np.array_equal(sexp[pc], gs[0])
                kr = int(blk.key_row0[b]) + n_before
                close(keys[kr], ei_ref, 2e-3)
                worst["key"] = max(worst["key"], float(np.abs(keys[kr] - ei_ref).max()
                                                       / np.sqrt(np.mean(ei_ref.astype(np.float64) ** 2))))
            # 3. indexer over the device's keys
            n = plan["n_comp"][b]
            k0 = int(blk.key_row0[b])
            ks = np.ascontiguousarray(keys[k0:k0 + n])
            sc = np.zeros(n, np.float32)
            O.lib().orc_indexer_scores(P(q_idx[b]), P(w_idx[b]), P(ks), C.c_int(0), C.c_int(n),
                                       C.c_int(64), C.c_int(128), P(sc))
            m = min(n, TOPK)
            if n > TOPK:
                assert np.array_equal(scores[k0:k0 + n].view(np.uint32), sc.view(np.uint32)), b
                sel = np.zeros(TOPK, np.int32)
                O.lib().orc_topk_positions(P(sc), C.c_int(n), C.c_int(TOPK), C.c_int(0), P(sel))
            else:
                sel = np.arange(n, dtype=np.int32)
            assert np.array_equal(rowlist[b, SWA:SWA + m], sel), f"seq {b}: positions differ"
            # 4. decode over window + selected rows, 5. inverse RoPE, 6. projection
            lrows = [blk.window_lrow(p - k) for k in range(SWA)] + list(sel)
            rows = np.array([blk.phys(b, int(l)) for l in lrows], np.int64)
            qf = synth.bf16_bits_to_f32(qb[b])
            o = O.attn_decode_fp8(qf, codes, sexp, tail.view(np.uint16), rows, sinks[b], n_threads=8)
            o_rot = np.zeros_like(o)
            O.lib().orc_rope_tail(P(o), P(o_rot), C.c_int(64), C.c_int(512), C.c_int(64), C.c_int(p),
                                  C.c_int(2), C.c_int(1))
            close(out_g[b], o_rot, 2e-3)
            yr = np.zeros(OUT, np.float32)
            O.lib().orc_bf16_matvec(P(w_out_bits), P(o_rot), P(yr), C.c_int(OUT), C.c_int(64 * 512))
            close(y_g[b], yr, 2e-3)
            rr = lambda g, r_: float(np.abs(g - r_).max() / np.sqrt(np.mean(r_.astype(np.float64) ** 2)))
            worst["out"] = max(worst["out"], rr(out_g[b], o_rot))
            worst["y"] = max(worst["y"], rr(y_g[b], yr))
    print(f"batched block: worst err/RMS out {worst['out']:.2e} y {worst['y']:.2e} "
          f"key {worst['key']:.2e}; emit FP8 midpoint flips {flips}")


def test_sparse_decode_full_size(gpu):
    """BASELINE configs[2] at its full size, as bench.py runs it: indexer over
    131072 bf16 keys (64 heads x 128), top-2048 including the last 128, decode
    over the 2048 gathered rows of a 131072-row FP8 cache. Positions and
    scores bit-exact; gathered rows' codes bit-exact; output 2e-3 x RMS."""
    from ds4cuda_amd import ops
    n, top_k, recent = 131072, 2048, 128
    keys = synth.to_bf16_bits(synth.normal(81, 1, n * 128)).reshape(n, 128)
    keys[5000:5040] = keys[777]                                   # planted ties
    qi = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(81, 2, 64 * 128))).reshape(64, 128)
    w = synth.normal(81, 3, 64) / np.float32(np.sqrt(128 * 64))
    x = synth.kv_rows_device(81, 4, n, gpu, outlier_frac=0.01)
    cache = ops.Fp8KVCache.empty(n, device=gpu)
    cache.append(x)
    qb = synth.to_bf16_bits(synth.normal(81, 5, 64 * 512)).reshape(1, 64, 512)
    sinks = synth.normal(81, 6, 64).reshape(1, 64)
    out = torch.empty((1, 64, 512), device=gpu)
    pos = torch.empty((1, top_k), dtype=torch.int32, device=gpu)
    _, _, scores = ops.indexer_topk_positions(t(qi, gpu), t(w, gpu),
                                              t(keys.view(np.int16), gpu).view(torch.bfloat16),
                                              top_k, recent, positions=pos[0])
    ops.flash_attn_decode_fp8(t(qb.view(np.int16), gpu).view(torch.bfloat16), t(sinks, gpu), out,
                              cache, [top_k], row_idx=pos)
    torch.cuda.synchronize()
    sc = np.zeros(n, np.float32)
    O.lib().orc_indexer_scores(P(qi), P(w), P(keys), C.c_int(2), C.c_int(n), C.c_int(64),
                               C.c_int(128), P(sc))
    ref_pos = np.zeros(top_k, np.int32)
    O.lib().orc_topk_positions(P(sc), C.c_int(n), C.c_int(top_k), C.c_int(recent), P(ref_pos))
    got_pos = host(pos)[0]
    assert np.array_equal(got_pos, ref_pos)
    assert np.array_equal(host(scores).view(np.uint32), sc.view(np.uint32))   # exact path
    assert np.array_equal(got_pos[-recent:], np.arange(n - recent, n))
    sel = torch.from_numpy(ref_pos.astype(np.int64)).to(gpu)
    xs = host(x[sel])
    c_ref, s_ref, t_ref, _ = O.fp8_quant_rows(xs)
    assert np.array_equal(host(cache.codes[sel]), c_ref)
    assert np.array_equal(host(cache.sexp[sel]), s_ref)
    assert np.array_equal(host(cache.tail[sel]).view(np.uint16), t_ref)
    ref = O.attn_decode_fp8(synth.bf16_bits_to_f32(qb[0]), c_ref, s_ref, t_ref,
                            np.arange(top_k), sinks[0], n_threads=8)
    close(host(out)[0], ref, 2e-3)
    err = np.abs(host(out)[0] - ref).max() / np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    print(f"sparse decode 131072 -> 2048: positions bit-exact, out err/RMS {err:.2e}")


def test_batched_block_graph_replay(gpu):
    """The captured step replays like the eager step: from the same saved
    state, replay k equals eager step k bit for bit (k = 1..3, with emits),
    with eager work and host synchronization between the replays."""
    nb = 4
    ctx = np.array([700, 1301, 2046, 4099])
    pos = (ctx - 1).astype(np.int64)   # sequence 2 emits on its first step
    w = make_weights(gpu)
    blk = BatchedAttentionBlock(w, nb, int(pos.max()) + 1, device=gpu)
    for b in range(nb):
        n = int(pos[b]) // 4
        blk.load_history(b, torch.from_numpy(synth.kv_rows(81, b, n)).to(gpu),
                         torch.from_numpy(synth.kv_rows(82, b, SWA)).to(gpu),
                         np.arange(pos[b] - SWA + 1, pos[b] + 1),
                         torch.from_numpy(synth.normal(83, b, n * 128).reshape(n, 128)).to(gpu))
    g = lambda s, shape: torch.from_numpy(synth.normal(84, s, int(np.prod(shape))).reshape(shape)).to(gpu)
    x, kv_cur = g(1, (nb, IN)), g(2, (nb, 512))
    q = g(3, (nb, 64, 512)).to(torch.bfloat16)
    q_idx, w_idx, sinks = g(4, (nb, 64, 128)), g(5, (nb, 64)) / float(np.sqrt(128 * 64)), g(6, (nb, 64))
    state = (blk.st_kv, blk.st_sc, blk.sti_kv, blk.sti_sc)
    saved = [s.clone() for s in state]
    eager = []
    for _ in range(3):
        eager.append(blk.step(pos, x, kv_cur, q, q_idx, w_idx, sinks).clone())
    torch.cuda.synchronize()
    assert not torch.equal(eager[0], eager[1])   # the state moved between the steps
    graph = blk.capture(pos, x, kv_cur, q, q_idx, w_idx, sinks)
    for s, v in zip(state, saved):
        s.copy_(v)
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(blk.y, eager[k]), k
        _ = (blk.y * 2).sum().item()   # eager work between replays


def test_batched_block_compressor_pair_equals_two_steps(gpu):
    """fused=True (both compressors in three launches,
    ds4hip_compressor_pair_step_batch_w32, the row pushes in one,
    ds4hip_batch_rows_push_f32, and the inverse RoPE in the decode merge)
    against fused=False (two ds4hip_compressor_decode_step_batch_w32 calls,
    two FP8 appends and a row scatter, a RoPE launch): the block output, both compressors' states, emitted rows, key
    rows and FP8 cache bit for bit over three steps (with emits: sequence 2
    emits on the first step, others later)."""
    nb = 4
    ctx = np.array([700, 1301, 2046, 4099])
    pos = (ctx - 1).astype(np.int64)
    w = make_weights(gpu)
    blks = [BatchedAttentionBlock(w, nb, int(pos.max()) + 4, device=gpu, fused=f) for f in (True, False)]
    for blk in blks:
        for b in range(nb):
            n = int(pos[b]) // 4
            blk.load_history(b, torch.from_numpy(synth.kv_rows(81, b, n)).to(gpu),
                             torch.from_numpy(synth.kv_rows(82, b, SWA)).to(gpu),
                             np.arange(pos[b] - SWA + 1, pos[b] + 1),
                             torch.from_numpy(synth.normal(83, b, n * 128).reshape(n, 128)).to(gpu))
    g = lambda s, shape: torch.from_numpy(synth.normal(85, s, int(np.prod(shape))).reshape(shape)).to(gpu)
    n_emit = 0
    for step in range(3):
        p = pos + step
        x, kv_cur = g(10 * step + 1, (nb, IN)), g(10 * step + 2, (nb, 512))
        q = g(10 * step + 3, (nb, 64, 512)).to(torch.bfloat16)
        q_idx = g(10 * step + 4, (nb, 64, 128))
        w_idx = g(10 * step + 5, (nb, 64)) / float(np.sqrt(128 * 64))
        sinks = g(10 * step + 6, (nb, 64))
        ys = [blk.step(p, x, kv_cur, q, q_idx, w_idx, sinks).clone() for blk in blks]
        torch.cuda.synchronize()
        n_emit += int(sum((int(v) + 1) % 4 == 0 for v in p))
        assert torch.isfinite(ys[0]).all()
        assert torch.equal(ys[0], ys[1]), step
        for name in ("st_kv", "st_sc", "sti_kv", "sti_sc", "emit", "emit_i"):
            assert torch.equal(getattr(blks[0], name), getattr(blks[1], name)), (step, name)
        # the key rows (the last one is the trash row that every non-emitting
        # sequence writes at once: its content is whichever write lands last)
        assert torch.equal(blks[0].keys[:-1], blks[1].keys[:-1]), step
        for name in ("codes", "sexp", "tail"):   # the cache, its trash row aside
            assert torch.equal(getattr(blks[0].cache, name)[:-1], getattr(blks[1].cache, name)[:-1]), (step, name)
    assert n_emit >= 2
