"""RoPE, matvecs, indexer and compressor on the GPU vs the oracle.

Bit-exact: indexer scores (fixed fma order) and every selected position/mask.
Tolerance (max |gpu - oracle| <= tol * RMS(oracle)): RoPE (cos/sin are libm vs
device math), matvecs and the compressor (different summation orders)."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from oracle import P
from ds4cuda_amd import ops, synth
from test_oracle_misc import q8_pack, rope

pytestmark = pytest.mark.gpu


def close(got, ref, tol):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) + 1e-30
    err = np.abs(got - ref).max()
    assert np.isfinite(got).all() and err <= tol * rms, f"err {err:.3e} > {tol} * rms {rms:.3e}"


def t(a, dev, dt=None):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a if dt is None else a.astype(dt)).to(dev)


@pytest.mark.parametrize("il,pos", [(0, 9), (1, 1000), (2, 4093), (3, 131071), (42, 7)])
def test_rope_forward_inverse(gpu, il, pos):
    x = synth.normal(1, il, 64 * 512).reshape(64, 512)
    xi = t(x, gpu)
    y = torch.empty_like(xi)
    ops.launch_tail_rope_yarn_f32(xi, y, 64, 512, 64, pos, il)
    z = y.clone()
    ops.launch_tail_rope_yarn_inverse_f32(z, z, 64, 512, 64, pos, il)   # in place
    torch.cuda.synchronize()
    ref = rope(x, pos, il)
    assert np.array_equal(y.cpu().numpy()[:, :448], x[:, :448])
    close(y.cpu().numpy(), ref, 1e-5)
    close(z.cpu().numpy(), rope(ref, pos, il, inverse=True), 1e-5)


@pytest.mark.parametrize("out_dim,in_dim", [(1024, 4096), (64, 4096), (256, 1000)])
def test_mul_mv_f16(gpu, out_dim, in_dim):
    w = (synth.normal(2, 1, out_dim * in_dim) * 0.02).astype(np.float16).view(np.uint16)
    x = synth.normal(2, 2, in_dim)
    y = torch.empty(out_dim, dtype=torch.float32, device=gpu)
    ops.launch_mul_mv_f16_f32(t(w.view(np.int16), gpu), t(x, gpu), y, out_dim, in_dim)
    torch.cuda.synchronize()
    ref = np.zeros(out_dim, np.float32)
    O.lib().orc_mul_mv_f16_f32(P(np.ascontiguousarray(w)), P(x), P(ref), C.c_int(out_dim),
                               C.c_int(in_dim))
    close(y.cpu().numpy(), ref, 1e-5)


def test_q8_grouped_and_dense(gpu):
    n_groups, group_dim, rank = 8, 4096, 1024
    w = synth.normal(3, 1, n_groups * rank * group_dim).reshape(n_groups * rank, group_dim) * 0.02
    Wb, _, _ = q8_pack(w)
    x = synth.normal(3, 2, n_groups * group_dim)
    y = torch.empty(n_groups * rank, dtype=torch.float32, device=gpu)
    ops.launch_mul_mv_q8_0_q8_0_grouped_f32(t(Wb, gpu), t(x, gpu), y, n_groups, group_dim, rank)
    xq = torch.empty(n_groups * group_dim, dtype=torch.int8, device=gpu)
    xs = torch.empty(n_groups * group_dim // 32, dtype=torch.float32, device=gpu)
    y2 = torch.empty_like(y)
    ops.launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(t(Wb, gpu), t(x, gpu), y2, n_groups,
                                                     group_dim, rank, xq, xs)
    torch.cuda.synchronize()
    ref = np.zeros(n_groups * rank, np.float32)
    O.lib().orc_q8_grouped_matvec(P(np.ascontiguousarray(Wb)), P(x), P(ref), C.c_int(n_groups),
                                  C.c_int(group_dim), C.c_int(rank))
    close(y.cpu().numpy(), ref, 1e-5)
    assert torch.equal(y, y2)
    # the int8 activations are an exact function of x
    xq_ref = np.zeros(x.size, np.int8)
    xs_ref = np.zeros(x.size // 32, np.float32)
    O.lib().orc_q8_quantize_act(P(x), C.c_int(x.size), P(xq_ref), P(xs_ref))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert np.array_equal(xs.cpu().numpy(), xs_ref)
    # dense 8192 -> 4096
    wd = synth.normal(4, 1, 4096 * 8192).reshape(4096, 8192) * 0.02
    Wd, _, _ = q8_pack(wd)
    xd = synth.normal(4, 2, 8192)
    yd = torch.empty(4096, dtype=torch.float32, device=gpu)
    xq2 = torch.empty(8192, dtype=torch.int8, device=gpu)
    xs2 = torch.empty(256, dtype=torch.float32, device=gpu)
    ops.launch_mul_mv_q8_0_q8_0_f32_prealloc(t(Wd, gpu), t(xd, gpu), yd, 4096, 8192, xq2, xs2)
    torch.cuda.synchronize()
    refd = np.zeros(4096, np.float32)
    O.lib().orc_q8_matvec(P(np.ascontiguousarray(Wd)), P(xd), P(refd), C.c_int(4096), C.c_int(8192))
    close(yd.cpu().numpy(), refd, 1e-5)


def test_mul_mm_bf16(gpu):
    n_rows, n_cols, nb = 512, 4096, 16
    W = synth.to_bf16_bits(synth.normal(5, 1, n_rows * n_cols) * 0.02).reshape(n_rows, n_cols)
    X = synth.normal(5, 2, nb * n_cols).reshape(nb, n_cols)
    Y = torch.empty((nb, n_rows), dtype=torch.float32, device=gpu)
    Wt = t(W.view(np.int16), gpu).view(torch.bfloat16)
    ops.mul_mm_bf16_f32(Wt, t(X, gpu), Y, n_rows, n_cols, nb)
    torch.cuda.synchronize()
    ref = X.astype(np.float64) @ synth.bf16_bits_to_f32(W).astype(np.float64).T
    close(Y.cpu().numpy(), ref, 1e-4)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("n_comp,top_k", [(3000, 512), (600, 512), (400, 512), (5000, 1)])
def test_indexer_mask_bit_exact(gpu, kind, n_comp, top_k):
    n_head, hd = 64, 128
    q = synth.normal(6, 1, n_head * hd)
    w = synth.normal(6, 2, n_head) / np.float32(np.sqrt(hd * n_head))
    kf = synth.normal(6, 3, n_comp * hd)
    if kind == 1:
        keys = kf.astype(np.float16)
        kt = t(keys.view(np.int16), gpu)
    elif kind == 2:
        keys = synth.to_bf16_bits(kf)
        kt = t(keys.view(np.int16), gpu).view(torch.bfloat16)
    else:
        keys = kf
        kt = t(keys, gpu)
    ref_s = np.zeros(n_comp, np.float32)
    O.lib().orc_indexer_scores(P(q), P(w), P(np.ascontiguousarray(keys)), C.c_int(kind),
                               C.c_int(n_comp), C.c_int(n_head), C.c_int(hd), P(ref_s))
    ref_m = np.zeros(n_comp, np.int32)
    O.lib().orc_topk_mask(P(ref_s), C.c_int(n_comp), C.c_int(top_k), P(ref_m))
    mask = torch.empty(n_comp, dtype=torch.int32, device=gpu)
    scores = torch.empty(n_comp, dtype=torch.float32, device=gpu)
    if kind == 0:
        ops.launch_indexer_score_topk_f32_i32(t(q, gpu), t(w, gpu), kt, n_comp, n_head, hd, top_k,
                                              mask, scores)
    elif kind == 1:
        ops.launch_indexer_score_topk_i32(t(q, gpu), t(w, gpu), kt, n_comp, n_head, hd, top_k,
                                          mask, scores)
    else:
        _, _, scores = ops.indexer_topk_positions(t(q, gpu), t(w, gpu), kt.view(n_comp, hd),
                                                  top_k, 0, mask=mask,
                                                  scores=scores)
    torch.cuda.synchronize()
    if n_comp > top_k:
        assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(mask.cpu().numpy(), ref_m)


def test_indexer_positions_with_ties_and_recent(gpu):
    n_comp, n_head, hd, top_k, recent = 131072, 64, 128, 2048, 128
    q = synth.to_bf16_bits(synth.normal(7, 1, n_head * hd))
    qf = synth.bf16_bits_to_f32(q)
    w = synth.normal(7, 2, n_head) / np.float32(np.sqrt(hd * n_head))
    kb = synth.to_bf16_bits(synth.normal(7, 3, n_comp * hd)).reshape(n_comp, hd)
    kb[1000:1100] = kb[5]            # planted duplicates -> tied scores
    ref_s = np.zeros(n_comp, np.float32)
    O.lib().orc_indexer_scores(P(qf), P(w), P(np.ascontiguousarray(kb)), C.c_int(2),
                               C.c_int(n_comp), C.c_int(n_head), C.c_int(hd), P(ref_s))
    ref_p = np.zeros(top_k, np.int32)
    O.lib().orc_topk_positions(P(ref_s), C.c_int(n_comp), C.c_int(top_k), C.c_int(recent),
                               P(ref_p))
    kt = t(kb.view(np.int16), gpu).view(torch.bfloat16)
    mask = torch.empty(n_comp, dtype=torch.int32, device=gpu)
    pos, _, scores = ops.indexer_topk_positions(t(qf, gpu), t(w, gpu), kt, top_k, recent, mask=mask)
    torch.cuda.synchronize()
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(pos.cpu().numpy(), ref_p)
    m = mask.cpu().numpy()
    assert m.sum() == top_k and np.array_equal(np.nonzero(m)[0], ref_p)


@pytest.mark.parametrize("case", ["spread", "bin_overflow", "zero_ties", "mask_only"])
def test_indexer_large_select_edges(gpu, case):
    """The one-workgroup selection of long candidate lists (more than 16384
    candidates) with designed scores: one head, q = e_0, w = 1 and fp32 keys
    give score = relu(key[0]) exactly. spread: few ties; bin_overflow: 40000
    equal keys (the threshold bin holds more than the 8192 listed keys, so
    the rescans run); zero_ties: half the keys relu to 0 and the selection
    reaches into those ties; mask_only: the 0/1 mask alone. Positions and
    mask bit-exact against the oracle's (score desc, index asc) rule."""
    n_head, hd = 1, 128
    rng = np.random.default_rng(11)
    n_comp, top_k, recent = {"spread": (200000, 2048, 128), "bin_overflow": (40000, 1000, 16),
                             "zero_ties": (50000, 26000, 64), "mask_only": (30000, 700, 0)}[case]
    k = np.zeros((n_comp, hd), np.float32)
    if case == "spread":
        k[:, 0] = np.round(rng.standard_normal(n_comp) * 64) / 64   # ~400 levels: ties too
    elif case == "bin_overflow":
        k[:, 0] = 1.0
    elif case == "zero_ties":
        k[:, 0] = rng.standard_normal(n_comp)
    else:
        k[:, 0] = rng.standard_normal(n_comp)
    k[:, 1:] = rng.standard_normal((n_comp, hd - 1)).astype(np.float32)
    q = np.zeros(hd, np.float32)
    q[0] = 1.0
    w = np.ones(1, np.float32)
    ref_s = np.zeros(n_comp, np.float32)
    O.lib().orc_indexer_scores(P(q), P(w), P(k), C.c_int(0), C.c_int(n_comp), C.c_int(n_head),
                               C.c_int(hd), P(ref_s))
    assert np.array_equal(ref_s, np.maximum(k[:, 0], 0))
    mask = torch.empty(n_comp, dtype=torch.int32, device=gpu)
    if case == "mask_only":
        ref_m = np.zeros(n_comp, np.int32)
        O.lib().orc_topk_mask(P(ref_s), C.c_int(n_comp), C.c_int(top_k), P(ref_m))
        ops.indexer_topk_positions(t(q, gpu), t(w, gpu), t(k, gpu), top_k, 0, mask=mask,
                                   positions=torch.empty(top_k, dtype=torch.int32, device=gpu))
        torch.cuda.synchronize()
        assert np.array_equal(mask.cpu().numpy(), ref_m)
        return
    ref_p = np.zeros(top_k, np.int32)
    O.lib().orc_topk_positions(P(ref_s), C.c_int(n_comp), C.c_int(top_k), C.c_int(recent), P(ref_p))
    pos, _, scores = ops.indexer_topk_positions(t(q, gpu), t(w, gpu), t(k, gpu), top_k, recent, mask=mask)
    torch.cuda.synchronize()
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(pos.cpu().numpy(), ref_p)
    assert np.array_equal(np.nonzero(mask.cpu().numpy())[0], ref_p)


def test_short_circuit_and_scale(gpu):
    out = torch.zeros(100, dtype=torch.int32, device=gpu)
    ops.launch_indexer_allowed_short_circuit_i32(out, 100, 512)
    y = torch.arange(70, dtype=torch.float32, device=gpu)
    ops.launch_scale_inplace_f32(y, 70, 0.5)
    torch.cuda.synchronize()
    assert (out == 1).all() and torch.equal(y, torch.arange(70, dtype=torch.float32, device=gpu) * 0.5)
    with pytest.raises(Exception):
        ops.launch_indexer_allowed_short_circuit_i32(out, 600, 512)


@pytest.mark.parametrize("is_attn,ratio,hd,il", [(1, 4, 512, 2), (0, 4, 128, 2), (1, 128, 512, 3)])
def test_compressor_steps(gpu, is_attn, ratio, hd, il):
    """Every state row at 1e-5; emitted rows: the pre-quantization row (the
    same step run with is_attn = 0 on a second state) at 2e-3 x RMS, and for the
    attention compressor the FP8 row via check_fp8_emit (bit-exact up to
    counted rounding-midpoint flips)."""
    from fp8_check import check_fp8_emit
    in_dim = 4096
    coff = 2 if ratio == 4 else 1
    width = coff * hd
    f16 = lambda a: np.ascontiguousarray(a.astype(np.float16).view(np.uint16))
    wkv = f16(synth.normal(8, 1, width * in_dim).reshape(width, in_dim) * 0.02)
    wg = f16(synth.normal(8, 2, width * in_dim).reshape(width, in_dim) * 0.02)
    ape = f16(synth.normal(8, 3, ratio * width).reshape(ratio, width) * 0.1)
    wn = (1 + 0.1 * synth.normal(8, 4, hd)).astype(np.float32)
    rows = coff * ratio
    skv = np.zeros((rows, width), np.float32)
    ssc = np.full((rows, width), -np.inf, np.float32)
    skv0, ssc0 = skv.copy(), ssc.copy()           # oracle, is_attn = 0 (pre-quantization rows)
    g_skv, g_ssc = t(skv, gpu), t(ssc, gpu)
    g_skv0, g_ssc0 = t(skv, gpu), t(ssc, gpu)
    g_wkv, g_wg, g_ape, g_wn = (t(wkv.view(np.int16), gpu), t(wg.view(np.int16), gpu),
                                t(ape.view(np.int16), gpu), t(wn, gpu))
    kv_cur = torch.empty(width, dtype=torch.float32, device=gpu)
    sc_cur = torch.empty(width, dtype=torch.float32, device=gpu)
    emit = torch.zeros(hd, dtype=torch.float32, device=gpu)
    emit0 = torch.zeros(hd, dtype=torch.float32, device=gpu)
    n_steps = ratio + ratio // 2 + 2 if ratio == 4 else ratio + 3
    worst, flips, n_emit = 0.0, 0, 0
    for pos in range(n_steps):
        x = synth.normal(9, pos, in_dim)
        ref_emit = np.zeros(hd, np.float32)
        ref_pre = np.zeros(hd, np.float32)
        r_ref = O.lib().orc_compressor_step(C.c_int(is_attn), P(x), P(wkv), P(wg), P(ape), P(wn),
                                            C.c_int(in_dim), C.c_int(hd), C.c_int(ratio),
                                            C.c_int(pos), C.c_int(il), P(skv), P(ssc),
                                            P(ref_emit))
        O.lib().orc_compressor_step(C.c_int(0), P(x), P(wkv), P(wg), P(ape), P(wn),
                                    C.c_int(in_dim), C.c_int(hd), C.c_int(ratio), C.c_int(pos),
                                    C.c_int(il), P(skv0), P(ssc0), P(ref_pre))
        xg = t(x, gpu)
        r = ops.launch_compressor_decode_step_f32_prealloc(is_attn, xg, g_wkv, g_wg, g_ape,
                                                           g_wn, in_dim, hd, ratio, pos, il, g_skv,
                                                           g_ssc, emit, kv_cur, sc_cur)
        r0 = ops.launch_compressor_decode_step_f32_prealloc(0, xg, g_wkv, g_wg, g_ape, g_wn,
                                                            in_dim, hd, ratio, pos, il, g_skv0,
                                                            g_ssc0, emit0, kv_cur, sc_cur)
        torch.cuda.synchronize()
        assert r == r_ref == r0
        close(g_skv.cpu().numpy(), skv, 1e-5)
        got_sc = g_ssc.cpu().numpy()
        fin = np.isfinite(ssc)
        assert np.array_equal(np.isfinite(got_sc), fin)
        close(got_sc[fin], ssc[fin], 1e-5)
        if r:
            n_emit += 1
            if is_attn:
                e, f = check_fp8_emit(emit.cpu().numpy(), emit0.cpu().numpy(), ref_emit, ref_pre)
                flips += f
            else:
                got = emit.cpu().numpy()
                close(got, ref_emit, 2e-3)
                e = float(np.abs(got - ref_emit).max() / np.sqrt(np.mean(ref_emit.astype(np.float64) ** 2)))
            worst = max(worst, e)
    assert n_emit >= 1
    print(f"compressor ratio {ratio} is_attn {is_attn}: {n_emit} emits, worst pre-quant "
          f"err/RMS {worst:.2e}, FP8 midpoint flips {flips}")


@pytest.mark.parametrize("il", [0, 2])
def test_fused_launches_equal_the_pairs(gpu, il):
    """The fused entry points against the launcher pairs they replace, bit for
    bit: the indexer query (f16 matvec + forward RoPE), the head weights
    (f16 matvec + scale) and Steps 14-16 (inverse RoPE + grouped and dense
    Q8_0 projections)."""
    from ds4cuda_amd import token
    g = torch.Generator(device=gpu)
    g.manual_seed(123 + il)
    pos = 300 + il
    # indexer query: 64 heads x 128 from 1024
    wq = token.f16_weights((64 * 128, 1024), g, gpu, 0.05)
    xq = torch.randn(1024, generator=g, device=gpu)
    a, b = torch.empty(64 * 128, device=gpu), torch.empty(64 * 128, device=gpu)
    ops.launch_mul_mv_f16_f32(wq, xq, a, 64 * 128, 1024)
    ops.launch_tail_rope_yarn_f32(a, a, 64, 128, 64, pos, il)
    ops.mul_mv_f16_rope_f32(wq, xq, b, 64, 128, 64, pos, il, 1024)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # head weights: 64 from 4096, scaled
    wp = token.f16_weights((64, 4096), g, gpu)
    x = torch.randn(4096, generator=g, device=gpu)
    a, b = torch.empty(64, device=gpu), torch.empty(64, device=gpu)
    sc = 1.0 / np.sqrt(128 * 64)
    ops.launch_mul_mv_f16_f32(wp, x, a, 64, 4096)
    ops.launch_scale_inplace_f32(a, 64, sc)
    ops.mul_mv_f16_scaled_f32(wp, x, b, 64, 4096, sc)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # Steps 14-16
    wa = token.q8_weights(8 * 1024, 4096, g, gpu)
    wb = token.q8_weights(4096, 8 * 1024, g, gpu)
    kqv = torch.randn(64 * 512, generator=g, device=gpu)
    back = torch.empty(64 * 512, device=gpu)
    low = torch.empty(8 * 1024, device=gpu)
    sq = torch.empty(64 * 512, dtype=torch.int8, device=gpu)
    ss = torch.empty(64 * 512 // 32, device=gpu)
    ref = torch.empty(4096, device=gpu)
    ops.launch_tail_rope_yarn_inverse_f32(kqv, back, 64, 512, 64, pos, il)
    ops.launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(wa, back, low, 8, 4096, 1024, sq, ss)
    ops.launch_mul_mv_q8_0_q8_0_f32_prealloc(wb, low, ref, 4096, 8 * 1024, sq, ss)
    out = torch.empty(4096, device=gpu)
    ops.attn_out_decode_f32(kqv, wa, wb, out, 64, 512, 64, pos, il, 8, 1024, 4096)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("n_rows,il", [(200, 0), (5000, 2), (3000, 3)])
def test_decode_merge_rope_q8_output(gpu, n_rows, il):
    """The decode merge's rotated Q8_0 output (decode_opts rope_q8) against
    the fp32 merge output rotated by the inverse tail RoPE launcher and
    quantized by the grouped Q8_0 launcher: int8 values and scales bit for
    bit, and Steps 15-16 from it (attn_out_decode_q8_f32) equal to
    attn_out_decode_f32 from the fp32 output. 200 rows take the narrow merge,
    3000 and 5000 the wide one; layers 0, 2, 3 cover the three RoPE
    parameter sets."""
    from ds4cuda_amd import synth, token
    g = torch.Generator(device=gpu)
    g.manual_seed(77 + il)
    pos = 4000 + il
    x = synth.kv_rows(78 + il, 1, n_rows)
    cache = ops.Fp8KVCache.empty(n_rows, device=gpu)
    cache.append(torch.from_numpy(x).to(gpu))
    q = torch.randn((1, 64, 512), generator=g, device=gpu) * 2.0
    sinks = torch.randn((1, 64), generator=g, device=gpu)
    kqv = torch.empty((1, 64, 512), device=gpu)
    ops.flash_attn_decode_fp8(q, sinks, kqv, cache, [n_rows])
    xq = torch.empty(64 * 512, dtype=torch.int8, device=gpu)
    xs = torch.empty(64 * 512 // 32, device=gpu)
    ops.flash_attn_decode_fp8(q, sinks, torch.empty_like(kqv), cache, [n_rows], rope_q8=(xq, xs, pos, il))
    back = torch.empty(64 * 512, device=gpu)
    ops.launch_tail_rope_yarn_inverse_f32(kqv.reshape(-1), back, 64, 512, 64, pos, il)
    wa = token.q8_weights(8 * 1024, 4096, g, gpu)
    wb = token.q8_weights(4096, 8 * 1024, g, gpu)
    low = torch.empty(8 * 1024, device=gpu)
    sq = torch.empty(64 * 512, dtype=torch.int8, device=gpu)
    ss = torch.empty(64 * 512 // 32, device=gpu)
    ops.launch_mul_mv_q8_0_q8_0_grouped_f32_prealloc(wa, back, low, 8, 4096, 1024, sq, ss)
    ref = torch.empty(4096, device=gpu)
    ops.attn_out_decode_f32(kqv.reshape(-1), wa, wb, ref, 64, 512, 64, pos, il, 8, 1024, 4096)
    got = torch.empty(4096, device=gpu)
    ops.attn_out_decode_q8_f32(xq, xs, wa, wb, got, 64, 512, 8, 1024, 4096)
    torch.cuda.synchronize()
    assert torch.equal(xq, sq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), ss.cpu().numpy().view(np.uint32))
    assert torch.isfinite(ref).all()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("counts", [[200, 50, 130], [3000, 700, 4000]])
def test_decode_merge_rope_f32_output(gpu, counts):
    """The decode merge's rotated fp32 output (decode_opts rope_out: per
    problem positions from a device array) against the fp32 merge output
    rotated by the batched inverse tail RoPE launcher, bit for bit; the first
    counts take the narrow merge, the second the wide one."""
    from ds4cuda_amd import synth
    n, il = len(counts), 2
    total = int(sum(counts))
    x = synth.kv_rows(91, 1, total)
    cache = ops.Fp8KVCache.empty(total, device=gpu)
    cache.append(torch.from_numpy(x).to(gpu))
    base = torch.tensor(np.concatenate([[0], np.cumsum(counts)[:-1]]), dtype=torch.int64, device=gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(92)
    q = torch.randn((n, 64, 512), generator=g, device=gpu).to(torch.bfloat16)
    sinks = torch.randn((n, 64), generator=g, device=gpu)
    pos = torch.tensor([4000, 17, 65000][:n], dtype=torch.int32, device=gpu)
    ref = torch.empty((n, 64, 512), device=gpu)
    ops.flash_attn_decode_fp8(q, sinks, ref, cache, counts, row_base=base)
    ops.tail_rope_yarn_batch_f32(ref, ref, n, 64, 512, 64, pos, il, inverse=True)
    got = torch.empty((n, 64, 512), device=gpu)
    ops.flash_attn_decode_fp8(q, sinks, got, cache, counts, row_base=base, rope_out=(pos, il))
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.cpu().numpy().view(np.uint32))
