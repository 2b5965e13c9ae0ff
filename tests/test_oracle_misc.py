"""Pins the oracle's RoPE, Q8_0 matvecs, indexer and compressor (oracle/misc.cpp,
oracle/indexer.cpp) against closed forms, fp64 brute force and invariants."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from oracle import P


def rope(x, pos, il, inverse=False, n_rot=64):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    O.lib().orc_rope_tail(P(x), P(out), C.c_int(x.shape[0]), C.c_int(x.shape[1]), C.c_int(n_rot),
                          C.c_int(pos), C.c_int(il), C.c_int(int(inverse)))
    return out


def test_rope_pos0_identity_and_inverse():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    for il in (0, 1, 2, 3, 10):
        assert np.allclose(rope(x, 0, il), x, atol=1e-6)
        y = rope(x, 12345, il)
        assert np.array_equal(y[:, :448], x[:, :448])
        back = rope(y, 12345, il, inverse=True)
        assert np.allclose(back, x, atol=2e-4)


def test_rope_closed_form_uncompressed_layer():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    pos = 77
    y = rope(x, pos, 0)
    k = np.arange(32)
    theta = pos * 10000.0 ** (-2.0 * k / 64)
    t = x[:, 448:].astype(np.float64)
    c, s = np.cos(theta), np.sin(theta)
    ref0 = t[:, 0::2] * c - t[:, 1::2] * s
    ref1 = t[:, 0::2] * s + t[:, 1::2] * c
    assert np.allclose(y[:, 448::2], ref0, atol=1e-4)
    assert np.allclose(y[:, 449::2], ref1, atol=1e-4)


def q8_pack(w):
    """fp32 [rows, cols] -> block_q8_0 bytes (f16 d = amax/127, int8 rint(w/d))."""
    rows, cols = w.shape
    blocks = w.reshape(rows, cols // 32, 32)
    d = (np.abs(blocks).max(axis=2) / 127.0).astype(np.float16)
    df = d.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(df[..., None] > 0, np.rint(blocks / df[..., None]), 0)
    q = np.clip(q, -128, 127).astype(np.int8)
    out = np.zeros((rows, cols // 32, 34), np.uint8)
    out[..., :2] = d.view(np.uint8).reshape(rows, cols // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(rows, -1), df, q


def test_q8_activation_quantization_rounding():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(256).astype(np.float32)
    x[:32] = 0.0
    x[40] = 127.5 * (np.abs(x[32:64]).max() / 127.0)
    xq = np.zeros(256, np.int8)
    xs = np.zeros(8, np.float32)
    O.lib().orc_q8_quantize_act(P(x), C.c_int(256), P(xq), P(xs))
    blocks = x.reshape(8, 32)
    d = np.abs(blocks).max(axis=1) / np.float32(127.0)
    assert np.array_equal(xs, d.astype(np.float32))
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1.0) / d.astype(np.float32), 0).astype(np.float32)
    ref = np.clip(np.rint(blocks * idv[:, None]), -128, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(xq, ref)
    assert (xq[:32] == 0).all()


def test_q8_grouped_matvec_brute_force():
    rng = np.random.default_rng(3)
    n_groups, group_dim, rank = 4, 256, 8
    w = rng.standard_normal((n_groups * rank, group_dim)).astype(np.float32)
    Wb, dw, qw = q8_pack(w)
    x = rng.standard_normal(n_groups * group_dim).astype(np.float32)
    y = np.zeros(n_groups * rank, np.float32)
    O.lib().orc_q8_grouped_matvec(P(np.ascontiguousarray(Wb)), P(x), P(y), C.c_int(n_groups),
                                  C.c_int(group_dim), C.c_int(rank))
    xq = np.zeros_like(x, dtype=np.int8)
    xs = np.zeros(x.size // 32, np.float32)
    O.lib().orc_q8_quantize_act(P(x), C.c_int(x.size), P(xq), P(xs))
    wd = (qw.astype(np.float64) * dw[..., None]).reshape(n_groups * rank, group_dim)
    xd = (xq.astype(np.float64).reshape(-1, 32) * xs[:, None]).reshape(-1)
    ref = np.array([wd[r] @ xd[(r // rank) * group_dim:(r // rank + 1) * group_dim]
                    for r in range(n_groups * rank)])
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
    # and close to the unquantized product
    exact = np.array([w[r] @ x[(r // rank) * group_dim:(r // rank + 1) * group_dim]
                      for r in range(n_groups * rank)])
    assert np.abs(y - exact).max() < 0.05 * np.abs(exact).max()


def test_q8_dense_matvec_brute_force():
    """orc_q8_matvec (cuda/dense_q8.cu, Step 16) against an fp64 product of
    the dequantized weights and activations built here from the block bytes:
    rows are independent (row r reads only W row r), each block's f16 scale
    multiplies its own 32 int8 values, the activation is quantized per 32."""
    rng = np.random.default_rng(31)
    n_rows, n_cols = 24, 512
    w = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
    w[3, 64:96] = 0.0                       # an all-zero weight block (d = 0)
    Wb, dw, qw = q8_pack(w)
    x = rng.standard_normal(n_cols).astype(np.float32)
    x[128:160] *= 1e-3                      # a block of small activations (own scale)
    y = np.zeros(n_rows, np.float32)
    O.lib().orc_q8_matvec(P(np.ascontiguousarray(Wb)), P(x), P(y), C.c_int(n_rows), C.c_int(n_cols))
    # activation quantization restated (d = amax / 127 in fp32, rint(x / d))
    xb = x.reshape(-1, 32)
    xd = (np.abs(xb).max(axis=1) / np.float32(127.0)).astype(np.float32)
    xq = np.clip(np.rint(xb * (np.float32(1.0) / xd)[:, None]), -128, 127)
    # per block: f16(d_w) * d_x as an fp32 product, times the exact int32 dot
    ref = np.zeros(n_rows)
    for r in range(n_rows):
        blk = Wb[r].reshape(-1, 34)
        dwb = blk[:, :2].copy().view(np.float16).reshape(-1).astype(np.float32)
        qwb = blk[:, 2:].view(np.int8).astype(np.int64)
        dots = (qwb * xq.astype(np.int64)).sum(axis=1)
        ref[r] = ((dwb * xd).astype(np.float64) * dots).sum()
    assert np.max(np.abs(y - ref)) <= 1e-6 * np.abs(ref).max()
    # a transposed or mis-scaled reading fails this: compare with the exact product
    exact = w.astype(np.float64) @ x.astype(np.float64)
    assert np.abs(y - exact).max() < 0.02 * np.abs(exact).max()
    # one-hot activation: y = the dequantized weight column (up to the activation scale)
    e = np.zeros(n_cols, np.float32)
    e[77] = 1.0
    O.lib().orc_q8_matvec(P(np.ascontiguousarray(Wb)), P(e), P(y), C.c_int(n_rows), C.c_int(n_cols))
    # block 2 of x: d = 1/127, xq[77] = 127, every other block d = 0
    dd = (dw[:, 2].astype(np.float32) * np.float32(1.0 / 127.0)).astype(np.float64)
    col = qw.reshape(n_rows, -1)[:, 77].astype(np.float64) * 127 * dd
    assert np.array_equal(y, col.astype(np.float32))


def test_bf16_matvec_brute_force():
    """orc_bf16_matvec (the cfg 5 attn_out checker) against an fp64 product of
    the bf16 weights decoded by torch and against hand-made rows."""
    import torch
    rng = np.random.default_rng(32)
    n_rows, n_cols = 16, 300
    wf = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
    wb = torch.from_numpy(wf).to(torch.bfloat16)
    bits = np.ascontiguousarray(wb.view(torch.int16).numpy().view(np.uint16))
    x = rng.standard_normal(n_cols).astype(np.float32)
    y = np.zeros(n_rows, np.float32)
    O.lib().orc_bf16_matvec(P(bits), P(x), P(y), C.c_int(n_rows), C.c_int(n_cols))
    ref = wb.to(torch.float64).numpy() @ x.astype(np.float64)
    assert np.array_equal(y, ref.astype(np.float32))   # fp64 sum, one rounding
    # row r = e_r (the identity) selects x[r]; a transposed W would not
    eye = torch.eye(n_rows, n_cols, dtype=torch.bfloat16)
    ib = np.ascontiguousarray(eye.view(torch.int16).numpy().view(np.uint16))
    O.lib().orc_bf16_matvec(P(ib), P(x), P(y), C.c_int(n_rows), C.c_int(n_cols))
    assert np.array_equal(y, x[:n_rows])


def test_indexer_scores_and_selection():
    rng = np.random.default_rng(4)
    n_head, hd, n = 8, 128, 500
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    w = rng.standard_normal(n_head).astype(np.float32)
    k = rng.standard_normal((n, hd)).astype(np.float32)
    s = np.zeros(n, np.float32)
    O.lib().orc_indexer_scores(P(q), P(w), P(k), C.c_int(0), C.c_int(n), C.c_int(n_head),
                               C.c_int(hd), P(s))
    ref = (np.maximum(k.astype(np.float64) @ q.T.astype(np.float64), 0) * w).sum(axis=1)
    assert np.allclose(s, ref, rtol=1e-4, atol=1e-3)
    # planted ties: lowest index wins
    s2 = s.copy()
    s2[[10, 20, 30]] = 1e9
    s2[[5, 7]] = s2[np.argsort(-s2)[3]]
    for top_k in (1, 3, 4, 64, 499, 500, 600):
        m = np.zeros(n, np.int32)
        O.lib().orc_topk_mask(P(s2), C.c_int(n), C.c_int(top_k), P(m))
        order = np.lexsort((np.arange(n), -s2.astype(np.float64)))
        ref = np.zeros(n, np.int32)
        ref[order[:min(top_k, n)]] = 1
        assert np.array_equal(m, ref), top_k
    pos = np.zeros(64, np.int32)
    cnt = O.lib().orc_topk_positions(P(s2), C.c_int(n), C.c_int(64), C.c_int(16), P(pos))
    old = np.lexsort((np.arange(n - 16), -s2[:n - 16].astype(np.float64)))[:48]
    assert cnt == 64 and np.array_equal(pos, np.sort(np.concatenate([old, np.arange(n - 16, n)])))


def comp_step(is_attn, x, wkv, wg, ape, wn, in_dim, hd, ratio, pos, il, skv, ssc):
    emit = np.zeros(hd, np.float32)
    r = O.lib().orc_compressor_step(C.c_int(is_attn), P(x), P(wkv), P(wg), P(ape), P(wn),
                                    C.c_int(in_dim), C.c_int(hd), C.c_int(ratio), C.c_int(pos),
                                    C.c_int(il), P(skv), P(ssc), P(emit))
    return r, emit


@pytest.mark.parametrize("ratio", [4, 128])
def test_compressor_invariants(ratio):
    rng = np.random.default_rng(5)
    in_dim, hd = 256, 128
    coff = 2 if ratio == 4 else 1
    width = coff * hd
    f16 = lambda a: np.ascontiguousarray(a.astype(np.float16).view(np.uint16))
    wkv = f16(rng.standard_normal((width, in_dim)) * 0.05)
    wg = f16(rng.standard_normal((width, in_dim)) * 0.05)
    ape = f16(np.zeros((ratio, width)))
    wn = np.ones(hd, np.float32)
    rows = coff * ratio
    skv = np.zeros((rows, width), np.float32)
    ssc = np.full((rows, width), -np.inf, np.float32)
    emits = []
    for pos in range(2 * ratio):
        x = rng.standard_normal(in_dim).astype(np.float32)
        before = skv.copy()
        r, e = comp_step(0, x, wkv, wg, ape, wn, in_dim, hd, ratio, pos, 0, skv, ssc)
        assert r == int((pos + 1) % ratio == 0)
        if not r:
            changed = np.nonzero((skv != before).any(axis=1))[0]
            assert len(changed) <= 1 and changed[0] == (ratio + pos % ratio if ratio == 4 else pos % ratio)
        else:
            emits.append(e)
            if ratio == 4:
                assert np.array_equal(skv[:4], skv[4:])      # ring shift duplicated the rows
            assert np.isclose(np.sqrt((e.astype(np.float64) ** 2).mean()), 1.0, rtol=1e-3)
    assert len(emits) == 2


def test_compressor_w32_matches_f16_on_f16_weights():
    # fp32 weights holding f16-representable values give the f16 step's result
    rng = np.random.default_rng(6)
    in_dim, hd, ratio = 256, 128, 4
    width = 2 * hd
    wkv16 = (rng.standard_normal((width, in_dim)) * 0.05).astype(np.float16)
    wg16 = (rng.standard_normal((width, in_dim)) * 0.05).astype(np.float16)
    ape = np.ascontiguousarray((rng.standard_normal((ratio, width)) * 0.1).astype(np.float16)
                               .view(np.uint16))
    wn = np.ones(hd, np.float32)
    st = [(np.zeros((2 * ratio, width), np.float32), np.full((2 * ratio, width), -np.inf, np.float32))
          for _ in range(2)]
    for pos in range(8):
        x = rng.standard_normal(in_dim).astype(np.float32)
        e16 = np.zeros(hd, np.float32)
        e32 = np.zeros(hd, np.float32)
        r16 = O.lib().orc_compressor_step(
            C.c_int(1), P(x), P(np.ascontiguousarray(wkv16.view(np.uint16))),
            P(np.ascontiguousarray(wg16.view(np.uint16))), P(ape), P(wn), C.c_int(in_dim),
            C.c_int(hd), C.c_int(ratio), C.c_int(pos), C.c_int(2), P(st[0][0]), P(st[0][1]), P(e16))
        r32 = O.lib().orc_compressor_step_w32(
            C.c_int(1), P(x), P(np.ascontiguousarray(wkv16.astype(np.float32))),
            P(np.ascontiguousarray(wg16.astype(np.float32))), P(ape), P(wn), C.c_int(in_dim),
            C.c_int(hd), C.c_int(ratio), C.c_int(pos), C.c_int(2), P(st[1][0]), P(st[1][1]), P(e32))
        assert r16 == r32
        assert np.array_equal(st[0][0], st[1][0]) and np.array_equal(st[0][1], st[1][1])
        assert np.array_equal(e16, e32)
