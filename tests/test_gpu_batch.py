"""Batched forms used by the batched-decode attention block: fp32 projection,
per-sequence tail RoPE, compressor step for 16 sequences and the batched
sparse selection — each against the oracle run one sequence at a time."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from oracle import P
from ds4cuda_amd import ops, synth
from test_gpu_ops import close, t
from test_oracle_misc import rope

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_rows,n_cols,nb", [(1024, 4096, 16), (256, 4096, 3), (100, 64, 1), (4096, 32768, 16)])
def test_mul_mm_f32(gpu, n_rows, n_cols, nb):
    W = synth.normal(51, 1, n_rows * n_cols).reshape(n_rows, n_cols) * 0.02
    X = synth.normal(51, 2, nb * n_cols).reshape(nb, n_cols)
    Y = torch.full((nb, n_rows), 7.0, device=gpu)
    ops.mul_mm_f32_f32(t(W, gpu), t(X, gpu), Y, n_rows, n_cols, nb)
    torch.cuda.synchronize()
    close(Y.cpu().numpy(), X.astype(np.float64) @ W.astype(np.float64).T, 1e-5)


@pytest.mark.parametrize("n_rows,n_cols,nb", [(100, 64, 1), (256, 4096, 3), (300, 2080, 5), (300, 2048, 7), (4096, 32768, 16)])
def test_mul_mm_bf16_shapes(gpu, n_rows, n_cols, nb):
    W = synth.to_bf16_bits(synth.normal(52, 1, n_rows * n_cols) * 0.02).reshape(n_rows, n_cols)
    X = synth.normal(52, 2, nb * n_cols).reshape(nb, n_cols)
    Y = torch.full((nb, n_rows), 7.0, device=gpu)
    ops.mul_mm_bf16_f32(t(W.view(np.int16), gpu).view(torch.bfloat16), t(X, gpu), Y, n_rows, n_cols, nb)
    torch.cuda.synchronize()
    ref = X.astype(np.float64) @ synth.bf16_bits_to_f32(W).astype(np.float64).T
    close(Y.cpu().numpy(), ref, 1e-4)


def test_mul_mm_deterministic(gpu):
    """The split-K partials are added in a fixed order: repeated runs of the
    batched projections (attn_out shape, bf16; compressor shape, fp32) are
    bit-identical."""
    W = t(synth.to_bf16_bits(synth.normal(56, 1, 4096 * 32768) * 0.02).view(np.int16),
          gpu).view(torch.bfloat16).reshape(4096, 32768)
    X = t(synth.normal(56, 2, 16 * 32768), gpu)
    Wf = t(synth.normal(56, 3, 1024 * 4096) * 0.02, gpu)
    Xf = t(synth.normal(56, 4, 16 * 4096), gpu)
    ys, yf = [], []
    for _ in range(3):
        Y = torch.empty((16, 4096), device=gpu)
        ops.mul_mm_bf16_f32(W, X, Y, 4096, 32768, 16)
        Yf = torch.empty((16, 1024), device=gpu)
        ops.mul_mm_f32_f32(Wf, Xf, Yf, 1024, 4096, 16)
        torch.cuda.synchronize()
        ys.append(Y.cpu().numpy())
        yf.append(Yf.cpu().numpy())
    assert all(np.array_equal(ys[0].view(np.uint32), y.view(np.uint32)) for y in ys[1:])
    assert all(np.array_equal(yf[0].view(np.uint32), y.view(np.uint32)) for y in yf[1:])


def test_rope_batch_inverse(gpu):
    n_seq, n_heads = 5, 64
    pos = np.array([3, 1000, 16383, 0, 77], np.int32)
    x = synth.normal(52, 1, n_seq * n_heads * 512).reshape(n_seq, n_heads, 512)
    xt = t(x, gpu)
    ops.tail_rope_yarn_batch_f32(xt, xt, n_seq, n_heads, 512, 64, t(pos, gpu), 2, inverse=True)
    torch.cuda.synchronize()
    got = xt.cpu().numpy()
    for b in range(n_seq):
        close(got[b], rope(x[b], int(pos[b]), 2, inverse=True), 1e-5)


def test_compressor_batch_matches_per_sequence(gpu):
    """Batched fp32-weight compressor against the oracle one sequence at a
    time: state at 1e-5; emitted rows through check_fp8_emit (pre-quantization
    row from the same batch run with is_attn = 0 at 2e-3 x RMS, FP8 row
    bit-exact up to counted midpoint flips)."""
    from fp8_check import check_fp8_emit
    n_seq, in_dim, hd, ratio, il = 16, 4096, 512, 4, 2
    width = 2 * hd
    rows = 2 * ratio
    wkv = (synth.normal(53, 1, width * in_dim) * 0.02).reshape(width, in_dim)
    wg = (synth.normal(53, 2, width * in_dim) * 0.02).reshape(width, in_dim)
    ape = np.ascontiguousarray((synth.normal(53, 3, ratio * width) * 0.1).astype(np.float16)
                               .view(np.uint16).reshape(ratio, width))
    wn = (1 + 0.1 * synth.normal(53, 4, hd)).astype(np.float32)
    stride = rows * width
    skv = np.zeros((n_seq, rows, width), np.float32)
    ssc = np.full((n_seq, rows, width), -np.inf, np.float32)
    skv0, ssc0 = skv.copy(), ssc.copy()
    g_kv, g_sc = t(skv, gpu), t(ssc, gpu)
    g_kv0, g_sc0 = t(skv, gpu), t(ssc, gpu)
    g_wkv, g_wg, g_ape, g_wn = t(wkv, gpu), t(wg, gpu), t(ape.view(np.int16), gpu), t(wn, gpu)
    emit = torch.zeros((n_seq, hd), device=gpu)
    emit0 = torch.zeros((n_seq, hd), device=gpu)
    scratch = ops.compressor_batch_scratch(n_seq, in_dim, hd, ratio, gpu)
    start = np.arange(n_seq) * 3 + 1          # sequences at different phases of the window
    worst, flips, n_emit = 0.0, 0, 0
    for step in range(6):
        pos = (start + step).astype(np.int32)
        x = synth.normal(54, step, n_seq * in_dim).reshape(n_seq, in_dim)
        xg, pg = t(x, gpu), t(pos, gpu)
        flags = ops.compressor_decode_step_batch_w32(
            True, xg, g_wkv, g_wg, g_ape, g_wn, in_dim, hd, ratio, pos, pg, il,
            g_kv, g_sc, stride, emit, scratch)
        flags0 = ops.compressor_decode_step_batch_w32(
            False, xg, g_wkv, g_wg, g_ape, g_wn, in_dim, hd, ratio, pos, pg, il,
            g_kv0, g_sc0, stride, emit0, scratch)
        torch.cuda.synchronize()
        got_e = emit.cpu().numpy()
        got_e0 = emit0.cpu().numpy()
        for b in range(n_seq):
            ref_e = np.zeros(hd, np.float32)
            ref_p = np.zeros(hd, np.float32)
            r = O.lib().orc_compressor_step_w32(
                C.c_int(1), P(x[b]), P(wkv), P(wg), P(ape), P(wn), C.c_int(in_dim), C.c_int(hd),
                C.c_int(ratio), C.c_int(int(pos[b])), C.c_int(il), P(skv[b]), P(ssc[b]),
                P(ref_e))
            O.lib().orc_compressor_step_w32(
                C.c_int(0), P(x[b]), P(wkv), P(wg), P(ape), P(wn), C.c_int(in_dim), C.c_int(hd),
                C.c_int(ratio), C.c_int(int(pos[b])), C.c_int(il), P(skv0[b]), P(ssc0[b]),
                P(ref_p))
            assert flags[b] == r == flags0[b]
            if r:
                n_emit += 1
                e, f = check_fp8_emit(got_e[b], got_e0[b], ref_e, ref_p)
                worst, flips = max(worst, e), flips + f
        close(g_kv.cpu().numpy(), skv, 1e-5)
        fin = np.isfinite(ssc)
        got_sc = g_sc.cpu().numpy()
        assert np.array_equal(np.isfinite(got_sc), fin)
        close(got_sc[fin], ssc[fin], 1e-5)
    assert n_emit >= 16
    print(f"batched compressor: {n_emit} emits, worst pre-quant err/RMS {worst:.2e}, "
          f"FP8 midpoint flips {flips}")


@pytest.mark.parametrize("sizes", ["few", "many"])
@pytest.mark.parametrize("key_kind", [0, 1, 2])
def test_indexer_batch_positions(gpu, key_kind, sizes):
    """Batched scorer + selection for fp32 (0), f16 (1) and bf16 (2) keys:
    scores and positions bit-exact against the oracle per sequence. few: up
    to 10240 keys scored in all (the lane-per-head scorer); many: more (the
    four-lane scorer)."""
    n_comp = [100, 512, 513, 2000, 4000, 3] + ([5000, 700] if sizes == "many" else [])
    n_seq, top_k, recent = len(n_comp), 512, 64
    row0 = np.concatenate([[0], np.cumsum(n_comp)[:-1]]) + 10
    n_rows = int(row0[-1] + n_comp[-1])
    kf = synth.normal(55, 1, n_rows * 128).reshape(n_rows, 128)
    if key_kind == 0:
        keys, tdt = np.ascontiguousarray(kf), torch.float32
    elif key_kind == 1:
        keys, tdt = np.ascontiguousarray(kf.astype(np.float16).view(np.uint16)), torch.float16
    else:
        keys, tdt = synth.to_bf16_bits(kf).reshape(n_rows, 128), torch.bfloat16
    keys[row0[3] + 200: row0[3] + 260] = keys[row0[3] + 5]       # tied scores
    q = synth.normal(55, 2, n_seq * 64 * 128).reshape(n_seq, 64, 128)
    w = synth.normal(55, 3, n_seq * 64).reshape(n_seq, 64) / np.float32(np.sqrt(128 * 64))
    scores = torch.zeros(n_rows, device=gpu)
    pos = torch.full((n_seq, top_k + 7), -1, dtype=torch.int32, device=gpu)
    gk = t(keys, gpu) if key_kind == 0 else t(keys.view(np.int16), gpu).view(tdt)
    ops.indexer_topk_positions_batch(t(q, gpu), t(w, gpu), gk, row0, n_comp, top_k, recent,
                                     scores, pos)
    torch.cuda.synchronize()
    got = pos.cpu().numpy()
    for s in range(n_seq):
        n = n_comp[s]
        if n <= top_k:
            assert np.array_equal(got[s, :n], np.arange(n))
            continue
        ks = np.ascontiguousarray(keys[row0[s]:row0[s] + n])
        sc = np.zeros(n, np.float32)
        O.lib().orc_indexer_scores(P(q[s]), P(w[s]), P(ks), C.c_int(key_kind), C.c_int(n),
                                   C.c_int(64), C.c_int(128), P(sc))
        assert np.array_equal(scores.cpu().numpy()[row0[s]:row0[s] + n].view(np.uint32),
                              sc.view(np.uint32))
        ref = np.zeros(top_k, np.int32)
        O.lib().orc_topk_positions(P(sc), C.c_int(n), C.c_int(top_k), C.c_int(recent), P(ref))
        assert np.array_equal(got[s, :top_k], ref), s


@pytest.mark.parametrize("case", ["levels", "zero_ties", "all_equal", "recent_only"])
def test_indexer_batch_select_edges(gpu, case):
    """The batched selection (one workgroup per sequence, keys in LDS) at the
    boundaries of its keys-per-thread count (1 to 9 candidates per thread),
    with designed scores: one head, q = e_0, w = 1 and fp32 keys
    give score = relu(key[0]) exactly. levels: ~20 score levels (ties
    everywhere); zero_ties: most keys relu to 0 and the selection reaches into
    them; all_equal: every key ties; recent_only: the recent window is the
    whole top-k (nothing selected). Positions bit-exact against the oracle's
    (score desc, index asc) rule."""
    top_k, recent = 512, 512 if case == "recent_only" else 64
    # n = 513 .. 9064: 449, 1024, 1025, 2048, 2049, 4096, 4097 and 9000 candidates
    n_comp = [513, 1088, 1089, 2112, 2113, 4160, 4161, 9064]
    n_seq = len(n_comp)
    row0 = np.concatenate([[0], np.cumsum(n_comp)[:-1]]) + 3
    n_rows = int(row0[-1] + n_comp[-1])
    rng = np.random.default_rng(23)
    k = rng.standard_normal((n_rows, 128)).astype(np.float32)
    if case in ("levels", "recent_only"):
        k[:, 0] = np.round(rng.standard_normal(n_rows) * 4) / 4
    elif case == "zero_ties":
        k[:, 0] = rng.standard_normal(n_rows) - 1.5
    else:
        k[:, 0] = 0.5
    q = np.zeros((n_seq, 1, 128), np.float32)
    q[:, 0, 0] = 1.0
    w = np.ones((n_seq, 1), np.float32)
    scores = torch.zeros(n_rows, device=gpu)
    pos = torch.full((n_seq, top_k), -1, dtype=torch.int32, device=gpu)
    ops.indexer_topk_positions_batch(t(q, gpu), t(w, gpu), t(k, gpu), row0, n_comp, top_k, recent,
                                     scores, pos)
    torch.cuda.synchronize()
    got = pos.cpu().numpy()
    for s in range(n_seq):
        n = n_comp[s]
        sc = np.maximum(k[row0[s]:row0[s] + n, 0], 0).astype(np.float32)
        assert np.array_equal(scores.cpu().numpy()[row0[s]:row0[s] + n], sc)
        ref = np.zeros(top_k, np.int32)
        O.lib().orc_topk_positions(P(sc), C.c_int(n), C.c_int(top_k), C.c_int(recent), P(ref))
        assert np.array_equal(got[s], ref), (s, n)
