"""Pins for the oracle functions whose invariants alone leave room for a
plausible mistake: the compressor's softmax pool (which rows and which column
half each window slot contributes), the YaRN ramp of compressed layers, and the
causal chunked prefill. Each check is computed independently of the oracle's
code: planted scores that make the pool a plain mean or a copy of one known
row, the published YaRN mix evaluated in fp64 with hand-derived correction
dims, and the prefill as per-query decode plus fp64 softmax attention."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from oracle import P


# ---------------------------------------------------------------- compressor
OFF = -60000.0        # f16-representable; exp(OFF - 0) is 0 in fp32


def f16bits(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16).view(np.uint16))


def run_compressor(ratio, hd, ape, n_steps, is_attn=0, il=0, seed=0, in_dim=64):
    """Drives orc_compressor_step with a zero gate projection, so every score
    is exactly the APE entry of the slot. Returns (kv per step [n, width] in
    fp64, emits {pos: row})."""
    rng = np.random.default_rng(seed)
    coff = 2 if ratio == 4 else 1
    width = coff * hd
    wkv16 = (rng.standard_normal((width, in_dim)) * 0.2).astype(np.float16)
    wkv = np.ascontiguousarray(wkv16.view(np.uint16))
    wg = f16bits(np.zeros((width, in_dim)))
    ape_b = f16bits(ape)
    wn = (1.0 + 0.25 * rng.standard_normal(hd)).astype(np.float32)
    skv = np.zeros((coff * ratio, width), np.float32)
    ssc = np.full((coff * ratio, width), -np.inf, np.float32)
    kvs, emits = [], {}
    for pos in range(n_steps):
        x = rng.standard_normal(in_dim).astype(np.float32)
        kvs.append(wkv16.astype(np.float64) @ x.astype(np.float64))
        e = np.zeros(hd, np.float32)
        r = O.lib().orc_compressor_step(C.c_int(is_attn), P(x), P(wkv), P(wg), P(ape_b), P(wn),
                                        C.c_int(in_dim), C.c_int(hd), C.c_int(ratio),
                                        C.c_int(pos), C.c_int(il), P(skv), P(ssc), P(e))
        if r:
            emits[pos] = e
    return np.array(kvs), emits, wn


def rms_norm64(v, wn):
    return v / np.sqrt((v ** 2).mean() + 1e-6) * wn


def rope64_il0(v, pos, n_rot=64):
    """Forward tail RoPE of an uncompressed layer in fp64 (theta_k =
    pos * 10000^(-2k/n_rot))."""
    out = v.copy()
    n_nope = v.size - n_rot
    k = np.arange(n_rot // 2)
    th = pos * 10000.0 ** (-2.0 * k / n_rot)
    x0, x1 = v[n_nope::2].copy(), v[n_nope + 1::2].copy()
    out[n_nope::2] = x0 * np.cos(th) - x1 * np.sin(th)
    out[n_nope + 1::2] = x0 * np.sin(th) + x1 * np.cos(th)
    return out


def check_emit(got, pooled, wn, rope_pos, tol=2e-6):
    ref = rope64_il0(rms_norm64(pooled, wn), rope_pos)
    assert np.abs(got - ref).max() <= tol * np.abs(ref).max(), np.abs(got - ref).max()


def test_pool_equal_scores_is_the_mean():
    # ratio 4, all scores 0. The first window's emit (pos 3) sees rows 0..3 still
    # at -inf, so it is the mean of the second-half columns of pos 0..3; the
    # second (pos 7) is the mean of pos 0..3's first halves and pos 4..7's second
    # halves (8 equal weights).
    hd = 128
    kv, emits, wn = run_compressor(4, hd, np.zeros((4, 2 * hd)), 8)
    assert sorted(emits) == [3, 7]
    check_emit(emits[3], kv[0:4, hd:].mean(axis=0), wn, 0)
    check_emit(emits[7], (kv[0:4, :hd].sum(axis=0) + kv[4:8, hd:].sum(axis=0)) / 8.0, wn, 4)


def test_pool_ratio128_single_live_score_copies_that_row():
    hd, m0 = 64, 37
    ape = np.full((128, hd), OFF)
    ape[m0] = 0.0
    kv, emits, wn = run_compressor(128, hd, ape, 128)
    assert sorted(emits) == [127]
    check_emit(emits[127], kv[m0], wn, 0)


@pytest.mark.parametrize("slot,half", [(2, 0), (1, 1), (3, 0), (0, 1)])
def test_pool_ratio4_half_row_selection(slot, half):
    # One live (slot, column-half) in the APE table. Window rows 0..3 contribute
    # their first-half columns j, rows 4..7 their second-half columns hd + j.
    # At the emit of pos 7, rows 0..3 hold pos 0..3 (ring shift of the first
    # window) and rows 4..7 hold pos 4..7.
    hd = 128
    ape = np.full((4, 2 * hd), OFF)
    ape[slot, half * hd:(half + 1) * hd] = 0.0
    kv, emits, wn = run_compressor(4, hd, ape, 8, seed=slot + 10 * half)
    src_pos = slot if half == 0 else 4 + slot
    check_emit(emits[7], kv[src_pos, half * hd:(half + 1) * hd], wn, 4)
    if half == 1:       # the first window reads only its second halves
        check_emit(emits[3], kv[slot, hd:], wn, 0)
    else:               # all first-window scores are OFF: equal weights, the mean
        check_emit(emits[3], kv[0:4, hd:].mean(axis=0), wn, 0)


def test_pool_attn_emit_is_fp8_round_trip_of_pooled_row():
    # is_attn = 1 adds the FP8 round trip of the normalized, rotated row; its
    # codes are order-free given the pre-quantization values.
    hd = 512
    kv, emits, wn = run_compressor(4, hd, np.zeros((4, 2 * hd)), 8, is_attn=1, seed=3)
    _, emits0, _ = run_compressor(4, hd, np.zeros((4, 2 * hd)), 8, is_attn=0, seed=3)
    for pos in (3, 7):
        _, _, _, deq = O.fp8_quant_rows(emits0[pos][None, :])
        assert np.array_equal(emits[pos], deq[0])


# ---------------------------------------------------------------- YaRN ramp
def rope_oracle(x, pos, il, inverse=False):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    O.lib().orc_rope_tail(P(x), P(out), C.c_int(x.shape[0]), C.c_int(x.shape[1]), C.c_int(64),
                          C.c_int(pos), C.c_int(il), C.c_int(int(inverse)))
    return out


def test_yarn_correction_dims_by_hand():
    # YaRN (Peng et al. 2023, "YaRN: Efficient Context Window Extension"),
    # correction dim for a rotation count b: n_rot * ln(L / (2 pi b)) / (2 ln base),
    # L = 65536 original context, base 160000 on compressed layers.
    n_rot, L, base = 64, 65536, 160000.0
    cd = lambda b: n_rot * np.log(L / (2 * np.pi * b)) / (2 * np.log(base))
    assert np.floor(cd(32.0)) == 15 and np.ceil(cd(1.0)) == 25


@pytest.mark.parametrize("il", [2, 3, 42])
@pytest.mark.parametrize("pos", [1, 7, 100])
def test_yarn_compressed_layer_fp64(il, pos):
    # Published YaRN "NTK-by-parts" mix with scale s = 16: pair k with
    # ramp r_k = 1 - clamp((k - 15) / (25 - 15), 0, 1) rotates by
    #   theta_k = (theta0_k / s) * (1 - r_k) + theta0_k * r_k,
    #   theta0_k = pos * base^(-2k / n_rot),
    # with magnitude scale mscale = 1: ds4 divides its attention factor by the
    # YaRN magnitude correction 1 + 0.1 ln(s), which cancels it.
    rng = np.random.default_rng(il * 1000 + pos)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    got = rope_oracle(x, pos, il)
    k = np.arange(32)
    theta0 = pos * 160000.0 ** (-2.0 * k / 64)
    ramp = 1.0 - np.clip((k - 15) / 10.0, 0.0, 1.0)
    theta = theta0 / 16.0 * (1 - ramp) + theta0 * ramp
    t = x[:, 448:].astype(np.float64)
    c, s = np.cos(theta), np.sin(theta)
    ref0 = t[:, 0::2] * c - t[:, 1::2] * s
    ref1 = t[:, 0::2] * s + t[:, 1::2] * c
    # fp32 running product: |d theta| <= 32 ulp * theta0 ~ 4e-6 * pos
    tol = 2e-5 + 8e-6 * pos
    assert np.abs(got[:, 448::2] - ref0).max() < tol
    assert np.abs(got[:, 449::2] - ref1).max() < tol
    assert np.array_equal(got[:, :448], x[:, :448])
    # the inverse is the rotation by -theta
    inv = rope_oracle(x, pos, il, inverse=True)
    assert np.abs(inv[:, 448::2] - (t[:, 0::2] * c + t[:, 1::2] * s)).max() < tol


# ---------------------------------------------------------------- prefill
def prefill_oracle(Q, codes, sexp, tail, n_cached, sinks):
    n_q, n_head, d = Q.shape
    out = np.zeros_like(Q)
    O.lib().orc_attn_prefill_fp8(P(np.ascontiguousarray(Q)), C.c_int(n_q), P(codes), P(sexp),
                                 P(tail), C.c_int(n_cached), P(sinks), P(out), C.c_int(n_head),
                                 C.c_int(d), C.c_int(64), C.c_int(1))
    return out


def test_prefill_query_equals_decode_over_its_causal_prefix():
    rng = np.random.default_rng(20)
    n_cached, n_q, H = 7, 5, 8
    x = (rng.standard_normal((n_cached + n_q, 512)) * 2).astype(np.float32)
    codes, sexp, tail, deq = O.fp8_quant_rows(x)
    Q = rng.standard_normal((n_q, H, 512)).astype(np.float32)
    sinks = rng.standard_normal(H).astype(np.float32)
    out = prefill_oracle(Q, codes, sexp, tail, n_cached, sinks)
    for t in range(n_q):
        dec = O.attn_decode_fp8(Q[t], codes, sexp, tail, np.arange(n_cached + t + 1), sinks)
        assert np.array_equal(out[t], dec), t
        # fp64 softmax attention with the sink as an extra key of value 0
        K = deq[:n_cached + t + 1].astype(np.float16).astype(np.float64)
        s = Q[t].astype(np.float64) @ K.T / np.sqrt(512)
        s = np.concatenate([s, sinks[:, None].astype(np.float64)], axis=1)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        ref = (w[:, :-1] @ K) / w.sum(axis=1, keepdims=True)
        assert np.abs(out[t] - ref).max() < 1e-5 * np.abs(ref).max()
    # causality: rows after a query's position do not change it
    codes2 = codes.copy()
    codes2[n_cached + 2:] ^= 0x05
    out2 = prefill_oracle(Q, codes2, sexp, tail, n_cached, sinks)
    assert np.array_equal(out2[:2], out[:2]) and not np.array_equal(out2[2:], out[2:])


def test_prefill_hand_case_two_rows_two_queries():
    # Rows: r0 = e_0 (one hot on dim 0), r1 = 2 e_1; every value is exactly
    # representable in FP8 and f16; r2 = 4 e_2. Scale 1/sqrt(512).
    # With n_cached = 1, query 0 sits at position 1 and sees rows 0 and 1;
    # query 1 (position 2) sees rows 0..2.
    d = 512
    x = np.zeros((3, d), np.float32)
    x[0, 0] = 1.0
    x[1, 1] = 2.0
    x[2, 2] = 4.0
    codes, sexp, tail, deq = O.fp8_quant_rows(x)
    assert np.array_equal(deq, x)
    Q = np.zeros((2, 1, d), np.float32)
    Q[0, 0, 0], Q[0, 0, 1] = 3.0, 1.0
    Q[1, 0, 2] = 2.0
    sink = np.array([0.5], np.float32)
    out = prefill_oracle(Q, codes, sexp, tail, 1, sink)
    c = 1.0 / np.sqrt(512.0)
    s0, s1 = 3.0 * c, 2.0 * c                       # query 0 logits for rows 0, 1
    e0, e1, es = np.exp(s0), np.exp(s1), np.exp(0.5)
    ref0 = np.zeros(d)
    ref0[0], ref0[1] = e0 / (e0 + e1 + es), 2.0 * e1 / (e0 + e1 + es)
    assert np.abs(out[0, 0] - ref0).max() < 1e-6
    t0, t1, t2 = 0.0, 0.0, 8.0 * c                  # query 1 logits for rows 0, 1, 2
    den = np.exp(t0) + np.exp(t1) + np.exp(t2) + es
    ref1 = np.zeros(d)
    ref1[0], ref1[1], ref1[2] = 1.0 / den, 2.0 / den, 4.0 * np.exp(t2) / den
    assert np.abs(out[1, 0] - ref1).max() < 1e-6
