"""Writes the committed golden fixtures of the attention path (DSST files plus
index.json) from the CPU oracle, after checking each case independently of
the oracle's code:

  fp8_rows    OCP E4M3FN codes / power-of-two block exponents / f16 tail of 16
              rows with planted special cases (all-zero block, rounding
              midpoints, tiny negatives, large magnitudes); checked against a
              numpy restatement of the quantization rule
              (cuda/fp8_kv.cuh:21-35, cuda/fp8_kv.cu:75-195) that searches the
              E4M3FN value set directly
  decode_fp8  one query (64 heads) over 64 FP8 rows with sinks
              (cuda/flash_attn.cuh:9-26); checked against fp64 softmax
              attention over the f16-rounded dequantized rows
  decode_mix  raw + masked compressed fp32 rows (cuda/flash_attn.cuh:90-117);
              checked in fp64
  indexer     ReLU-weighted scores of 300 bf16 keys with planted ties, the
              top-40 mask and the top-40 positions with the last 8 forced
              (cuda/indexer_allowed.cu:68-279); scores checked in fp64, the
              selections against a stable sort by (score desc, index asc)
  rope        forward tail RoPE for il 0 / 2 / 3 and the inverse for il 2 at
              position 70000 (cuda/rope.cu:114-259); checked: dims < 448
              untouched, rotation norms kept, inverse of forward
  rms_norm    one 4096 row with a weight (cuda/norm.cu:4-7); checked in fp64
  compressor  8 ratio-4 attention steps (two emits) and 8 indexer-compressor
              steps with fp32 weights (cuda/compressor.cu:64-349); the emitted
              rows and final states are recorded; 128 ratio-128 steps (one
              emit)
  prefill     2 queries over 40 cached rows + causal self (the chunked prefill
              the reference runs token by token); checked per query in fp64
  q8_grouped  Q8_0 x Q8_0 grouped matvec, 2 groups x rank 16
              (cuda/attn_out.cu:119-197); checked against exact int32 block
              sums scaled in fp64

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

import oracle as O                      # noqa: E402
from oracle import P                    # noqa: E402
from ds4cuda_amd import synth           # noqa: E402
import dsst                             # noqa: E402


def e4m3_values():
    """The 127 finite non-negative E4M3FN values, by code (OCP definition)."""
    v = []
    for c in range(127):
        e, m = c >> 3, c & 7
        v.append(m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(v)


def numpy_fp8_rows(x, n_rot=64):
    """Independent restatement: scale 2^ceil(log2(max(amax,1e-4)/448)), value
    x / scale clamped to +-448, nearest E4M3FN value with ties to the even
    code, sign kept (negative zero for tiny negatives)."""
    vals = e4m3_values()
    n, d = x.shape
    nope = d - n_rot
    codes = np.zeros((n, nope), np.uint8)
    sexp = np.zeros((n, 8), np.int8)
    for r in range(n):
        for b in range(nope // 64):
            blk = x[r, 64 * b:64 * b + 64].astype(np.float64)
            amax = max(np.abs(blk).max(), 1e-4)
            e = int(np.ceil(np.log2(amax / 448.0)))
            sexp[r, b] = e
            for i, xv in enumerate(blk):
                a = min(abs(xv) / 2.0 ** e, 448.0)
                k = int(np.searchsorted(vals, a))
                if k == 0:
                    c = 0
                elif k >= len(vals):
                    c = len(vals) - 1
                else:
                    lo, hi = vals[k - 1], vals[k]
                    c = k - 1 if a - lo < hi - a else k if a - lo > hi - a else (k - 1 if (k - 1) % 2 == 0 else k)
                codes[r, 64 * b + i] = c | (0x80 if np.signbit(xv) else 0)
    tail = x[:, nope:].astype(np.float16).view(np.uint16)
    return codes, sexp, tail


def rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.abs(np.asarray(a, np.float64) - b).max() / (np.sqrt(np.mean(b ** 2)) + 1e-300))


def attn64(Q, K, V, sinks, scale):
    out = np.zeros((Q.shape[0], V.shape[1]))
    for h in range(Q.shape[0]):
        s = K @ Q[h] * scale
        m = max(s.max() if len(s) else -np.inf, sinks[h])
        p = np.exp(s - m)
        out[h] = (p @ V) / (np.exp(sinks[h] - m) + p.sum())
    return out


def main():
    idx = {}

    def put(case, name, a, **meta):
        fn = f"{case}_{name}.bin"
        dsst.write(HERE / fn, a)
        idx.setdefault(case, {"tensors": {}, "params": {}})
        idx[case]["tensors"][name] = {"file": fn, "shape": list(np.shape(a)), "dtype": str(np.asarray(a).dtype)}
        idx[case]["params"].update(meta)

    # ---- fp8_rows
    x = synth.kv_rows(401, 0, 16, outlier_frac=0.2)
    x[1, :64] = 0.0                                        # all-zero block -> 2^-22
    mids = np.array([1.0625, -1.0625, 1.1875, 2.0 ** -10, 1.5 * 2 ** -9, -3 * 2 ** -10, 448.0, 440.0])
    x[2, :64] = np.resize(mids, 64)                        # amax 448 -> scale 1; midpoints
    x[3, 64:128] = -1e-30                                  # tiny negatives -> -0
    x[4, 128:192] *= 1e4                                   # large block
    x[5, 448:512] = np.resize([1.0 + 2 ** -11, 2049.0, 65504.0, -6.1e-5], 64)   # f16 tail midpoints
    x = x.astype(np.float32)
    codes, sexp, tail, deq = O.fp8_quant_rows(x)
    c2, s2, t2 = numpy_fp8_rows(x)
    assert np.array_equal(codes, c2) and np.array_equal(sexp, s2) and np.array_equal(tail, t2)
    put("fp8_rows", "x", x)
    put("fp8_rows", "codes", codes.astype(np.int32))
    put("fp8_rows", "sexp", sexp.astype(np.int32))
    put("fp8_rows", "tail", tail.view(np.float16))
    put("fp8_rows", "deq", deq, head_dim=512, n_rot=64)

    # ---- decode_fp8
    n_kv = 64
    src = synth.kv_rows(402, 0, n_kv, outlier_frac=0.05).astype(np.float32)
    c, s, t, dq = O.fp8_quant_rows(src)
    q = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(402, 1, 64 * 512))).reshape(64, 512)
    sinks = synth.normal(402, 2, 64).astype(np.float32)
    out = O.attn_decode_fp8(q, c, s, t, np.arange(n_kv), sinks)
    kv16 = dq.astype(np.float16).astype(np.float64)
    ref = attn64(q.astype(np.float64), kv16, kv16, sinks.astype(np.float64), 1 / np.sqrt(512))
    assert rel(out, ref) < 1e-5, rel(out, ref)
    put("decode_fp8", "kv_src", src)
    put("decode_fp8", "q", q)
    put("decode_fp8", "sinks", sinks)
    put("decode_fp8", "out", out, n_kv=n_kv, note="q holds bf16 values; rows are kv_src after the FP8 rule")

    # ---- decode_mix
    raw = synth.normal(403, 0, 24 * 512).reshape(24, 512).astype(np.float32)
    comp = (2 * synth.normal(403, 1, 20 * 512)).reshape(20, 512).astype(np.float32)
    allowed = (synth.uniform(403, 2, 20) < 0.6).astype(np.int32)
    qm = synth.normal(403, 3, 64 * 512).reshape(64, 512).astype(np.float32)
    sm = synth.normal(403, 4, 64).astype(np.float32)
    outm = O.attn_decode_mixed_f32(qm, raw, comp, allowed, sm)
    kv = np.concatenate([raw, comp[allowed == 1]]).astype(np.float16).astype(np.float64)
    refm = attn64(qm.astype(np.float64), kv, kv, sm.astype(np.float64), 1 / np.sqrt(512))
    assert rel(outm, refm) < 5e-5, rel(outm, refm)   # fp32 exp and sums
    put("decode_mix", "q", qm)
    put("decode_mix", "raw", raw)
    put("decode_mix", "comp", comp)
    put("decode_mix", "allowed", allowed)
    put("decode_mix", "sinks", sm)
    put("decode_mix", "out", outm)

    # ---- indexer
    n_comp, k, n_recent = 300, 40, 8
    keys = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(404, 0, n_comp * 128))).reshape(n_comp, 128)
    qi = synth.normal(404, 1, 64 * 128).reshape(64, 128).astype(np.float32)
    wi = (synth.normal(404, 2, 64) / np.sqrt(128 * 64)).astype(np.float32)

    def score_all(kk):
        sc = np.zeros(n_comp, np.float32)
        O.lib().orc_indexer_scores(P(qi), P(wi), P(np.ascontiguousarray(synth.to_bf16_bits(kk))), C.c_int(2),
                                   C.c_int(n_comp), C.c_int(64), C.c_int(128), P(sc))
        return sc
    # planted ties across the selection boundary: the key ranked 36th is
    # copied into positions 10..19, so 11 equal scores straddle rank 40
    s0 = score_all(keys)
    tie = int(np.argsort(-s0[20:], kind="stable")[35]) + 20
    keys[10:20] = keys[tie]
    kb = synth.to_bf16_bits(keys)
    scores = score_all(keys)
    s64 = (np.maximum(keys.astype(np.float64) @ qi.astype(np.float64).T, 0) * wi.astype(np.float64)).sum(1)
    assert np.abs(scores - s64).max() <= 1e-5 * np.abs(s64).max()
    assert len(set(scores[[tie] + list(range(10, 20))].tolist())) == 1   # the ties are exact
    mask = np.zeros(n_comp, np.int32)
    O.lib().orc_topk_mask(P(scores), C.c_int(n_comp), C.c_int(k), P(mask))
    order = sorted(range(n_comp), key=lambda i: (-float(scores[i]), i))
    assert set(np.flatnonzero(mask).tolist()) == set(order[:k])
    ranks = [order.index(i) for i in [tie] + list(range(10, 20))]
    assert min(ranks) < k <= max(ranks)                    # the tie group straddles the boundary
    pos = np.zeros(k, np.int32)
    got = O.lib().orc_topk_positions(P(scores), C.c_int(n_comp), C.c_int(k), C.c_int(n_recent), P(pos))
    rest = sorted(range(n_comp - n_recent), key=lambda i: (-float(scores[i]), i))[:k - n_recent]
    assert got == k and pos.tolist() == sorted(rest + list(range(n_comp - n_recent, n_comp)))
    put("indexer", "q", qi)
    put("indexer", "w", wi)
    put("indexer", "keys", keys.astype(np.float32))
    put("indexer", "scores", scores)
    put("indexer", "mask", mask)
    put("indexer", "positions", pos, top_k=k, n_recent=n_recent,
        tie_key=tie, note="keys hold bf16 values; keys 10..19 repeat the tie key")

    # ---- rope
    xr = synth.normal(405, 0, 4 * 512).reshape(4, 512).astype(np.float32)
    put("rope", "x", xr, pos=70000, n_rot=64)
    for il, inv in ((0, 0), (2, 0), (3, 0), (2, 1)):
        y = np.zeros_like(xr)
        O.lib().orc_rope_tail(P(xr), P(y), C.c_int(4), C.c_int(512), C.c_int(64), C.c_int(70000),
                              C.c_int(il), C.c_int(inv))
        assert np.array_equal(y[:, :448], xr[:, :448])
        if il < 2:   # no YaRN scaling on uncompressed layers: pairs keep their norm
            n0 = np.hypot(xr[:, 448::2], xr[:, 449::2])
            n1 = np.hypot(y[:, 448::2], y[:, 449::2])
            assert np.allclose(n0, n1, rtol=1e-5)
        put("rope", f"il{il}_{'inv' if inv else 'fwd'}", y)

    # ---- rms_norm
    xn = (3 * synth.normal(406, 0, 4096)).astype(np.float32)
    wn = (1 + 0.1 * synth.normal(406, 1, 4096)).astype(np.float32)
    yn = np.zeros_like(xn)
    O.lib().orc_rms_norm_f32(P(xn), P(wn), P(yn), C.c_int(4096), C.c_float(1e-6))
    x64 = xn.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean() + 1e-6) * wn
    assert rel(yn, ref) < 1e-6
    put("rms_norm", "x", xn)
    put("rms_norm", "w", wn)
    put("rms_norm", "y", yn, eps=1e-6)

    # ---- compressor (fp32 weights, in_dim 32, ratio 4, il 2)
    in_dim, steps = 32, 8
    for is_attn, hd, tag in ((1, 512, "attn"), (0, 128, "index")):
        width = 2 * hd
        wkv = (0.2 * synth.normal(407, 10 * is_attn + 0, width * in_dim)).reshape(width, in_dim).astype(np.float32)
        wg = (0.2 * synth.normal(407, 10 * is_attn + 1, width * in_dim)).reshape(width, in_dim).astype(np.float32)
        ape = (0.1 * synth.normal(407, 10 * is_attn + 2, 4 * width)).astype(np.float16).reshape(4, width)
        wnorm = (1 + 0.1 * synth.normal(407, 10 * is_attn + 3, hd)).astype(np.float32)
        xs = synth.normal(407, 10 * is_attn + 4, steps * in_dim).reshape(steps, in_dim).astype(np.float32)
        skv = np.zeros((8, width), np.float32)
        ssc = np.full((8, width), -np.inf, np.float32)
        emits = []
        for p in range(steps):
            e = np.zeros(hd, np.float32)
            r = O.lib().orc_compressor_step_w32(
                C.c_int(is_attn), P(xs[p]), P(wkv), P(wg), P(np.ascontiguousarray(ape.view(np.uint16))),
                P(wnorm), C.c_int(in_dim), C.c_int(hd), C.c_int(4), C.c_int(p), C.c_int(2), P(skv), P(ssc),
                P(e))
            assert r == int((p + 1) % 4 == 0)
            if r:
                emits.append(e)
        case = f"compressor_{tag}"
        put(case, "w_kv", wkv)
        put(case, "w_gate", wg)
        put(case, "ape", ape)
        put(case, "w_norm", wnorm)
        put(case, "x", xs)
        put(case, "emits", np.stack(emits))
        put(case, "state_kv", skv)
        put(case, "state_score", ssc, in_dim=in_dim, head_dim=hd, ratio=4, il=2, steps=steps,
            positions="0..7 from a fresh state")

    # ---- prefill: 2 queries (64 heads) over 40 cached rows + causal self
    n_cached, n_q = 40, 2
    xp = synth.kv_rows(408, 0, n_cached + n_q, outlier_frac=0.1).astype(np.float32)
    cp, sp, tp, dp = O.fp8_quant_rows(xp)
    qp = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(408, 1, n_q * 64 * 512))).reshape(n_q, 64, 512)
    sinks_p = synth.normal(408, 2, 64).astype(np.float32)
    outp = np.zeros_like(qp)
    O.lib().orc_attn_prefill_fp8(P(np.ascontiguousarray(qp)), C.c_int(n_q), P(cp), P(sp), P(tp),
                                 C.c_int(n_cached), P(sinks_p), P(outp), C.c_int(64), C.c_int(512),
                                 C.c_int(64), C.c_int(1))
    kvp = dp.astype(np.float16).astype(np.float64)
    for t in range(n_q):
        kt = kvp[:n_cached + t + 1]
        ref = attn64(qp[t].astype(np.float64), kt, kt, sinks_p.astype(np.float64), 1 / np.sqrt(512))
        assert rel(outp[t], ref) < 1e-5, (t, rel(outp[t], ref))
    put("prefill", "kv_src", xp)
    put("prefill", "q", qp)
    put("prefill", "sinks", sinks_p)
    put("prefill", "out", outp, n_cached=n_cached, n_q=n_q,
        note="query t attends rows 0 .. n_cached + t of kv_src after the FP8 rule")

    # ---- Q8_0 x Q8_0 grouped matvec: 2 groups of 256 inputs, rank 16
    n_groups, group_dim, rank = 2, 256, 16
    wq = (0.05 * synth.normal(409, 0, n_groups * rank * group_dim)).reshape(n_groups * rank, group_dim)
    blocks = wq.reshape(n_groups * rank, group_dim // 32, 32)
    d16 = (np.abs(blocks).max(axis=2) / 127.0).astype(np.float16)
    df = d16.astype(np.float64)
    qw = np.clip(np.where(df[..., None] > 0, np.rint(blocks / np.where(df > 0, df, 1)[..., None]), 0), -128, 127)
    qw = qw.astype(np.int8)
    Wb = np.zeros((n_groups * rank, group_dim // 32, 34), np.uint8)
    Wb[..., :2] = d16.view(np.uint8).reshape(n_groups * rank, group_dim // 32, 2)
    Wb[..., 2:] = qw.view(np.uint8)
    Wb = Wb.reshape(n_groups * rank, -1)
    xg = synth.normal(409, 1, n_groups * group_dim).astype(np.float32)
    yg = np.zeros(n_groups * rank, np.float32)
    O.lib().orc_q8_grouped_matvec(P(np.ascontiguousarray(Wb)), P(xg), P(yg), C.c_int(n_groups),
                                  C.c_int(group_dim), C.c_int(rank))
    # independent: per-32 activation quantization (d = amax / 127, round to
    # nearest even) and the int32 sums, each block scaled by d_w * d_x, in fp64
    xb = xg.astype(np.float64).reshape(-1, 32)
    dx = np.abs(xb).max(axis=1) / 127.0
    xq = np.clip(np.rint(xb / np.where(dx > 0, dx, 1)[:, None]), -127, 127)
    ref = np.zeros(n_groups * rank)
    for r in range(n_groups * rank):
        g = r // rank
        for b in range(group_dim // 32):
            isum = int(np.dot(qw[r, b].astype(np.int64), xq[g * group_dim // 32 + b].astype(np.int64)))
            ref[r] += float(df[r, b]) * dx[g * group_dim // 32 + b] * isum
    assert rel(yg, ref) < 1e-5, rel(yg, ref)
    put("q8_grouped", "w_q8", Wb.astype(np.int32))
    put("q8_grouped", "x", xg)
    put("q8_grouped", "y", yg, n_groups=n_groups, group_dim=group_dim, rank=rank,
        note="w_q8 holds the block_q8_0 bytes (f16 d, 32 int8), one per int32")

    # ---- compressor, ratio 128 (fp32 weights, in_dim 16, il 3): 128 steps, one emit
    in_dim, hd = 16, 512
    wkv = (0.2 * synth.normal(410, 0, hd * in_dim)).reshape(hd, in_dim).astype(np.float32)
    wg = (0.2 * synth.normal(410, 1, hd * in_dim)).reshape(hd, in_dim).astype(np.float32)
    ape = (0.1 * synth.normal(410, 2, 128 * hd)).astype(np.float16).reshape(128, hd)
    wnorm = (1 + 0.1 * synth.normal(410, 3, hd)).astype(np.float32)
    xs = synth.normal(410, 4, 128 * in_dim).reshape(128, in_dim).astype(np.float32)
    skv = np.zeros((128, hd), np.float32)
    ssc = np.full((128, hd), -np.inf, np.float32)
    emit = None
    for p in range(128):
        e = np.zeros(hd, np.float32)
        r = O.lib().orc_compressor_step_w32(
            C.c_int(1), P(xs[p]), P(wkv), P(wg), P(np.ascontiguousarray(ape.view(np.uint16))), P(wnorm),
            C.c_int(in_dim), C.c_int(hd), C.c_int(128), C.c_int(p), C.c_int(3), P(skv), P(ssc), P(e))
        assert r == int(p == 127)
        if r:
            emit = e
    put("compressor_r128", "w_kv", wkv)
    put("compressor_r128", "w_gate", wg)
    put("compressor_r128", "ape", ape)
    put("compressor_r128", "w_norm", wnorm)
    put("compressor_r128", "x", xs)
    put("compressor_r128", "emit", emit, in_dim=in_dim, head_dim=hd, ratio=128, il=3, steps=128)

    (HERE / "index.json").write_text(json.dumps(idx, indent=1, sort_keys=True) + "\n")
    total = sum((HERE / t["file"]).stat().st_size for c in idx.values() for t in c["tensors"].values())
    print(f"wrote {sum(len(c['tensors']) for c in idx.values())} fixtures, {total / 1e3:.0f} KB")


if __name__ == "__main__":
    main()
