"""The committed golden fixtures (tests/golden, DSST files written by
tests/golden/make_golden.py) against the CPU oracle: every recorded output
must be reproduced bit for bit from the recorded inputs, so a change of the
oracle's arithmetic shows here; the fixtures' independent checks (a numpy
restatement of the FP8 rule, fp64 attention, stable-sort selection) run again
on the recorded data. The GPU tests compare the kernels with the oracle, so
the kernels meet these vectors through it."""
import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from oracle import P

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import dsst                 # noqa: E402
import make_golden as MG    # noqa: E402

INDEX = json.loads((GOLD / "index.json").read_text())


def T(case, name):
    meta = INDEX[case]["tensors"][name]
    return dsst.read(GOLD / meta["file"]).reshape(meta["shape"])


def test_index_lists_every_file():
    files = {t["file"] for c in INDEX.values() for t in c["tensors"].values()}
    on_disk = {p.name for p in GOLD.glob("*.bin")}
    assert files == on_disk


def test_fp8_rows():
    x = T("fp8_rows", "x")
    codes, sexp, tail, deq = O.fp8_quant_rows(x)
    assert np.array_equal(codes.astype(np.int32), T("fp8_rows", "codes"))
    assert np.array_equal(sexp.astype(np.int32), T("fp8_rows", "sexp"))
    assert np.array_equal(tail, T("fp8_rows", "tail").view(np.uint16))
    assert np.array_equal(deq, T("fp8_rows", "deq"))
    c2, s2, t2 = MG.numpy_fp8_rows(x)
    assert np.array_equal(c2, codes) and np.array_equal(s2, sexp) and np.array_equal(t2, tail)
    assert (sexp[1, 0] == -22) and (codes[3, 64:128] == 0x80).all()


def test_decode_fp8():
    src, q, sinks = T("decode_fp8", "kv_src"), T("decode_fp8", "q"), T("decode_fp8", "sinks")
    c, s, t, dq = O.fp8_quant_rows(src)
    out = O.attn_decode_fp8(q, c, s, t, np.arange(src.shape[0]), sinks)
    assert np.array_equal(out, T("decode_fp8", "out"))
    kv = dq.astype(np.float16).astype(np.float64)
    assert MG.rel(out, MG.attn64(q.astype(np.float64), kv, kv, sinks.astype(np.float64), 1 / np.sqrt(512))) < 1e-5


def test_decode_mix():
    q, raw, comp = T("decode_mix", "q"), T("decode_mix", "raw"), T("decode_mix", "comp")
    allowed, sinks = T("decode_mix", "allowed"), T("decode_mix", "sinks")
    out = O.attn_decode_mixed_f32(q, raw, comp, allowed, sinks)
    assert np.array_equal(out, T("decode_mix", "out"))
    kv = np.concatenate([raw, comp[allowed == 1]]).astype(np.float16).astype(np.float64)
    assert MG.rel(out, MG.attn64(q.astype(np.float64), kv, kv, sinks.astype(np.float64), 1 / np.sqrt(512))) < 5e-5


def test_indexer():
    from ds4cuda_amd import synth
    q, w, keys = T("indexer", "q"), T("indexer", "w"), T("indexer", "keys")
    prm = INDEX["indexer"]["params"]
    n, k, nr = keys.shape[0], prm["top_k"], prm["n_recent"]
    scores = np.zeros(n, np.float32)
    O.lib().orc_indexer_scores(P(q), P(w), P(np.ascontiguousarray(synth.to_bf16_bits(keys))), C.c_int(2),
                               C.c_int(n), C.c_int(64), C.c_int(128), P(scores))
    assert np.array_equal(scores, T("indexer", "scores"))
    mask = np.zeros(n, np.int32)
    O.lib().orc_topk_mask(P(scores), C.c_int(n), C.c_int(k), P(mask))
    assert np.array_equal(mask, T("indexer", "mask"))
    pos = np.zeros(k, np.int32)
    assert O.lib().orc_topk_positions(P(scores), C.c_int(n), C.c_int(k), C.c_int(nr), P(pos)) == k
    assert np.array_equal(pos, T("indexer", "positions"))
    order = sorted(range(n), key=lambda i: (-float(scores[i]), i))
    assert set(np.flatnonzero(mask).tolist()) == set(order[:k])
    rest = sorted(range(n - nr), key=lambda i: (-float(scores[i]), i))[:k - nr]
    assert pos.tolist() == sorted(rest + list(range(n - nr, n)))


def test_rope():
    x = T("rope", "x")
    for il, inv in ((0, 0), (2, 0), (3, 0), (2, 1)):
        y = np.zeros_like(x)
        O.lib().orc_rope_tail(P(x), P(y), C.c_int(4), C.c_int(512), C.c_int(64), C.c_int(70000), C.c_int(il),
                              C.c_int(inv))
        assert np.array_equal(y, T("rope", f"il{il}_{'inv' if inv else 'fwd'}")), (il, inv)


def test_rms_norm():
    x, w = T("rms_norm", "x"), T("rms_norm", "w")
    y = np.zeros_like(x)
    O.lib().orc_rms_norm_f32(P(x), P(w), P(y), C.c_int(x.size), C.c_float(1e-6))
    assert np.array_equal(y, T("rms_norm", "y"))


@pytest.mark.parametrize("tag,is_attn", [("attn", 1), ("index", 0)])
def test_compressor(tag, is_attn):
    case = f"compressor_{tag}"
    prm = INDEX[case]["params"]
    wkv, wg, ape = T(case, "w_kv"), T(case, "w_gate"), T(case, "ape")
    wn, xs = T(case, "w_norm"), T(case, "x")
    hd, in_dim = prm["head_dim"], prm["in_dim"]
    skv = np.zeros((8, 2 * hd), np.float32)
    ssc = np.full((8, 2 * hd), -np.inf, np.float32)
    emits = []
    for p in range(prm["steps"]):
        e = np.zeros(hd, np.float32)
        r = O.lib().orc_compressor_step_w32(
            C.c_int(is_attn), P(np.ascontiguousarray(xs[p])), P(wkv), P(wg),
            P(np.ascontiguousarray(ape.view(np.uint16))), P(wn), C.c_int(in_dim), C.c_int(hd), C.c_int(4),
            C.c_int(p), C.c_int(prm["il"]), P(skv), P(ssc), P(e))
        if r:
            emits.append(e)
    assert np.array_equal(np.stack(emits), T(case, "emits"))
    assert np.array_equal(skv, T(case, "state_kv")) and np.array_equal(ssc, T(case, "state_score"))


def test_dsst_rejects_bad_files(tmp_path):
    good = tmp_path / "g.bin"
    dsst.write(good, np.arange(5, dtype=np.int32))
    assert dsst.read(good).tolist() == [0, 1, 2, 3, 4]
    b = good.read_bytes()
    for bad in (b"XSST" + b[4:], b[:-4], b[:8] + b"\x07" + b[9:]):
        p = tmp_path / "b.bin"
        p.write_bytes(bad)
        with pytest.raises(ValueError):
            dsst.read(p)


def test_prefill():
    src, q, sinks = T("prefill", "kv_src"), T("prefill", "q"), T("prefill", "sinks")
    n_cached = INDEX["prefill"]["params"]["n_cached"]
    c, s, t, dq = O.fp8_quant_rows(src)
    out = np.zeros_like(q)
    O.lib().orc_attn_prefill_fp8(P(np.ascontiguousarray(q)), C.c_int(q.shape[0]), P(c), P(s), P(t),
                                 C.c_int(n_cached), P(sinks), P(out), C.c_int(64), C.c_int(512), C.c_int(64),
                                 C.c_int(1))
    assert np.array_equal(out, T("prefill", "out"))
    kv = dq.astype(np.float16).astype(np.float64)
    for i in range(q.shape[0]):
        k = kv[:n_cached + i + 1]
        assert MG.rel(out[i], MG.attn64(q[i].astype(np.float64), k, k, sinks.astype(np.float64),
                                        1 / np.sqrt(512))) < 1e-5


def test_q8_grouped():
    prm = INDEX["q8_grouped"]["params"]
    w = np.ascontiguousarray(T("q8_grouped", "w_q8").astype(np.uint8))
    x = T("q8_grouped", "x")
    y = np.zeros(prm["n_groups"] * prm["rank"], np.float32)
    O.lib().orc_q8_grouped_matvec(P(w), P(x), P(y), C.c_int(prm["n_groups"]), C.c_int(prm["group_dim"]),
                                  C.c_int(prm["rank"]))
    assert np.array_equal(y, T("q8_grouped", "y"))


def test_compressor_ratio128():
    case = "compressor_r128"
    prm = INDEX[case]["params"]
    wkv, wg, ape = T(case, "w_kv"), T(case, "w_gate"), T(case, "ape")
    wn, xs = T(case, "w_norm"), T(case, "x")
    hd = prm["head_dim"]
    skv = np.zeros((128, hd), np.float32)
    ssc = np.full((128, hd), -np.inf, np.float32)
    emit = None
    for p in range(prm["steps"]):
        e = np.zeros(hd, np.float32)
        if O.lib().orc_compressor_step_w32(C.c_int(1), P(np.ascontiguousarray(xs[p])), P(wkv), P(wg),
                                           P(np.ascontiguousarray(ape.view(np.uint16))), P(wn),
                                           C.c_int(prm["in_dim"]), C.c_int(hd), C.c_int(128), C.c_int(p),
                                           C.c_int(prm["il"]), P(skv), P(ssc), P(e)):
            emit = e
    assert emit is not None and np.array_equal(emit, T(case, "emit"))
