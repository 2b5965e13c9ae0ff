"""Import of a reference session file (DS4CUDAK, fp32 rows) into the FP8
session: counters, ring placement (raw row i of a layer holds position
pos - n_raw + i and lands in slot (pos - n_raw + i) % 128), FP8 codes of the
window and compressed rows bit-exact against the oracle's quantization,
compressor / indexer state copied bit for bit, and decode attention over the
imported rows against the oracle over the file's rows."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
import ds4cudak_file as F
from ds4cuda_amd import session, synth

pytestmark = pytest.mark.gpu


def d2h(ptr, n):
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    torch.cuda.synchronize()
    b = np.empty(n, np.uint8)
    assert hip.hipMemcpy(b.ctypes.data, ptr, n, 2) == 0
    return b


@pytest.mark.parametrize("max_ctx,pos", [(256, 203), (64, 64)])
def test_import_reference_session(gpu, tmp_path, max_ctx, pos):
    # max_ctx 64: the ratio-128 states (128 x 512 floats) are larger than the
    # 64-row window buffer the import stages rows through
    cap_raw, caps = F.geometry(max_ctx)
    nc = min(50, caps[2])
    raw0 = synth.kv_rows(501, 0, cap_raw, outlier_frac=0.02).astype(np.float32)
    raw2 = synth.kv_rows(501, 2, cap_raw).astype(np.float32)
    comp2 = np.zeros((caps[2], 512), np.float32)
    comp2[:nc] = 2 * synth.kv_rows(501, 3, nc)
    st_kv = synth.normal(501, 4, F.attn_cells(4)).astype(np.float32)
    st_sc = synth.normal(501, 5, F.attn_cells(4)).astype(np.float32)
    idx = np.zeros((caps[2], 128), np.float32)
    idx[:nc] = synth.normal(501, 6, nc * 128).reshape(nc, 128)
    layers = {0: {"n_raw": cap_raw, "raw": raw0},
              2: {"n_raw": cap_raw, "raw": raw2, "comp": comp2, "n_comp": nc, "st_kv": st_kv,
                  "st_sc": st_sc, "idx": idx, "n_idx": nc}}
    path = tmp_path / "ref.kvc"
    F.write(path, max_ctx, pos, pos, range(7), layers)
    s = session.Session(max_ctx)
    try:
        assert s.import_ds4cudak(path) == (pos, pos)
        L0, L2 = s.layer(0), s.layer(2)
        assert (L0.n_raw, L0.raw_head, L0.n_comp) == (cap_raw, pos % cap_raw, 0)
        assert (L2.n_raw, L2.n_comp, L2.n_index_comp) == (cap_raw, nc, nc)
        # FP8 codes of the ring: raw row i in slot (pos - 128 + i) % 128
        codes, sexp, tail, deq0 = O.fp8_quant_rows(raw0)
        rows = cap_raw + L0.cap_comp
        got = d2h(s.s.codes + L0.row_base * 448, rows * 448).reshape(rows, 448)
        for i in range(cap_raw):
            assert np.array_equal(got[L0.cap_comp + (pos - cap_raw + i) % cap_raw], codes[i]), i
        # compressed rows of layer 2 in order
        c2, _, _, deq_c = O.fp8_quant_rows(comp2[:nc])
        got2 = d2h(s.s.codes + L2.row_base * 448, nc * 448).reshape(nc, 448)
        assert np.array_equal(got2, c2)
        # state copied as it is
        assert np.array_equal(d2h(L2.attn_state_kv, st_kv.nbytes).view(np.float32), st_kv)
        assert np.array_equal(d2h(L2.attn_state_score, st_sc.nbytes).view(np.float32), st_sc)
        assert np.array_equal(d2h(L2.index_comp_kv, nc * 128 * 4).view(np.float32), idx[:nc].reshape(-1))
        # decode over the imported rows against the oracle over the file's rows
        q = synth.normal(502, 0, 64 * 512).reshape(64, 512).astype(np.float32)
        sinks = synth.normal(502, 1, 64).astype(np.float32)
        for il, kv in ((0, raw0), (2, np.concatenate([raw2, comp2[:nc]]))):
            out = torch.empty(64 * 512, device=gpu)
            s.decode(il, torch.from_numpy(q.reshape(-1)).to(gpu), torch.from_numpy(sinks).to(gpu), out)
            torch.cuda.synchronize()
            cq, sq, tq, _ = O.fp8_quant_rows(kv)
            ref = O.attn_decode_fp8(q, cq, sq, tq, np.arange(kv.shape[0]), sinks)
            err = np.abs(out.cpu().numpy().reshape(64, 512) - ref).max() / np.sqrt(np.mean(ref.astype(np.float64) ** 2))
            assert err < 2e-3, (il, err)
    finally:
        s.close()


def test_reference_file_round_trip(gpu, tmp_path):
    """A reference file whose rows are what the reference holds (window rows
    FP8 values rounded to f16, compressed rows FP8 values with an f16 tail)
    comes back byte for byte from import followed by export, except that a
    -0.0 in a coded dim comes back as +0.0 (the reference's quantizer rule)."""
    max_ctx, pos = 256, 300
    cap_raw, caps = F.geometry(max_ctx)

    def window(seed):
        return O.fp8_quant_rows(synth.kv_rows(511, seed, cap_raw).astype(np.float32))[3].astype(np.float16).astype(np.float32)

    def comp(seed, n, cap):
        out = np.zeros((cap, 512), np.float32)
        d = O.fp8_quant_rows(synth.kv_rows(511, seed, n).astype(np.float32))[3]
        d[:, 448:] = d[:, 448:].astype(np.float16).astype(np.float32)
        out[:n] = d
        return out
    layers = {}
    for il in range(43):
        r = F.ratio(il)
        L = {"n_raw": cap_raw, "raw": window(il)}
        if r:
            n = min(pos // r, caps[il])
            L.update(n_comp=n, comp=comp(100 + il, n, caps[il]),
                     st_kv=synth.normal(512, il, F.attn_cells(r)), st_sc=synth.normal(513, il, F.attn_cells(r)))
            if r == 4:
                idx = np.zeros((caps[il], 128), np.float32)
                idx[:n] = synth.normal(514, il, n * 128).reshape(n, 128)
                L.update(idx=idx, n_idx=n, ist_kv=synth.normal(515, il, F.IDX_CELLS),
                         ist_sc=synth.normal(516, il, F.IDX_CELLS))
        layers[il] = L
    src, back, exp = tmp_path / "src.kvc", tmp_path / "back.kvc", tmp_path / "exp.kvc"
    F.write(src, max_ctx, pos, pos, range(40), layers)
    # The reference's quantizer takes the sign from x < 0 (cuda/fp8_kv.cu:102),
    # so a -0.0 in a coded dim (an FP8 -0 the reference holds) quantizes to +0:
    # the export writes +0.0 there. Everything else comes back unchanged.
    for L in layers.values():
        for name in ("raw", "comp"):
            if name in L:
                x = L[name].copy()
                x[:, :448] = np.where(x[:, :448] == 0, np.float32(0), x[:, :448])
                L[name] = x
    F.write(exp, max_ctx, pos, pos, range(40), layers)
    s = session.Session(max_ctx)
    try:
        s.import_ds4cudak(src)
        s.export_ds4cudak(back, prompt_token_ids=range(40))
    finally:
        s.close()
    a, b = exp.read_bytes(), back.read_bytes()
    assert len(a) == len(b)
    assert src.read_bytes() != a    # the case above occurs in this file
    assert a == b
