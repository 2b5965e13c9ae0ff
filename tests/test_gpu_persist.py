"""Disk persistence of the FP8 session (include/ds4hip_session.h; the
reference's save/load of cuda/kv_persist.cu:1-539 adapted to the 584 B/row
cache): save -> load into a fresh session restores the arena byte for byte,
the counters, pos and n_tokens_processed; a decode over the restored rows is
bit-identical; mismatched geometry, a truncated file, a wrong magic and an
unwritable path are refused."""
import ctypes as C
import struct

import numpy as np
import pytest
import torch

from ds4cuda_amd import Ds4HipError, session, synth

pytestmark = pytest.mark.gpu

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return _hip


def d2h(ptr, n):
    torch.cuda.synchronize()
    buf = np.empty(n, np.uint8)
    assert hip().hipMemcpy(buf.ctypes.data, ptr, n, 2) == 0
    return buf


def h2d(ptr, arr):
    arr = np.ascontiguousarray(arr)
    assert hip().hipMemcpy(ptr, arr.ctypes.data, arr.nbytes, 1) == 0


def fill(s, gpu):
    """Rows in several layers (layer 0's ring wraps), compressed rows and
    indexer keys, and planted compressor state."""
    for il, n in ((0, 140), (2, 21), (3, 9), (42, 3)):
        for t in range(n):
            s.push_raw(il, torch.from_numpy(synth.normal(50 + il, t, 512)).to(gpu))
    for il, n in ((2, 5), (3, 2), (42, 1)):
        for t in range(n):
            s.push_comp(il, torch.from_numpy(synth.normal(60 + il, t, 512) * 3).to(gpu))
    for t in range(4):
        s.push_index_comp(2, torch.from_numpy(synth.normal(70, t, 128)).to(gpu))
    torch.cuda.synchronize()
    for il in (2, 3):
        L = s.layer(il)
        coff = 2 if L.compress_ratio == 4 else 1
        cells = coff * L.compress_ratio * coff * 512
        h2d(L.attn_state_kv, synth.normal(80 + il, 0, cells))
        h2d(L.attn_state_score, synth.normal(80 + il, 1, cells))
    L2 = s.layer(2)
    h2d(L2.index_state_kv, synth.normal(90, 0, 8 * 256))
    h2d(L2.index_state_score, synth.normal(90, 1, 8 * 256))
    s.s.pos = 777
    s.s.n_tokens_processed = 780


def expected_size(s):
    total = 4096 + 8
    for il in range(43):
        L = s.layer(il)
        rows = L.cap_comp + L.cap_raw
        b = rows * (448 + 8 + 128) + rows * 4
        if L.compress_ratio:
            coff = 2 if L.compress_ratio == 4 else 1
            b += 2 * coff * L.compress_ratio * coff * 512 * 4
        if L.has_indexer:
            b += L.cap_comp * 128 * 4 + 2 * 8 * 256 * 4
        total += 64 + b
    return total


def test_save_load_round_trip(gpu, tmp_path):
    path = tmp_path / "kv.ds4hip"
    s = session.Session(1024)
    s2 = session.Session(1024)
    try:
        fill(s, gpu)
        s.save(path, prompt_token_ids=range(100, 200))
        assert path.stat().st_size == expected_size(s)
        hdr = path.read_bytes()[:4096]
        assert hdr[:8] == b"DS4HIPK8"
        version, n_layer, max_ctx, pos, n_tok, n_prompt, cap_raw = struct.unpack_from("<7I", hdr, 8)
        assert (version, n_layer, max_ctx, pos, n_tok, n_prompt, cap_raw) == (1, 43, 1024, 777, 780, 64, 128)
        assert list(struct.unpack_from("<64i", hdr, 56)) == list(range(100, 164))
        assert path.read_bytes()[-8:] == b"DS4HIP01"

        pos, n_tok = s2.load(path)
        assert (pos, n_tok) == (777, 780)
        assert (s2.s.pos, s2.s.n_tokens_processed) == (777, 780)
        for il in range(43):
            a, b = s.layer(il), s2.layer(il)
            assert (a.n_raw, a.raw_head, a.n_comp, a.n_index_comp) == \
                   (b.n_raw, b.raw_head, b.n_comp, b.n_index_comp), il
        assert s.layer(0).n_raw == 128 and s.layer(0).raw_head == 140 % 128
        assert np.array_equal(d2h(s.s.arena_base, s.s.arena_bytes), d2h(s2.s.arena_base, s2.s.arena_bytes))

        # decode over the restored rows: bit-identical to the original session's
        q = torch.from_numpy(synth.normal(95, 0, 64 * 512)).to(gpu)
        sinks = torch.from_numpy(synth.normal(95, 1, 64)).to(gpu)
        for il in (0, 2, 3):
            o1 = torch.empty(64 * 512, device=gpu)
            o2 = torch.empty(64 * 512, device=gpu)
            s.decode(il, q, sinks, o1)
            s2.decode(il, q, sinks, o2)
            torch.cuda.synchronize()
            assert torch.equal(o1, o2), il

        # a restored session keeps working: push on top, and reload over it
        s2.push_raw(2, torch.from_numpy(synth.normal(96, 0, 512)).to(gpu))
        assert s2.layer(2).n_raw == 22
        s2.reset()
        assert s2.load(path) == (777, 780)
        assert s2.layer(2).n_raw == 21
    finally:
        s.close()
        s2.close()


def test_load_refuses_bad_files(gpu, tmp_path):
    path = tmp_path / "kv.ds4hip"
    s = session.Session(512)
    other = session.Session(1024)
    try:
        s.save(path)
        data = path.read_bytes()
        # another max_context: geometry mismatch, -22
        with pytest.raises(Ds4HipError) as e:
            other.load(path)
        assert e.value.code == -22
        # truncated payload: -5
        cut = tmp_path / "cut.ds4hip"
        cut.write_bytes(data[: len(data) // 2])
        with pytest.raises(Ds4HipError) as e:
            s.load(cut)
        assert e.value.code == -5
        # wrong magic: -22
        bad = tmp_path / "bad.ds4hip"
        bad.write_bytes(b"XXXXXXXX" + data[8:])
        with pytest.raises(Ds4HipError) as e:
            s.load(bad)
        assert e.value.code == -22
        # wrong trailer: -22
        tr = tmp_path / "tr.ds4hip"
        tr.write_bytes(data[:-8] + b"DS4HIP99")
        with pytest.raises(Ds4HipError) as e:
            s.load(tr)
        assert e.value.code == -22
        # missing file and unwritable path: -5
        with pytest.raises(Ds4HipError) as e:
            s.load(tmp_path / "missing")
        assert e.value.code == -5
        with pytest.raises(Ds4HipError) as e:
            s.save(tmp_path / "no_such_dir" / "kv")
        assert e.value.code == -5
        # the intact file still loads
        assert s.load(path) == (0, 0)
    finally:
        s.close()
        other.close()
