"""Host-side arena sizing of the FP8 session (no GPU needed)."""
from ds4cuda_amd import session


def align(n):
    return (n + 255) // 256 * 256


def expected_bytes(max_ctx):
    cap_raw = min(128, max_ctx)
    ratio = lambda il: 0 if il < 2 else (4 if il % 2 == 0 else 128)
    caps = [max_ctx // ratio(il) + 2 if ratio(il) else 0 for il in range(43)]
    rows = sum(c + cap_raw for c in caps) + 128   # + the prefill chunk's staging rows
    b = align(rows * 448) + align(rows * 8) + align(rows * 128)
    b += sum(align((cap_raw + c) * 4) for c in caps)
    for il in range(43):
        r = ratio(il)
        if not r:
            continue
        coff = 2 if r == 4 else 1
        b += 2 * align(coff * r * coff * 512 * 4)
        if r == 4:
            b += align(caps[il] * 128 * 4) + 2 * align(8 * 256 * 4)
    return b


def test_arena_bytes_formula():
    for ctx in (1, 100, 128, 4096, 16384, 131072):
        assert session.arena_bytes(ctx) == expected_bytes(ctx), ctx
    assert session.arena_bytes(0) == 0
    # FP8 rows: the 4K-context arena is far below the fp32 reference's ~93 MB
    assert session.arena_bytes(4096) < 45e6


# ---- prefill chunk row lists (host form; the device form shares the entry function)

import ctypes as C

import numpy as np
import pytest

from ds4cuda_amd import lib


def described(max_ctx):
    s = session.SessionState()
    assert lib().ds4hip_session_state_describe(C.byref(s), max_ctx) == 0
    return s


def expected_lists(L, n_cache_rows, p0, n_tok, n_comp, n_sel, sel):
    """What a single-token step at position p0 + t attends, rewritten for the
    chunk: window positions below p0 in the ring (slot x % cap_raw after the
    compressed rows), positions p0 .. p0 + t in staging rows 0 .. t, then the
    token's compressed rows (all, or its selection)."""
    stage_rel = n_cache_rows - L.row_base
    out = []
    for t in range(n_tok):
        P = p0 + t
        win = range(max(0, P - L.cap_raw + 1), P + 1)
        rows = [L.cap_comp + x % L.cap_raw if x < p0 else stage_rel + (x - p0) for x in win]
        rows += list(range(n_comp[t])) if n_sel[t] == n_comp[t] else list(sel[t][:n_sel[t]])
        out.append(rows)
    return out


def host_lists(s, il, p0, n_tok, n_comp, n_sel, sel, stride):
    nc = np.asarray(n_comp, np.int32)
    ns = np.asarray(n_sel, np.int32)
    lists = np.full((n_tok, stride), -7, np.int32)
    counts = np.zeros(n_tok, np.int64)
    selp = None
    sel_stride = 0
    if sel is not None:
        sel = np.ascontiguousarray(sel, np.int32)
        selp, sel_stride = sel.ctypes.data_as(C.c_void_p), sel.shape[1]
    rc = lib().ds4hip_session_chunk_rows_host(C.byref(s), il, p0, n_tok, nc.ctypes.data_as(C.c_void_p),
                                              ns.ctypes.data_as(C.c_void_p), selp, sel_stride,
                                              lists.ctypes.data_as(C.c_void_p), stride,
                                              counts.ctypes.data_as(C.c_void_p))
    return rc, lists, counts


@pytest.mark.parametrize("il,p0,n_tok,ctx", [(0, 0, 5, 4096), (0, 3, 128, 4096), (0, 150, 41, 4096),
                                            (2, 127, 2, 4096), (3, 1000, 128, 4096), (2, 130, 126, 4096),
                                            (0, 20, 44, 64), (2, 37, 27, 64), (3, 0, 64, 64)])
def test_chunk_rows_match_token_steps(il, p0, n_tok, ctx):
    s = described(ctx)
    L = s.layers[il]
    L.n_raw, L.raw_head = min(p0, L.cap_raw), p0 % L.cap_raw
    rng = np.random.default_rng(il * 1000 + p0)
    ratio = L.compress_ratio
    n_comp = [((p0 + t + 1) // ratio if ratio else 0) for t in range(n_tok)]
    sel = None
    n_sel = list(n_comp)
    if ratio == 4:   # a selection of 8 for tokens with more than 8 compressed rows
        sel = np.zeros((n_tok, 8), np.int32)
        for t in range(n_tok):
            if n_comp[t] > 8:
                sel[t] = np.sort(rng.choice(n_comp[t], 8, replace=False))
                n_sel[t] = 8
    stride = 128 + n_tok + max(n_comp + [0]) + 3
    rc, lists, counts = host_lists(s, il, p0, n_tok, n_comp, n_sel, sel, stride)
    assert rc == 0
    exp = expected_lists(L, s.n_cache_rows, p0, n_tok, n_comp, n_sel, sel)
    for t in range(n_tok):
        assert counts[t] == len(exp[t]), t
        assert lists[t, :counts[t]].tolist() == exp[t], t
        assert (lists[t, counts[t]:] == -7).all()   # nothing past the count
        # every window row is a row of this layer's ring or of the staging area
        win = lists[t, :counts[t] - n_sel[t]]
        ring = (win >= L.cap_comp) & (win < L.cap_comp + L.cap_raw)
        stage = (win >= s.n_cache_rows - L.row_base) & (win < s.n_cache_rows - L.row_base + 128)
        assert (ring | stage).all()
        # every entry the decode will read lies inside the arena's rows
        # (relative to the layer's first row: the layer's rows and the staging rows)
        assert counts[t] <= stride
        ent = lists[t, :counts[t]]
        assert (ent >= 0).all() and (ent < s.n_cache_rows - L.row_base + 128).all()
        comp = lists[t, counts[t] - n_sel[t]:counts[t]]
        assert (comp < max(n_comp[t], 1)).all()


def test_chunk_rows_refuse_bad_arguments():
    s = described(4096)
    L = s.layers[0]
    L.n_raw, L.raw_head = 100, 100
    ok = host_lists(s, 0, 100, 4, [0] * 4, [0] * 4, None, 256)
    assert ok[0] == 0
    assert host_lists(s, 0, 101, 4, [0] * 4, [0] * 4, None, 256)[0] == -22     # ring not at p0
    assert host_lists(s, 0, 100, 129, [0] * 129, [0] * 129, None, 256)[0] == -22   # > 128 tokens
    assert host_lists(s, 0, 100, 4, [0] * 4, [0] * 4, None, 100)[0] == -22     # list too short
    assert host_lists(s, 0, 100, 4, [0] * 4, [0] * 4, None, 256)[0] == 0
    s64 = described(64)
    s64.layers[0].n_raw, s64.layers[0].raw_head = 60, 60
    assert host_lists(s64, 0, 60, 4, [0] * 4, [0] * 4, None, 256)[0] == 0
    assert host_lists(s64, 0, 60, 5, [0] * 5, [0] * 5, None, 256)[0] == -22   # past max_context
    s64.layers[0].n_raw, s64.layers[0].raw_head = 0, 0
    assert host_lists(s64, 0, 0, 64, [0] * 64, [0] * 64, None, 256)[0] == 0
    s100 = described(100)   # cap_raw 100: a chunk of more tokens than the window holds
    assert host_lists(s100, 0, 0, 101, [0] * 101, [0] * 101, None, 256)[0] == -22
    L2 = s.layers[2]
    L2.n_raw, L2.raw_head = 100, 100
    assert host_lists(s, 2, 100, 2, [30, 30], [8, 8], None, 256)[0] == -22     # selection missing
    assert host_lists(s, 2, 100, 2, [3, 3], [4, 3], np.zeros((2, 8)), 256)[0] == -22   # more than n_comp
    assert host_lists(s, 2, 100, 2, [30, 30], [9, 9], np.zeros((2, 8)), 256)[0] == -22  # past sel_stride


def test_describe_matches_arena_bytes():
    for ctx in (100, 4096, 131072):
        s = described(ctx)
        assert s.arena_bytes == session.arena_bytes(ctx)
        assert not s.arena_base and not s.codes
        assert s.layers[42].row_base + s.layers[42].cap_comp + s.layers[42].cap_raw == s.n_cache_rows
