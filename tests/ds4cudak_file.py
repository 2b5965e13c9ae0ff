"""Writer of the reference's session file format ("DS4CUDAK",
cuda/kv_persist.cuh:6-37,57-88, written by cuda/kv_persist.cu:184-340): the
header and layer metas are the reference's structs written as they are (360
and 64 bytes, little-endian), each layer's buffers at full capacity, then
residual_hc and the trailer. Test data for ds4hip_ds4cudak_probe and
ds4hip_session_import_ds4cudak."""
from __future__ import annotations

import struct

import numpy as np

N_LAYER, HD, IHD = 43, 512, 128


def ratio(il):
    return 0 if il < 2 else (4 if il % 2 == 0 else 128)


def geometry(max_ctx):
    cap_raw = min(128, max_ctx)
    caps = [max_ctx // ratio(il) + 2 if ratio(il) else 0 for il in range(N_LAYER)]
    return cap_raw, caps


def attn_cells(r):
    coff = 2 if r == 4 else 1
    return coff * r * coff * HD


IDX_CELLS = 2 * 4 * 2 * IHD


def layer_payload(r, cap_raw, cap_comp):
    b = cap_raw * HD * 4
    if r:
        b += cap_comp * HD * 4 + 2 * attn_cells(r) * 4
        if r == 4:
            b += cap_comp * IHD * 4 + 2 * IDX_CELLS * 4
    return b


def write(path, max_ctx, pos, n_tokens, prompt_ids=(), layers=None, residual=None):
    """layers: {il: dict(raw=[cap_raw, 512], n_raw, comp=[cap_comp, 512], n_comp,
    st_kv, st_sc, idx=[cap_comp, 128], n_idx, ist_kv, ist_sc)}; missing
    buffers are zeros (scores -inf), missing counts 0."""
    layers = layers or {}
    cap_raw, caps = geometry(max_ctx)
    ids = list(prompt_ids)[:64]
    with open(path, "wb") as f:
        f.write(struct.pack("<8s8I", b"DS4CUDAK", 1, N_LAYER, max_ctx, pos, n_tokens, len(ids), cap_raw, 0))
        f.write(struct.pack("<64i", *(ids + [0] * (64 - len(ids)))))
        f.write(struct.pack("<8Q", *([0] * 8)))
        for il in range(N_LAYER):
            r, cc = ratio(il), caps[il]
            L = layers.get(il, {})
            f.write(struct.pack("<8iQ3Q", il, r, int(r == 4), cap_raw, cc, L.get("n_raw", 0),
                                L.get("n_comp", 0), L.get("n_idx", 0), layer_payload(r, cap_raw, cc), 0, 0, 0))

            def buf(name, shape, fill=0.0):
                a = L.get(name)
                if a is None:
                    a = np.full(shape, fill, np.float32)
                a = np.ascontiguousarray(a, np.float32)
                assert a.size == int(np.prod(shape)), (il, name)
                f.write(a.tobytes())
            buf("raw", (cap_raw, HD))
            if r:
                buf("comp", (cc, HD))
                buf("st_kv", (attn_cells(r),))
                buf("st_sc", (attn_cells(r),), -np.inf)
                if r == 4:
                    buf("idx", (cc, IHD))
                    buf("ist_kv", (IDX_CELLS,))
                    buf("ist_sc", (IDX_CELLS,), -np.inf)
        res = np.zeros(4 * 4096, np.float32) if residual is None else np.asarray(residual, np.float32)
        f.write(res.tobytes())
        f.write(b"DS4CUDA1")
