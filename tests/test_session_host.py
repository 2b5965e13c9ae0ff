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
