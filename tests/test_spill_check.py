"""The build's copy-ring spill check (ds4cuda_amd/spill_check.py) on small
hand-written gfx950 assembly: it must report a spill store that any path
reaches while a global_load_lds copy may be outstanding, and nothing else."""
from ds4cuda_amd.spill_check import ring_violations


def kern(body: str) -> str:
    return "k:\n" + "\n".join("\t" + ln if not ln.startswith(".") else ln
                              for ln in body.strip().splitlines()) + "\n\ts_endpgm\n"


def test_store_after_copy_is_reported():
    asm = kern("""
global_load_lds_dwordx4 v1, s[0:1]
scratch_store_dword off, v2, off
s_waitcnt vmcnt(0)
""")
    assert ring_violations(asm, "k") == ["scratch_store_dword off, v2, off"]


def test_access_after_full_wait_or_before_copies_is_allowed():
    asm = kern("""
scratch_store_dword off, v2, off
global_load_lds_dwordx4 v1, s[0:1]
s_waitcnt vmcnt(0) lgkmcnt(0)
scratch_load_dword v3, off, off
""")
    assert ring_violations(asm, "k") == []


def test_partial_wait_keeps_the_ring_open():
    asm = kern("""
global_load_lds_dwordx4 v1, s[0:1]
s_waitcnt vmcnt(5)
scratch_store_dword off, v3, off
s_waitcnt vmcnt(0)
""")
    assert len(ring_violations(asm, "k")) == 1


def test_reloads_only_tighten_the_waits():
    # a reload returns in order with the copies: reported only on request
    asm = kern("""
global_load_lds_dwordx4 v1, s[0:1]
scratch_load_dword v3, off, off
s_waitcnt vmcnt(0)
""")
    assert ring_violations(asm, "k") == []
    assert ring_violations(asm, "k", loads=True) == ["scratch_load_dword v3, off, off"]


def test_loop_back_edge_carries_outstanding_copies():
    # the spill at the loop head is reached from the copy at the loop's end
    asm = kern("""
s_mov_b32 s4, 0
.LBB0_1:
scratch_store_dword off, v3, off
v_add_u32 v4, v3, v4
global_load_lds_dwordx4 v1, s[0:1]
s_cmp_lt_u32 s4, 8
s_cbranch_scc1 .LBB0_1
s_waitcnt vmcnt(0)
""")
    assert ring_violations(asm, "k") == ["scratch_store_dword off, v3, off"]


def test_loop_that_drains_before_its_back_edge_is_allowed():
    asm = kern("""
.LBB0_1:
scratch_store_dword off, v3, off
global_load_lds_dwordx4 v1, s[0:1]
s_waitcnt vmcnt(0)
s_cmp_lt_u32 s4, 8
s_cbranch_scc1 .LBB0_1
""")
    assert ring_violations(asm, "k") == []


def test_branch_join_takes_the_worse_path():
    asm = kern("""
s_cbranch_scc1 .LBB0_2
global_load_lds_dwordx4 v1, s[0:1]
.LBB0_2:
scratch_store_dword off, v2, off
s_waitcnt vmcnt(0)
""")
    assert len(ring_violations(asm, "k")) == 1
