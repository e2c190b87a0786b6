"""Host-side checks of the build's assembly guard (no GPU needed)."""

from flashfusedmoe_amd.build import unsafe_scratch_ops


def test_scratch_between_dma_and_counted_wait_is_flagged():
    asm = """_ZN5ffmoe4kernE:
  buffer_load_dwordx4 v1, s[0:3], 0 offen lds
  scratch_store_dword off, v0, off offset:4
  s_waitcnt vmcnt(4)
"""
    bad = unsafe_scratch_ops(asm)
    assert len(bad) == 1 and bad[0][0] == "_ZN5ffmoe4kernE"


def test_scratch_after_full_drain_or_before_dma_is_allowed():
    asm = """_ZN5ffmoe4kernE:
  scratch_load_dword v0, off, off
  buffer_load_dwordx4 v1, s[0:3], 0 offen lds
  s_waitcnt vmcnt(0)
  scratch_store_dword off, v0, off offset:4
  buffer_load_dwordx4 v1, s[0:3], 0 offen lds
  s_waitcnt vmcnt(8)
.LBB0_3:
  scratch_store_dword off, v0, off offset:8
  s_waitcnt vmcnt(2)
"""
    assert unsafe_scratch_ops(asm) == []


def test_claim_register_read_before_its_wait_is_flagged():
    from flashfusedmoe_amd.build import unwaited_claim_reads
    # one path waits, the branch target spills the claim register first
    asm = """_ZN5ffmoe4kernE:
  global_atomic_add v7, v[2:3], v4, off sc0
  s_cbranch_scc1 .LBB0_2
  s_waitcnt vmcnt(0)
  v_readfirstlane_b32 s0, v7
.LBB0_2:
  scratch_store_dword off, v7, off offset:8
  s_waitcnt vmcnt(0)
  s_endpgm
.Lfunc_end0:
"""
    bad = unwaited_claim_reads(asm)
    assert len(bad) == 1 and "scratch_store_dword" in bad[0][2]


def test_claim_register_after_its_wait_is_allowed():
    from flashfusedmoe_amd.build import unwaited_claim_reads
    asm = """_ZN5ffmoe4kernE:
  global_atomic_add v7, v[2:3], v4, off sc0
  v_mov_b32 v8, v9
  s_branch .LBB0_2
.LBB0_2:
  s_waitcnt vmcnt(0) lgkmcnt(0)
  v_readfirstlane_b32 s0, v[6:7]
  s_endpgm
.Lfunc_end0:
"""
    assert unwaited_claim_reads(asm) == []
