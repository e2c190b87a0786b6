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
