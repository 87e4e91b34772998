"""Host tests of the early-read scan over compiled assembly (attnarc_amd.isa_check)."""

from __future__ import annotations

from attnarc_amd.isa_check import scan

_HEAD = "_ZN4demo6kernelEv:\n"


def _asm(*body: str) -> str:
    return _HEAD + "\n".join(body) + "\n"


def test_spill_of_an_inline_asm_scalar_load_before_its_wait_is_reported():
    asm = _asm("\t;;#ASMSTART", "\ts_load_dword s0, s[2:3], 0x0", "\t;;#ASMEND",
               "\tv_writelane_b32 v96, s0, 42", "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND")
    found = scan(asm)
    assert len(found) == 1 and "v_writelane_b32 v96, s0, 42" in found[0]


def test_write_of_the_destination_before_the_wait_is_reported():
    asm = _asm("\t;;#ASMSTART", "\ts_load_dword s48, s[52:53], 0x0", "\t;;#ASMEND",
               "\tv_readlane_b32 s48, v106, 33", "\ts_waitcnt lgkmcnt(0)")
    assert len(scan(asm)) == 1


def test_use_after_the_wait_is_clean():
    asm = _asm("\t;;#ASMSTART", "\ts_load_dword s0, s[2:3], 0x0", "\t;;#ASMEND", "\ts_add_u32 s4, s5, s6",
               "\ts_waitcnt lgkmcnt(0)", "\tv_writelane_b32 v96, s0, 42")
    assert scan(asm) == []


def test_loads_and_wait_in_one_statement_are_clean():
    asm = _asm("\t;;#ASMSTART", "\ts_buffer_load_dwordx16 s[36:51], s[20:23], s26",
               "\ts_buffer_load_dwordx16 s[84:99], s[20:23], s27", "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND",
               "\tv_writelane_b32 v1, s36, 0")
    assert scan(asm) == []


def test_compiler_issued_loads_are_not_checked():
    asm = _asm("\ts_load_dword s0, s[2:3], 0x0", "\tv_writelane_b32 v96, s0, 42", "\ts_waitcnt lgkmcnt(0)")
    assert scan(asm) == []


def test_vector_load_read_before_vmcnt_is_reported_and_lds_dma_is_not():
    asm = _asm("\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]", "\t;;#ASMEND",
               "\tv_mov_b32_e32 v20, v5", "\ts_waitcnt vmcnt(0)")
    assert len(scan(asm)) == 1
    dma = _asm("\t;;#ASMSTART", "\tglobal_load_lds_dwordx4 v4, s[0:1] nt", "\t;;#ASMEND", "\tv_mov_b32_e32 v20, v4")
    assert scan(dma) == []
    waited = _asm("\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]", "\t;;#ASMEND",
                  "\ts_waitcnt vmcnt(0)", "\tv_mov_b32_e32 v20, v5")
    assert scan(waited) == []


def test_partial_vmcnt_covers_only_with_enough_later_loads():
    # vmcnt(1) with one later load completes the first load ...
    covered = _asm("\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]", "\t;;#ASMEND",
                   "\tglobal_load_dwordx4 v[8:11], v2, s[0:1] offset:16", "\ts_waitcnt vmcnt(1)",
                   "\tv_mov_b32_e32 v20, v5")
    assert scan(covered) == []
    # ... but not with none: the load may still be in flight
    uncovered = _asm("\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]", "\t;;#ASMEND",
                     "\ts_waitcnt vmcnt(1)", "\tv_mov_b32_e32 v20, v5", "\ts_waitcnt vmcnt(0)")
    assert len(scan(uncovered)) == 1


def test_scalar_load_needs_lgkmcnt_zero():
    asm = _asm("\t;;#ASMSTART", "\ts_load_dword s0, s[2:3], 0x0", "\t;;#ASMEND", "\ts_load_dword s9, s[2:3], 0x4",
               "\ts_waitcnt lgkmcnt(1)", "\ts_add_u32 s4, s0, s6", "\ts_waitcnt lgkmcnt(0)")
    assert len(scan(asm)) == 1


def test_hazard_reached_through_a_loop_back_edge_is_reported():
    # the use precedes the load in text order but follows it around the loop
    asm = _asm(".LBB0_1:", "\tv_mov_b32_e32 v20, v5", "\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]",
               "\t;;#ASMEND", "\ts_cbranch_scc1 .LBB0_1", "\ts_waitcnt vmcnt(0)", "\ts_endpgm")
    found = scan(asm)
    assert len(found) == 1 and "v_mov_b32_e32 v20, v5" in found[0]


def test_both_sides_of_a_branch_are_followed():
    asm = _asm("\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]", "\t;;#ASMEND",
               "\ts_cbranch_scc0 .LBB0_2", "\ts_waitcnt vmcnt(0)", "\ts_branch .LBB0_3", ".LBB0_2:",
               "\tv_add_f32_e32 v21, v6, v6", ".LBB0_3:", "\ts_endpgm")
    found = scan(asm)
    assert len(found) == 1 and "v_add_f32_e32 v21, v6, v6" in found[0]


def test_constant_false_loop_branch_is_not_followed():
    # vcc = exec & ~(-1) = 0: the s_cbranch_vccnz back to the header is never taken
    asm = _asm(".LBB0_1:", "\tv_mov_b32_e32 v20, v5", "\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v2, s[0:1]",
               "\t;;#ASMEND", "\ts_mov_b64 s[8:9], -1", "\ts_cbranch_scc1 .LBB0_2", "\ts_andn2_b64 vcc, exec, s[8:9]",
               "\ts_cbranch_vccnz .LBB0_1", ".LBB0_2:", "\ts_waitcnt vmcnt(0)", "\ts_endpgm")
    assert scan(asm) == []
    # with the register set elsewhere the branch may be taken
    live = asm.replace("s_mov_b64 s[8:9], -1", "s_mov_b64 s[8:9], s[10:11]")
    assert len(scan(live)) == 1
