"""The build's DPP wait-state check (lazyweights_amd/build.py dpp_violations) on hand-written disassembly: the
hazards it must refuse and the forms it must accept (the check guards the inline-assembly DPP products, which the
compiler's hazard recognizer does not see)."""
from lazyweights_amd.build import dpp_violations

HEAD = "0000000000001000 <k>:\n"


def line(addr, text, target=None):
    t = " <k+0x%x>" % target if target is not None else ""
    return "\t%s // %012X: 00000000%s\n" % (text, addr, t)


DPP = "v_dot2c_f32_f16_dpp v10, v5, v7 row_newbcast:3 row_mask:0xf bank_mask:0xf bound_ctrl:1"


def body(*rows):
    return HEAD + "".join(line(0x1000 + 4 * i, r) for i, r in enumerate(rows))


def test_valu_write_of_the_dpp_source_right_before_is_refused():
    pad = ["s_mov_b32 s0, 0"] * 6
    assert dpp_violations(body(*pad, "v_mov_b32_e32 v5, v1", DPP))
    assert dpp_violations(body(*pad, "v_add_u32_e32 v5, v1, v2", "v_nop", DPP))


def test_two_wait_states_or_another_register_are_accepted():
    pad = ["s_mov_b32 s0, 0"] * 6
    assert not dpp_violations(body(*pad, "v_mov_b32_e32 v5, v1", "s_nop 1", DPP))
    assert not dpp_violations(body(*pad, "v_mov_b32_e32 v5, v1", "v_nop", "v_nop", DPP))
    assert not dpp_violations(body(*pad, "v_mov_b32_e32 v6, v1", DPP))  # v6 is not the DPP source
    assert not dpp_violations(body(*pad, "global_load_dword v5, v[2:3], off", DPP))  # memory writes: no hazard


def test_exec_write_needs_five_wait_states():
    pad = ["s_mov_b32 s0, 0"] * 6
    assert dpp_violations(body(*pad, "s_mov_b64 exec, s[4:5]", "v_nop", "v_nop", DPP))
    assert not dpp_violations(body(*pad, "s_mov_b64 exec, s[4:5]", "s_nop 4", DPP))


def test_a_dpp_operation_at_a_block_start_needs_its_waits_inside_the_block():
    rows = ["s_mov_b32 s0, 0"] * 4 + [DPP]
    text = HEAD + "".join(line(0x1000 + 4 * i, r) for i, r in enumerate(rows))
    text += line(0x1000 + 4 * len(rows), "s_branch 0", target=4 * 4)  # jumps to the DPP operation
    assert dpp_violations(text)
    rows = ["s_mov_b32 s0, 0"] * 4 + ["s_nop 4", DPP]
    text = HEAD + "".join(line(0x1000 + 4 * i, r) for i, r in enumerate(rows))
    text += line(0x1000 + 4 * len(rows), "s_branch 0", target=4 * 4)  # jumps to the s_nop
    assert not dpp_violations(text)


def test_vcmpx_writes_exec_and_needs_five_wait_states():
    """v_cmpx writes EXEC implicitly (its first operand names vcc or an SGPR pair, not exec)."""
    pad = ["s_mov_b32 s0, 0"] * 6
    assert dpp_violations(body(*pad, "v_cmpx_gt_u32_e32 vcc, s4, v1", DPP))
    assert dpp_violations(body(*pad, "v_cmpx_gt_u32_e64 s[4:5], s4, v1", "v_nop", "v_nop", DPP))
    assert not dpp_violations(body(*pad, "v_cmpx_gt_u32_e32 vcc, s4, v1", "s_nop 4", DPP))


def test_mfma_write_of_the_dpp_source_needs_the_matrix_core_wait():
    pad = ["s_mov_b32 s0, 0"] * 6
    mfma = "v_mfma_f32_4x4x4_16b_f16 v[4:7], v[0:1], v[2:3], v[4:7]"
    assert dpp_violations(body(*pad, mfma, "s_nop 2", DPP))       # v5 written by the MFMA, 3 wait states
    assert dpp_violations(body(*pad, mfma, "s_nop 7", "s_nop 7", DPP))  # 16
    assert not dpp_violations(body(*pad, mfma, "s_nop 7", "s_nop 7", "s_nop 2", DPP))  # 19
    assert not dpp_violations(body(*pad, "v_mfma_f32_4x4x4_16b_f16 v[8:11], v[0:1], v[2:3], v[8:11]", DPP))
