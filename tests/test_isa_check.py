"""The build-time hazard check of inline-assembly MFMAs and DPP reads (h3metal_amd/isa_check.py) on small hand-written
assembly listings: each hazard it exists for is reported, and the patterns it must accept (enough wait states,
back-to-back accumulation onto the same registers) are not."""

from h3metal_amd.isa_check import XDL_WAIT, scan

ASM_MFMA = """;;#ASMSTART
v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]
;;#ASMEND"""


def listing(*lines):
    return "\n".join(["kern:"] + list(lines))


def test_valu_read_of_a_pending_accumulator_is_reported():
    bad = scan(listing(ASM_MFMA, "v_accvgpr_read_b32 v8, a3"))
    assert len(bad) == 1 and "a', 3" in bad[0]


def test_enough_wait_states_clear_the_accumulator():
    assert XDL_WAIT == 18  # a 16-pass XDL result, read or overwritten by another instruction
    # s_nop N is N + 1 wait states
    assert scan(listing(ASM_MFMA, "s_nop 7", "s_nop 7", "s_nop 1", "v_accvgpr_read_b32 v8, a3")) == []
    assert scan(listing(ASM_MFMA, *(["v_add_f32 v9, v9, v9"] * XDL_WAIT), "v_accvgpr_read_b32 v8, a3")) == []
    # one wait state short
    assert len(scan(listing(ASM_MFMA, "s_nop 7", "s_nop 7", "s_nop 0", "v_accvgpr_read_b32 v8, a3"))) == 1
    assert len(scan(listing(ASM_MFMA, *(["v_add_f32 v9, v9, v9"] * (XDL_WAIT - 1)),
                            "v_accvgpr_read_b32 v8, a3"))) == 1


def test_back_to_back_accumulation_is_accepted():
    same = "v_mfma_f32_32x32x16_bf16 a[0:15], v[8:11], v[12:15], a[0:15]"
    assert scan(listing(ASM_MFMA, same)) == []
    assert scan(listing(ASM_MFMA, ";;#ASMSTART", same, ";;#ASMEND", same)) == []


def test_other_reads_of_a_pending_accumulator_are_reported():
    # another opcode accumulating onto it, a partial overlap of srcC, the accumulator as a multiplicand
    other = "v_mfma_f32_32x32x8_f16 a[0:15], v[8:9], v[10:11], a[0:15]"
    part = "v_mfma_f32_32x32x16_bf16 a[16:31], v[8:11], v[12:15], a[8:23]"
    mult = "v_mfma_f32_32x32x16_bf16 a[16:31], a[0:3], v[12:15], a[16:31]"
    for line in (other, part, mult):
        assert len(scan(listing(ASM_MFMA, line))) == 1, line


def test_valu_write_just_before_an_mfma_operand_is_reported():
    w = "v_mov_b32 v5, 0"
    mfma = "v_mfma_f32_32x32x16_bf16 a[32:47], v[0:3], v[4:7], a[32:47]"
    assert len(scan(listing(w, mfma))) == 1
    assert len(scan(listing(w, "s_nop 0", mfma))) == 1
    assert scan(listing(w, "s_nop 1", mfma)) == []


def test_a_new_function_starts_clean():
    assert scan(listing(ASM_MFMA) + "\nother_kern:\nv_accvgpr_read_b32 v8, a3") == []


def test_valu_write_just_before_a_dpp_read_is_reported():
    w = "v_fmac_f32_e32 v1, v2, v3"
    dpp = "v_fmac_f32_dpp v1, v1, v9 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1"
    assert len(scan(listing(w, dpp))) == 1
    assert len(scan(listing(w, "s_nop 0", dpp))) == 1
    assert scan(listing(w, "s_nop 1", dpp)) == []
    # two independent instructions in between are two wait states as well
    assert scan(listing(w, "v_add_f32 v5, v6, v7", "v_add_f32 v5, v6, v7", dpp)) == []
    # only the DPP operand (src0) counts: the other source may be written just before
    assert scan(listing("v_mov_b32 v9, 0", dpp)) == []
    # four DPP fmacs after one s_nop 1, each on its own value (the form the row kernels use)
    block = ["s_nop 1"] + [f"v_fmac_f32_dpp v{i}, v{i}, v9 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1"
                           for i in range(1, 5)]
    assert scan(listing(*[f"v_add_f32 v{i}, v{i}, v{i}" for i in range(1, 5)], *block)) == []
