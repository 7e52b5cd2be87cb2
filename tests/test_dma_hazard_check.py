"""The build's assembly check (csrc/check_dma_hazards.py) on small hand-written gfx950 listings:
a VALU write of an SGPR that an inline-asm LDS copy reads as its base fewer than 5 wait states
before it is flagged, on the straight path and through a branch into the copy's block; s_nop
wait states, SALU writes and copies without an SGPR base pass."""
import importlib.util
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "..", "lingbot-world-v2_amd", "csrc", "check_dma_hazards.py")
spec = importlib.util.spec_from_file_location("check_dma_hazards", PATH)
chk = importlib.util.module_from_spec(spec)
spec.loader.exec_module(chk)


def _run(tmp_path, body):
    p = tmp_path / "k.s"
    p.write_text("kernel:\n" + body)
    return chk.main([str(p)])


def test_readlane_right_before_the_copy_is_flagged(tmp_path):
    assert _run(tmp_path, """\
\tv_readlane_b32 s26, v214, 5
\ts_mov_b32 m0, s23
\tv_readlane_b32 s27, v214, 6
\tglobal_load_lds_dwordx4 v2, s[26:27]
\ts_endpgm
""") == 1


def test_five_wait_states_pass(tmp_path):
    assert _run(tmp_path, """\
\tv_readfirstlane_b32 s27, v3
\ts_nop 4
\tglobal_load_lds_dwordx4 v2, s[26:27]
\tv_readfirstlane_b32 s29, v3
\ts_mov_b32 m0, s1
\ts_add_u32 s5, s5, 1
\ts_add_u32 s6, s6, 1
\ts_add_u32 s7, s7, 1
\ts_add_u32 s8, s8, 1
\tglobal_load_lds_dwordx4 v2, s[28:29]
\ts_endpgm
""") == 0


def test_carry_output_and_other_registers(tmp_path):
    # a carry output into the base is a VALU write; a write of another SGPR is not
    assert _run(tmp_path, """\
\tv_mad_u64_u32 v[34:35], s[0:1], v33, s29, v[178:179]
\tglobal_load_lds_dwordx4 v34, s[0:1]
\ts_endpgm
""") == 1
    assert _run(tmp_path, """\
\tv_mad_u64_u32 v[34:35], s[8:9], v33, s29, v[178:179]
\tv_mov_b32_e32 v37, s7
\tglobal_load_lds_dwordx4 v34, s[6:7]
\tglobal_load_lds_dword v[4:5], off
\ts_endpgm
""") == 0


def test_hazard_through_a_branch(tmp_path):
    # the write sits before a branch to the copy's block; the fall-through path is clean
    body = """\
\tv_readfirstlane_b32 s11, v1
\ts_cbranch_scc1 .LBB0_2
\ts_nop 7
.LBB0_2:
\tglobal_load_lds_dwordx4 v2, s[10:11]
\ts_endpgm
"""
    assert _run(tmp_path, body) == 1
    assert _run(tmp_path, body.replace("\ts_cbranch_scc1 .LBB0_2\n", "\ts_nop 7\n\ts_cbranch_scc1 .LBB0_2\n")) == 0


def test_every_source_with_inline_asm_copies_is_checked_by_the_build():
    """Every kernel source that issues the inline-asm LDS copies (dma16 / dma4, or the
    instruction itself) has its assembly in the Makefile's ASMS list, so the build checks it."""
    import re
    csrc = os.path.join(HERE, "..", "lingbot-world-v2_amd", "csrc")
    mk = open(os.path.join(csrc, "Makefile")).read()
    asms = re.search(r"^ASMS\s*:=(.*)$", mk, re.M).group(1)
    checked = set(re.findall(r"(\w+)\.s\b", asms))
    users = set()
    for f in os.listdir(csrc):
        if f.endswith(".hip"):
            src = open(os.path.join(csrc, f)).read()
            if re.search(r"\bdma16(_guarded)?\s*\(|\bdma4\s*\(|global_load_lds", src):
                users.add(f[:-4])
    assert users, "no source issues the copies: the pattern is stale"
    assert users <= checked, f"not checked by the build: {sorted(users - checked)}"
