"""The build's device-assembly check for inline-asm loads
(barq-inference_amd/csrc/isa_check_asm_loads.py): it accepts code that leaves
the asm-loaded registers alone until the vmcnt wait, flags a read or a write
of one of them before it, and passes on the library's own built assembly."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "barq-inference_amd", "csrc")
CHECK = os.path.join(CSRC, "isa_check_asm_loads.py")

GOOD = """_Zk:
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[10:11], off offset:4
\t;;#ASMEND
\t;;#ASMSTART
\tglobal_load_dword v30, v[2:3], off
\t;;#ASMEND
\t;;#ASMSTART
\ts_mov_b32 m0, s2
\tbuffer_load_dwordx4 v25, s[4:7], s3 offen nt lds
\t;;#ASMEND
\tv_add_u32_e32 v12, v13, v14
\ts_waitcnt vmcnt(1)
\tv_add_u32_e32 v12, v6, v30
\ts_endpgm
"""

# a runtime switch over the wait count (as wait_vmcnt_upto8 compiles), two
# copies issued after the asm load, then a constant covering wait
SWITCH = """_Zk:
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[10:11], off offset:4
\t;;#ASMEND
\t;;#ASMSTART
\ts_mov_b32 m0, s2
\tbuffer_load_dwordx4 v25, s[4:7], s3 offen nt lds
\t;;#ASMEND
\t;;#ASMSTART
\ts_mov_b32 m0, s2
\tbuffer_load_dwordx4 v26, s[4:7], s3 offen nt lds
\t;;#ASMEND
\ts_cmp_eq_u32 s7, 0
\ts_cbranch_scc1 .LBB0_2
\ts_waitcnt vmcnt(8)
\ts_branch .LBB0_3
.LBB0_2:
\ts_waitcnt vmcnt(0)
.LBB0_3:
\ts_waitcnt vmcnt(2)
\tv_add_u32_e32 v12, v6, v7
\ts_endpgm
"""


def run(tmp_path, text):
    p = tmp_path / "k.s"
    p.write_text(text)
    return subprocess.run([sys.executable, CHECK, str(p)], capture_output=True, text=True).returncode


def test_accepts_untouched_registers(tmp_path):
    assert run(tmp_path, GOOD) == 0


@pytest.mark.parametrize("planted", ["v_add_u32_e32 v12, v13, v8",     # reads a pending register
                                     "v_mov_b32_e32 v30, 0",           # writes one
                                     "v_pk_add_u16 v[12:13], v[5:6], v1"])   # a range that overlaps
def test_flags_a_touched_register(tmp_path, planted):
    assert run(tmp_path, GOOD.replace("v_add_u32_e32 v12, v13, v14", planted)) == 1


def test_library_assembly_passes():
    files = sorted(glob.glob(os.path.join(CSRC, "_build", "*.hip.s")))
    if not files:
        pytest.skip("device assembly not built")
    r = subprocess.run([sys.executable, CHECK] + files, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_accepts_a_switch_closed_by_a_covering_wait(tmp_path):
    assert run(tmp_path, SWITCH) == 0


ASM_V30 = "\t;;#ASMSTART\n\tglobal_load_dword v30"


@pytest.mark.parametrize("text", [
    # a use between two asm loads of a run
    GOOD.replace(ASM_V30, "\tv_mov_b32_e32 v7, 0\n" + ASM_V30),
    # an asm load after an lgkmcnt-only wait is still tracked
    GOOD.replace(ASM_V30, "\ts_waitcnt lgkmcnt(0)\n" + ASM_V30).replace("vmcnt(1)", "vmcnt(3)"),
    # a wait that leaves the youngest asm load outstanding (one load after it)
    GOOD.replace("vmcnt(1)", "vmcnt(2)"),
    # a pending register reused as a copy's offset
    GOOD.replace("buffer_load_dwordx4 v25,", "buffer_load_dwordx4 v8,"),
    # one side of a branch reaches the use without a covering wait
    SWITCH.replace("\ts_waitcnt vmcnt(2)\n\tv_add", "\tv_add"),
], ids=["between_loads", "after_lgkmcnt_wait", "uncovered_wait", "as_copy_offset", "branch_path"])
def test_flags_the_unsafe_shapes(tmp_path, text):
    assert run(tmp_path, text) == 1
