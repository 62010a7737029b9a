"""CPU checks of the built library's gfx950 code: no LDS DMA after a too-recent
M0 write, no VMEM read of a freshly VALU-written SGPR, no VGPR touched while
a load into it is in flight (the scanner's docstring states each rule)."""
import os
import re

import pytest

from isa_scan import code_objects, disassemble, scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "xstar-infer_amd", "xstar_cpp_py", "libxs_moe.so")


@pytest.fixture(scope="module")
def disasm(tmp_path_factory):
    if not os.path.exists(SO):
        pytest.skip("libxs_moe.so not built")
    if not os.path.exists("/opt/rocm/llvm/bin/llvm-objdump"):
        pytest.skip("no llvm-objdump")
    work = tmp_path_factory.mktemp("co")
    return [disassemble(c) for c in code_objects(SO, str(work))]


def test_library_has_the_gemm_code(disasm):
    text = "\n".join(disasm)
    assert len(disasm) >= 8                                  # one code object per HIP source
    assert text.count("global_load_lds_dwordx4") > 1000      # the LDS-ring GEMMs' DMAs
    assert re.search(r"v_mfma_\w*f8", text)                  # FP8 MFMA


def test_no_wait_state_or_inflight_register_hazards(disasm):
    found = [f for t in disasm for f in scan(t)]
    assert not found, "\n".join(map(str, found[:20]))


def test_scanner_flags_planted_hazards():
    """Each rule fires on a minimal planted case and stays quiet when the wait is there."""
    m0 = "\ts_mov_b32 m0, s4\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n"
    assert [f[0] for f in scan(m0)] == ["m0"]
    assert scan("\ts_mov_b32 m0, s4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n") == []
    sg = "\tv_readfirstlane_b32 s6, v3\n\ts_nop 2\n\tglobal_load_dwordx4 v[4:7], v1, s[6:7]\n"
    assert [f[0] for f in scan(sg)] == ["sgpr"]
    assert scan(sg.replace("s_nop 2", "s_nop 4")) == []
    late = "\tglobal_load_dwordx4 v[8:11], v[2:3], off\n\tv_mov_b32_e32 v9, 0\n"
    assert [f[0] for f in scan(late)] == ["vmem"]
    waited = "\tglobal_load_dwordx4 v[8:11], v[2:3], off\n\ts_waitcnt vmcnt(0)\n\tv_mov_b32_e32 v9, 0\n"
    assert scan(waited) == []
    # a second load into the same register lands after the first (in-order return)
    assert scan("\tglobal_load_dword v8, v[2:3], off\n\tglobal_load_dword v8, v[4:5], off\n") == []
    # but a load whose address register is still being loaded into is flagged
    assert [f[0] for f in scan("\tglobal_load_dwordx2 v[2:3], v[4:5], off\n\tglobal_load_dword v8, v[2:3], off\n")] == ["vmem"]
    # vmcnt(1) retires the older of two loads only
    two = ("\tglobal_load_dwordx4 v[8:11], v[2:3], off\n\tglobal_load_dwordx4 v[12:15], v[2:3], off\n"
           "\ts_waitcnt vmcnt(1)\n\tv_add_f32_e32 v8, v8, v8\n\tv_add_f32_e32 v12, v12, v12\n")
    assert [(f[0], f[2].split()[1]) for f in scan(two)] == [("vmem", "v12,")]


def test_scanner_follows_branches_and_back_edges():
    """A load in flight is followed over the control-flow graph: into a branch
    target, and around a loop's back edge into the next iteration."""
    branch = ("\tglobal_load_dwordx4 v[8:11], v[2:3], off\n\ts_cbranch_scc1 L1\n"
              "\ts_waitcnt vmcnt(0)\n\ts_branch L2\n"
              "L1:\n\tv_add_f32_e32 v9, v9, v9\n"
              "L2:\n\ts_endpgm\n")
    assert [(f[0], f[2].split()[0]) for f in scan(branch)] == [("vmem", "v_add_f32_e32")]
    # both paths wait before the join: nothing in flight there
    joined = branch.replace("L1:\n\tv_add", "L1:\n\ts_waitcnt vmcnt(0)\n\tv_add")
    assert scan(joined) == []
    # the load of one iteration is still in flight at the top of the next
    loop = ("L0:\n\tv_mov_b32_e32 v12, 0\n\tglobal_load_dword v12, v[2:3], off\n"
            "\ts_cbranch_scc1 L0\n\ts_waitcnt vmcnt(0)\n\ts_endpgm\n")
    assert [f[0] for f in scan(loop)] == ["vmem"]
    assert scan(loop.replace("\ts_cbranch_scc1 L0\n", "\ts_waitcnt vmcnt(0)\n\ts_cbranch_scc1 L0\n")) == []
    # the paths are aligned from the newest load: vmcnt(1) on the join retires
    # the older load of the longer path only
    two = ("\tglobal_load_dword v8, v[2:3], off\n\ts_cbranch_scc1 L1\n"
           "\tglobal_load_dword v9, v[2:3], off\n"
           "L1:\n\ts_waitcnt vmcnt(1)\n\tv_mov_b32_e32 v8, 0\n\tv_mov_b32_e32 v9, 0\n")
    assert [(f[0], f[2].split()[1]) for f in scan(two)] == [("vmem", "v8,"), ("vmem", "v9,")]
    # an M0 write at the end of the fall-through predecessor counts for a DMA
    # at a branch target
    m0 = "\ts_cbranch_scc1 L1\n\ts_mov_b32 m0, s4\nL1:\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n"
    assert [f[0] for f in scan(m0)] == ["m0"]
    assert scan(m0.replace("s4\n", "s4\n\ts_nop 0\n")) == []
