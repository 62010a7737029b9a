"""Host emulation of the weight-direct GEMMs: FP8 prefill (moe_gemm_wd.hip),
FP8 decode (moe_gemm_wdd.hip) and MXFP4 (moe_gemm_wd4.hip).

Each kernel's own source runs on the CPU with one thread per lane: each LDS DMA
poisons its destination and lands only when the kernel's vmcnt wait retires it
in issue order (register loads count in the same queue), every global and LDS
address is checked against its buffer, and scalar operands are checked to be
wave-uniform.  The outputs are compared with a float64 recomputation of the
layer from the same FP8 inputs.  This is the CPU check of the kernel's
indexing, ring waits and bounds; the GPU tests check its results on the card."""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EMU = os.path.join(ROOT, "tests", "emu")
HIP = os.path.join(ROOT, "xstar-infer_amd", "csrc", "hip")
CLANG = "/opt/rocm/llvm/bin/clang++"


def _build(d, gen, src, main):
    inc = {"gen_wd.py": "wd_emu.inc", "gen_wdd.py": "wdd_emu.inc", "gen_wd4.py": "wd4_emu.inc"}[gen]
    subprocess.run([sys.executable, os.path.join(EMU, gen), os.path.join(HIP, src),
                    os.path.join(HIP, "moe_gemm.hpp"), str(d / inc)], check=True, cwd=EMU)
    # the references of the bit-identity checks: the tiled kernel of
    # moe_gemm.hip and the tall-tile LDS-ring kernel of moe_gemm_wide.hip
    subprocess.run([sys.executable, os.path.join(EMU, "gen_tiled.py"), os.path.join(HIP, "moe_gemm.hip"),
                    str(d / "tiled_emu.inc")], check=True, cwd=EMU)
    subprocess.run([sys.executable, os.path.join(EMU, "gen_wide.py"), os.path.join(HIP, "moe_gemm_wide.hip"),
                    str(d / "wide_emu.inc")], check=True, cwd=EMU)
    exe = d / main.replace(".cpp", "")
    subprocess.run([CLANG, "-O2", "-std=c++20", "-pthread", "-Wno-psabi", "-I", EMU, "-I", str(d),
                    "-I", os.path.join(ROOT, "include"), os.path.join(EMU, main), "-o", str(exe)], check=True)
    return str(exe)


@pytest.fixture(scope="module")
def emu_dir(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ not found")
    d = tmp_path_factory.mktemp("emu")
    yield d
    shutil.rmtree(d, ignore_errors=True)


@pytest.fixture(scope="module")
def wd_emu(emu_dir):
    return _build(emu_dir, "gen_wd.py", "moe_gemm_wd.hip", "wd_main.cpp")


@pytest.fixture(scope="module")
def wdd_emu(emu_dir):
    return _build(emu_dir, "gen_wdd.py", "moe_gemm_wdd.hip", "wdd_main.cpp")


@pytest.fixture(scope="module")
def wd4_emu(emu_dir):
    return _build(emu_dir, "gen_wd4.py", "moe_gemm_wd4.hip", "wd4_main.cpp")


def _check(out, returncode):
    assert returncode == 0 and "errors 0" in out, out[-3000:]
    act = float(re.search(r"gate_up act: .* rel (\S+)", out).group(1))
    y = float(re.search(r"down y: .* rel (\S+)", out).group(1))
    # gate_up's output is SwiGLU requantised to e4m3 (3 mantissa bits): at most
    # half a step, 2^-4 of the value, per element
    assert act < 0.0625, out[-2000:]
    # down is f32 accumulation of exact FP8 products
    assert y < 1e-5, out[-2000:]


def test_weight_direct_gemms_emulated(wd_emu):
    # 64 tokens, 4 experts top-2, Zipf(1.1), shared expert, H=1024, I=512 (the
    # smallest shape the kernel takes: K a multiple of 512, grid x of 4): full,
    # partial and short tiles; DMAs land at their waits, not at issue
    r = subprocess.run([wd_emu, "64", "4", "2", "1.1", "3", "1024", "512", "4", "0", "1", "1"],
                       capture_output=True, text=True, timeout=900,
                       env=dict(os.environ, EMU_CMP_WIDE="1", EMU_CMP_SHARED="1"))
    out = r.stdout + r.stderr
    _check(out, r.returncode)
    # the tall-tile LDS-ring kernel (192-row tiles) on the same inputs writes
    # the same bytes: the same per-row arithmetic in the same order; so does
    # the shared segment run alone, in 128-row tiles the kernel computes itself
    assert "tall-tile kernel: errors 0, identical bytes: yes" in out, out[-2000:]
    assert "shared segment alone: errors 0, identical bytes: yes" in out, out[-2000:]


@pytest.mark.parametrize("args,pd", [
    # 16 tokens, 32 experts top-4 + shared, H=1024, I=512: one tile per expert
    # (the launcher's prefetch depth: 8 steps)
    (["16", "32", "4", "0", "5", "1024", "512"], None),
    # 40 tokens, 8 experts top-2, Zipf(1.1), no shared expert, H=512, I=1024:
    # experts of several 16-row tiles, ragged last tiles; 4-step prefetch
    (["40", "8", "2", "1.1", "6", "512", "1024"], "4"),
])
def test_weight_direct_decode_gemms_emulated(wdd_emu, args, pd):
    shared = "0" if args[0] == "40" else "1"
    env = dict(os.environ, EMU_CMP_TILED="1")
    if pd:
        env["EMU_WDD_PD"] = pd
    r = subprocess.run([wdd_emu, *args, "8", "0", "1", shared], capture_output=True, text=True, timeout=900,
                       env=env)
    out = r.stdout + r.stderr
    _check(out, r.returncode)
    # the 16-row tiled kernel on the same inputs writes the same bytes: the
    # MFMAs get the same operands and the folds run in the same order
    assert "identical bytes: yes" in out, out[-2000:]


@pytest.mark.parametrize("mode", ["0", "1"])
def test_weight_direct_mxfp4_gemms_emulated(wd4_emu, mode):
    # 64 tokens, 4 experts top-2, Zipf(1.1), 64-row tiles, H=1024, I=512 (the
    # loop form); MXFP4 weights, MXFP8 activations, e8m0 scales.  Mode 0 lands
    # each DMA at its wait (a read before its wait sees poison), mode 1 at issue
    # (a refill of a ring slot that a wave still reads corrupts that read).
    r = subprocess.run([wd4_emu, "64", "4", "2", "1.1", "3", "1024", "512", "4", mode, "1", "64"],
                       capture_output=True, text=True, timeout=900, env=dict(os.environ, EMU_CMP_TILED="1"))
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "errors 0" in out, out[-3000:]
    # the 64-row MXFP4 tiled kernel on the same inputs writes the same bytes
    assert "identical bytes: yes" in out, out[-2000:]
    # every act element within the bound its block's e8m0 scale sets: the
    # clamp at 448 x 2^se, else half an e4m3 step
    assert int(re.search(r"outside the MXFP8 bound (\d+)", out).group(1)) == 0, out[-2000:]
    assert float(re.search(r"down y: .* rel (\S+)", out).group(1)) < 1e-5, out[-2000:]


def test_emulated_check_catches_misdirected_dma(wd_emu):
    # the same case with the M0 wait-state hazard modelled (1% of DMAs land at
    # the previous DMA's LDS destination): the check above must then fail
    env = dict(os.environ, EMU_HAZARD="1", EMU_HAZARD_P="0.01", EMU_HAZARD_SEED="7")
    r = subprocess.run([wd_emu, "64", "4", "2", "1.1", "3", "1024", "512", "4", "0", "1", "1"],
                       capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    hits = int(re.search(r"hazard hits (\d+)", out).group(1))
    assert hits > 0, out[-2000:]
    m_act = re.search(r"gate_up act: .* rel (\S+)", out)
    m_y = re.search(r"down y: .* rel (\S+)", out)
    act = float(m_act.group(1)) if m_act else float("inf")
    y = float(m_y.group(1)) if m_y else float("inf")
    assert r.returncode != 0 or not (act < 0.0625 and y < 1e-5), out[-2000:]
