"""Builds the MoE operator in-tree.

  xstar_cpp_py/libxs_moe.so   HIP kernels + C ABI (include/xs_moe.h), hipcc for gfx950
  xstar_cpp_py/xstar_cpp*.so  pybind11 module: Tensor + ops (g++, links libxs_moe.so)

Usage: python xstar-infer_amd/build.py [--only hip|py]
"""
from __future__ import annotations

import argparse
import glob
import os
import re
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "xstar_cpp_py")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed FP32 instructions are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    # MFMA results in VGPRs: the FP8 kernels fold every partial product with VALU FMAs
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # atomics stay as written: the wave-aggregating rewrite reads an atomic's
    # result right after issuing it, which would stall the persistent GEMMs'
    # scheduler wave (it reads a claim several steps later)
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def _run(cmd):
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _scratch_users(remarks: str):
    """Kernels whose resource-usage remarks report scratch (register spills)."""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            bad.append((name, int(m.group(1))))
    return bad


def _hazards(so_path):
    """isa_scan over every code object of the library (empty: none found)."""
    import tempfile

    sys.path.insert(0, HERE)
    from isa_scan import code_objects, disassemble, scan

    with tempfile.TemporaryDirectory() as d:
        return [f for co in code_objects(so_path, d) for f in scan(disassemble(co))]


def build_hip() -> str:
    os.makedirs(OUT, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "hip", "*.hip")))
    out = os.path.join(OUT, "libxs_moe.so")
    tmp = out + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(HERE, "csrc", "hip"), *srcs, "-o", tmp, "-Wl,-soname,libxs_moe.so"]
    print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        print("\n".join(l for l in r.stdout.splitlines() if "remark:" not in l), flush=True)
        raise subprocess.CalledProcessError(r.returncode, cmd)
    # every kernel keeps its state in registers: a spill to scratch fails the build
    bad = _scratch_users(r.stdout)
    if bad:
        os.remove(tmp)
        raise RuntimeError("kernels spill to scratch: " + ", ".join(f"{n} ({b} B/lane)" for n, b in bad))
    # the asm-level wait-state and in-flight-register checks over the machine code
    found = _hazards(tmp)
    if found:
        os.remove(tmp)
        raise RuntimeError("machine-code hazards: " + "; ".join(map(str, found[:10])))
    os.replace(tmp, out)
    return out


def build_py() -> str:
    import pybind11

    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "src", "**", "*.cpp"), recursive=True))
    srcs.append(os.path.join(HERE, "csrc", "bindings", "python_bindings.cpp"))
    ext = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(OUT, "xstar_cpp" + ext)
    tmp = out + ".tmp"
    inc = [pybind11.get_include(), sysconfig.get_paths()["include"], os.path.join(ROOT, "include"),
           os.path.join(HERE, "csrc", "include")]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
          *[f"-I{i}" for i in inc], *srcs, "-o", tmp, f"-L{OUT}", "-lxs_moe",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["hip", "py"], default=None)
    a = ap.parse_args(argv)
    if a.only in (None, "hip"):
        build_hip()
    if a.only in (None, "py") and os.path.exists(os.path.join(HERE, "csrc", "bindings", "python_bindings.cpp")):
        build_py()


if __name__ == "__main__":
    sys.exit(main())
