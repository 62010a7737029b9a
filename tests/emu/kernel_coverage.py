"""Kernel instantiations of the built library against those an emulated run
launched (EMU_KERNEL_LOG=<file>: every kernel emulated through gen_fwd.py
notes its __PRETTY_FUNCTION__ once per launch).

usage: kernel_coverage.py <libxs_moe.so> <log>   prints the missing ones.
The library's list comes from its gfx950 code objects' kernel descriptors
(<name>.kd symbols), demangled; both sides are reduced to name<args>."""
import os
import re
import subprocess
import sys
import tempfile

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "xstar-infer_amd"))
from isa_scan import code_objects  # noqa: E402


def library_kernels(so):
    syms = set()
    with tempfile.TemporaryDirectory() as d:
        for co in code_objects(so, d):
            out = subprocess.run(["/opt/rocm/llvm/bin/llvm-objdump", "-t", co], capture_output=True, text=True,
                                 check=True).stdout
            syms.update(m.group(1) for m in re.finditer(r"(\S+)\.kd$", out, re.M))
    dem = subprocess.run(["c++filt"], input="\n".join(sorted(syms)), capture_output=True, text=True,
                         check=True).stdout.splitlines()
    out = set()
    for s in dem:
        m = re.search(r"(\w+)<(.*)>\(", s)
        out.add(m.group(1) + "<" + m.group(2).replace(" ", "") + ">" if m else re.search(r"(\w+)\(", s).group(1))
    return out


def launched(log):
    out = set()
    for line in open(log):
        if "(" not in line:
            continue
        name = re.search(r"(\w+)\(", line).group(1)
        b = re.search(r"\[(.*)\]\s*$", line.strip())
        if b:
            vals = [v.split(" = ", 1)[1].replace(" ", "") for v in re.split(r", (?=\w+ = )", b.group(1))]
            name += "<" + ",".join(vals) + ">"
        out.add(name)
    return out


if __name__ == "__main__":
    lib, hit = library_kernels(sys.argv[1]), launched(sys.argv[2])
    print(f"{len(lib)} kernels in the library, {len(lib & hit)} launched")
    for k in sorted(lib - hit):
        print("missing", k)
