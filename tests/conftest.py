import os
import sys

import pytest


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "xstar-infer_amd")
for p in (ROOT, PKG, os.path.join(PKG, "xstar_cpp_py")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running")


EMU_CLANG = "/opt/rocm/llvm/bin/clang++"
EMU_FLAGS = ["-O1", "-std=c++20", "-pthread", "-Wno-psabi", "-ffp-contract=off"]


@pytest.fixture(scope="session")
def emu_fwd_lib(tmp_path_factory):
    """The library's own HIP sources compiled for the host emulator
    (tests/emu/gen_fwd.py): (include flags, object files, link flags) for a
    driver that calls the C ABI with every kernel run on the CPU."""
    import shutil
    import subprocess
    if not os.path.exists(EMU_CLANG):
        pytest.skip("clang++ not found")
    import oracle
    oracle.lib()          # builds oracle/_build/liboracle.so if needed
    emu = os.path.join(ROOT, "tests", "emu")
    d = tmp_path_factory.mktemp("fwd_lib")
    subprocess.run([sys.executable, os.path.join(emu, "gen_fwd.py"), os.path.join(PKG, "csrc", "hip"), str(d)],
                   check=True, cwd=emu)
    inc = ["-I", str(d), "-I", emu, "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle")]
    srcs = sorted(f for f in os.listdir(d) if f.endswith(".cpp"))
    procs = [subprocess.Popen([EMU_CLANG, *EMU_FLAGS, *inc, "-c", str(d / f), "-o", str(d / (f[:-4] + ".o"))])
             for f in srcs]
    assert all(p.wait() == 0 for p in procs)
    build = os.path.join(ROOT, "oracle", "_build")
    yield inc, [str(d / (f[:-4] + ".o")) for f in srcs], ["-L", build, "-loracle", f"-Wl,-rpath,{build}"]
    shutil.rmtree(d, ignore_errors=True)


def emu_link(lib, main_src, exe):
    """Links a driver (a .cpp under tests/emu) against emu_fwd_lib's objects."""
    import subprocess
    inc, objs, link = lib
    subprocess.run([EMU_CLANG, *EMU_FLAGS, *inc, main_src, *objs, "-o", str(exe), *link], check=True)
    return str(exe)
