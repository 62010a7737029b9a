"""Self-test of the host emulator's lane scheduling (tests/emu/emu.hpp), on
which every emulation test relies: lanes run as cooperative fibers that
switch only at block barriers and wave exchanges.  A kernel with both gives
its known result; a wave exchange reached by only part of a wave (a shuffle
on one half, a readfirstlane on the other) is reported; lanes that wait at
barriers the others never reach stop the run with a message, not a hang."""
import os
import subprocess

import pytest

EMU = os.path.join(os.path.dirname(os.path.abspath(__file__)), "emu")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.fixture(scope="module")
def selftest(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ not found")
    exe = tmp_path_factory.mktemp("emu_selftest") / "selftest"
    subprocess.run([CLANG, "-O1", "-std=c++20", "-pthread", "-Wno-psabi", "-I", EMU,
                    os.path.join(EMU, "selftest_main.cpp"), "-o", str(exe)], check=True)
    return str(exe)


def _run(exe, mode):
    r = subprocess.run([exe, mode], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout + r.stderr


def test_barriers_and_shuffles_give_the_known_sum(selftest):
    rc, out = _run(selftest, "ok")
    assert rc == 0 and "result mismatches 0" in out and "errors 0" in out, out


def test_divergent_wave_exchange_is_reported(selftest):
    rc, out = _run(selftest, "div_shuffle")
    assert rc == 0, out
    assert "a wave exchange under divergent control flow" in out, out


def test_divergent_barrier_stops_the_run(selftest):
    rc, out = _run(selftest, "deadlock")
    assert rc != 0, out
    assert "every live lane waits at a barrier the others never reach" in out, out
