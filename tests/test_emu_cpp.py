"""Host emulation of the C++ Tensor ops, the reference-idiom boundary
(csrc/src: tensor.cpp, ops/moe.cpp, ops/rmsnorm.cpp, ops/moe_weights.cpp,
weight_io.cpp, mmap_file.cpp), linked against the emulated library: the ops
call the library's C ABI as on the card, and every kernel runs from its
source on the CPU (tests/emu/cpp_main.cpp).  The CPU counterpart of the
compute parts of tests/test_cpp_moe.py and tests/test_gpu_weights.py:

- moe() equals xs_moe_forward on the same buffers bit for bit, routes like
  the reference's gemm_cpu logits, and stays within 2e-2 of the oracle's
  layer: FP8 with the shared expert, f32 input, the pre-norm with a
  residual, MXFP4 routed experts;
- load_moe_layer on a two-file FP8 checkpoint (DeepSeek-style names, gate
  and up stacked into w13) returns exactly what was written, and
  moe_block_ffn on it equals moe() with the norm and residual bit for bit;
- a dense BF16 checkpoint is quantized while loading exactly as the oracle's
  128x128 block quantization, an all-zero block included;
- rmsnorm(), moe_router_logits(exact), moe_route() (groups, scaling, no
  renormalisation) and moe_permute() equal the C ABI / oracle bit for bit."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "xstar-infer_amd", "csrc")


@pytest.fixture(scope="module")
def cpp_emu(emu_fwd_lib, tmp_path_factory):
    from conftest import EMU_CLANG, EMU_FLAGS
    inc, objs, link = emu_fwd_lib
    srcs = [os.path.join(CSRC, "src", f) for f in ("tensor.cpp", "mmap_file.cpp", "weight_io.cpp")]
    srcs += [os.path.join(CSRC, "src", "ops", f) for f in ("moe.cpp", "moe_weights.cpp", "rmsnorm.cpp")]
    exe = tmp_path_factory.mktemp("cpp_emu") / "cpp_emu"
    subprocess.run([EMU_CLANG, *EMU_FLAGS, *inc, "-I", os.path.join(CSRC, "include"),
                    os.path.join(ROOT, "tests", "emu", "cpp_main.cpp"), *srcs, *objs, "-o", str(exe), *link],
                   check=True)
    return str(exe)


def test_cpp_ops_emulated(cpp_emu, tmp_path):
    r = subprocess.run([cpp_emu, str(tmp_path)], capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert re.search(r"^errors 0$", out, re.M), out[-3000:]
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"^(.+?) mismatches (\d+)$", out, re.M)}
    assert len(c) == 12 and all(v == 0 for v in c.values()), out
