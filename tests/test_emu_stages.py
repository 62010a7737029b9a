"""Host emulation of the stage entry points of the C ABI, the CPU
counterpart of tests/test_gpu_stages.py: each call runs the library's own
launcher and kernel source on the CPU (tests/emu/stages_main.cpp over the
objects of tests/emu/gen_fwd.py) and is compared with the CPU oracle.

- activation quant, FP8 1x128 and MXFP8, bf16 and f32 input: bit for bit;
- weight quant, FP8 128x128 blocks and MXFP4, batched: bit for bit;
- the codec inputs cover many binades, zero values and zero groups, values
  at e4m3 / e2m1 rounding ties after scaling, and near-overflow values;
- RMSNorm: within 2 bf16 codes of the oracle's sequential sum (f32: the
  summation-order bound), and its fused FP8 quant equal, bit for bit, to the
  quantization of its own output, for every chunk count of the one-wave-per-row
  kernel (hidden 512..8192) and for the block kernel (hidden above 8192, not a
  multiple of 8, misaligned rows);
- route: plain, exact ties, group-limited, E not a multiple of 64, E = 1024
  with top-16, E = 1, scaling, with and without renormalisation and bias:
  indices and weights bit for bit;
- permute: counts, offsets, permutation and inverse bit for bit from 1 to
  2000 tokens, and the two rejections (an expert named twice in a row, an
  index out of range) with their messages;
- router logits with the chain router, bf16 and f32: gemm_cpu's bits;
- the single FP8 GEMM (gemm_dense.hip), split-K with its partial-tile
  exchange and whole-K: within 4e-3 of float64 on the dequantized operands,
  and the same bits on a second call."""
import os
import re
import subprocess

import pytest

EMU = os.path.join(os.path.dirname(os.path.abspath(__file__)), "emu")


@pytest.fixture(scope="module")
def stages_emu(emu_fwd_lib, tmp_path_factory):
    from conftest import emu_link
    return emu_link(emu_fwd_lib, os.path.join(EMU, "stages_main.cpp"), tmp_path_factory.mktemp("stages") / "stages")


SEEDS = [1, 2, 3]


@pytest.fixture(scope="module")
def stage_runs(stages_emu):
    """The three seeds' runs at once: {seed: (returncode, output)}."""
    from concurrent.futures import ThreadPoolExecutor

    def one(seed):
        r = subprocess.run([stages_emu, str(seed)], capture_output=True, text=True, timeout=600)
        return r.returncode, r.stdout + r.stderr

    with ThreadPoolExecutor(len(SEEDS)) as ex:
        return dict(zip(SEEDS, ex.map(one, SEEDS)))


@pytest.mark.parametrize("seed", SEEDS)
def test_stages_emulated(stage_runs, seed):
    rc, out = stage_runs[seed]
    assert rc == 0, out[-3000:]
    assert re.search(r"^errors 0$", out, re.M), out[-3000:]
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"^(.+?) mismatches (\d+)$", out, re.M)}
    assert len(c) == 14 and all(v == 0 for v in c.values()), out
    assert "permute errors ok" in out, out
