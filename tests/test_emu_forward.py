"""Host emulation of the whole default forward: the library's own C ABI
(xs_moe_forward, xs_moe_forward_noalloc, xs_moe_plan), dispatch, workspace
layout and launchers compiled for the host, with every kernel launch running
the kernel's source on the CPU (tests/emu/gen_fwd.py, hip_emu.hpp; one fiber
per lane, DMAs landing at their waits, addresses checked against their
buffers, every wave exchange checked to be reached by all live lanes).

Each case runs one forward on a poisoned workspace and compares against the
CPU oracle: routing, weights, counts, offsets, permutation and inverse bit
for bit against the oracle's routing of the logits the forward routed on;
the top-k against the oracle's routing from x for the certified and chain
routers (and the logits bit for bit for the chain router); the output within
the layer's 2e-2 bound of the oracle's dequantize-then-f32 layer.  With the
pre-norm the oracle runs on xs_rmsnorm's output (as the GPU test does), and
that row is checked within 2 bf16 codes (f32: the summation-order bound of
2H + 8 ulps) of the oracle's norm, whose sequential sum can differ from the
kernel's by an ulp of inv.  The cases
cover each GEMM family of the default dispatch: one-block-per-tile, the
persistent stream-K kernels, the tall tiles with the separate and the fused
combine, MXFP4 routed experts, the pre-norm with a residual, the
no-allocation entry point, f32 inputs, E = 1024 with top-16, group-limited
routing with scaling and no renormalisation, NaN / Inf tokens, and, with
XS_EMU_FULL=1, the weight-direct GEMMs behind XS_WEIGHT_DIRECT=1 (packed by
the library's own packing kernels) and the layer at the V4-Flash shape
(decode at 1, 16, 64 and 256 tokens, MXFP4 at 64)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EMU = os.path.join(ROOT, "tests", "emu")


@pytest.fixture(scope="module")
def fwd_emu(emu_fwd_lib, tmp_path_factory):
    from conftest import emu_link
    return emu_link(emu_fwd_lib, os.path.join(EMU, "fwd_main.cpp"), tmp_path_factory.mktemp("fwd_emu") / "fwd_emu")


# name, env, (T H I E k seed fp4 shared router x_f32 zipf norm residual noalloc [frag [toggle]]), expected routed GEMM
CASES = [
    ("tiled", {"XS_MOE_STREAM": "0"}, (64, 256, 256, 8, 2, 1, 0, 1, 1, 0, 0, 0, 0, 0), 0),
    ("stream", {}, (64, 256, 256, 8, 2, 1, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("tall", {}, (300, 256, 256, 4, 2, 2, 0, 1, 1, 0, 1.1, 0, 0, 0), 2),
    ("tall_fused_combine", {"XS_FUSE_COMBINE": "1"}, (300, 256, 256, 4, 2, 2, 0, 1, 1, 0, 1.1, 0, 0, 0), 2),
    # the combine in the shared expert's down epilogue: the same bits as the
    # separate combine (a second forward with the switch set), with the
    # pre-norm and a residual, and for f32 layers
    ("tall_shared_combine", {}, (300, 256, 256, 4, 2, 3, 0, 1, 1, 0, 1.1, 1, 1, 0, 0, "XS_SHARED_COMBINE=1"), 2),
    ("tall_shared_combine_f32", {}, (300, 256, 256, 4, 2, 4, 0, 1, 2, 1, 1.1, 0, 1, 0, 0, "XS_SHARED_COMBINE=1"), 2),
    ("c1_f32_chain", {}, (64, 256, 128, 8, 2, 11, 0, 1, 2, 1, 0, 0, 0, 0), 0),
    ("mxfp4_stream", {}, (48, 512, 512, 16, 6, 3, 1, 1, 1, 0, 0, 0, 0, 0), 1),
    ("mxfp4_tiled64", {"XS_MOE_STREAM": "0"}, (160, 512, 512, 16, 6, 4, 1, 1, 1, 0, 0, 0, 0, 0), 0),
    ("norm_residual", {}, (100, 512, 256, 16, 4, 5, 0, 1, 1, 0, 0, 1, 1, 0), 1),
    ("noalloc", {}, (40, 512, 256, 16, 4, 6, 0, 1, 1, 0, 0, 0, 0, 1), 1),
    ("decode_t1", {}, (1, 1024, 512, 64, 6, 8, 0, 1, 1, 0, 0, 0, 0, 0), 0),
    ("mfma_router", {}, (64, 256, 256, 8, 2, 7, 0, 1, 0, 0, 0, 0, 0, 0), 1),
    ("e1024_top16", {}, (48, 256, 128, 1024, 16, 10, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("f32_norm_residual", {}, (64, 256, 128, 8, 2, 12, 0, 1, 1, 1, 0, 1, 1, 0), 0),
    # group-limited routing (8 groups, keep 3), no renormalisation, scaling 2.5
    ("groups_scaling", {"EMU_ROUTE": "8,3,0,2.5"}, (64, 256, 256, 64, 6, 13, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("groups_mfma_router", {"EMU_ROUTE": "8,3,1,2.5"}, (40, 512, 256, 32, 4, 14, 0, 1, 0, 0, 0, 0, 0, 0), 1),
    # NaN / Inf in three tokens' rows of x: routing in range and the oracle's,
    # only those tokens' outputs non-finite (no spread through shared tiles,
    # split-K or stream-K partials)
    ("poison_nan_tall", {"EMU_POISON": "nan"}, (300, 512, 256, 16, 4, 15, 0, 1, 1, 0, 0, 0, 0, 0), 2),
    ("poison_inf_decode_chain", {"EMU_POISON": "inf"}, (16, 512, 256, 16, 4, 16, 0, 1, 2, 0, 0, 0, 0, 0), 1),
    ("poison_nan_mxfp4", {"EMU_POISON": "nan"}, (48, 512, 512, 16, 6, 17, 1, 1, 1, 0, 0, 0, 0, 0), 1),
    # every token through the certified router's exact pass
    ("exact_pass_everywhere", {"XS_ROUTER_MARGIN": "1e30"}, (24, 512, 256, 16, 4, 26, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("exact_pass_noalloc", {"XS_ROUTER_MARGIN": "1e30"}, (24, 512, 256, 16, 4, 27, 0, 1, 1, 0, 0, 0, 0, 1), 1),
]
# the weight-direct GEMMs (opt-in), packed by the library's own packing
# kernels; one to two minutes of CPU each: with XS_EMU_FULL=1
FULL_CASES = [
    ("wd_decode_packed_only", {"XS_WEIGHT_DIRECT": "1"}, (16, 1024, 512, 16, 4, 24, 0, 1, 1, 0, 0, 0, 0, 0, 2), 4),
    ("wd_prefill", {"XS_WEIGHT_DIRECT": "1"}, (300, 1024, 512, 4, 2, 22, 0, 1, 1, 0, 1.1, 0, 0, 0, 1), 3),
    ("wd_mxfp4", {"XS_WEIGHT_DIRECT": "1"}, (160, 1024, 512, 16, 6, 23, 1, 1, 1, 0, 0, 0, 0, 0, 1), 5),
    ("wd_mxfp4_packed_only", {"XS_WEIGHT_DIRECT": "1"}, (100, 1024, 512, 16, 6, 25, 1, 1, 1, 0, 0, 0, 0, 0, 2), 5),
]
# the layer at the V4-Flash shape (H 4096, I 2048, 256 experts, top-6 and the
# shared expert): decode batches of configs[3] on their real kernels and K
# lengths, and MXFP4 routed experts (configs[4]'s layer) at 64 tokens; one to
# four minutes of CPU each
FULL_CASES += [
    ("v4flash_decode_t1", {}, (1, 4096, 2048, 256, 6, 42, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("v4flash_decode_t16", {}, (16, 4096, 2048, 256, 6, 41, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("v4flash_decode_t64", {}, (64, 4096, 2048, 256, 6, 43, 0, 1, 1, 0, 0, 0, 0, 0), 1),
    ("v4flash_decode_t256", {}, (256, 4096, 2048, 256, 6, 44, 0, 1, 1, 0, 1.1, 0, 0, 0), 1),
    ("v4flash_mxfp4_t64", {}, (64, 4096, 2048, 256, 6, 45, 1, 1, 1, 0, 0, 0, 0, 0), 1),
    # the weight-direct GEMMs (opt-in) on packed-only layers at this shape
    ("v4flash_wd_decode_t16", {"XS_WEIGHT_DIRECT": "1"}, (16, 4096, 2048, 256, 6, 51, 0, 1, 1, 0, 0, 0, 0, 0, 2), 4),
    ("v4flash_wd_mxfp4_t64", {"XS_WEIGHT_DIRECT": "1"}, (64, 4096, 2048, 256, 6, 52, 1, 1, 1, 0, 0, 0, 0, 0, 2), 5),
]
# prefill at the V4-Flash shape on the tall tiles (1400 tokens, Zipf(1.1)
# routing as configs[2]), configs[4] itself (MXFP4, 2048 tokens) and
# configs[2] itself (8192 tokens): about 10, 20 and 35 minutes of CPU, with
# XS_EMU_HUGE=1
HUGE_CASES = [
    ("v4flash_prefill_t1400", {}, (1400, 4096, 2048, 256, 6, 46, 0, 1, 1, 0, 1.1, 0, 0, 0), 2),
    ("v4flash_mxfp4_t2048", {}, (2048, 4096, 2048, 256, 6, 47, 1, 1, 1, 0, 1.1, 0, 0, 0), 1),
    ("v4flash_prefill_t8192", {}, (8192, 4096, 2048, 256, 6, 48, 0, 1, 1, 0, 1.1, 0, 0, 0), 2),
    ("v4flash_wd_prefill_t1400", {"XS_WEIGHT_DIRECT": "1"}, (1400, 4096, 2048, 256, 6, 53, 0, 1, 1, 0, 1.1, 0, 0, 0, 1),
     3),
]
if os.environ.get("XS_EMU_FULL") == "1":
    CASES += FULL_CASES
if os.environ.get("XS_EMU_HUGE") == "1":
    CASES += HUGE_CASES
if os.environ.get("XS_EMU_FULL") == "1" or os.environ.get("XS_EMU_HUGE") == "1":
    # every case runs in the first test's setup (forward_runs): beyond the
    # default per-test limit with the full-size cases
    pytestmark = pytest.mark.timeout(4 * 3600)


def run_forward(exe, env, args):
    r = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=900,
                       env=dict(os.environ, **env))
    return r.returncode, r.stdout + r.stderr


def check_forward(rc, out, env, args, routed=None, tile_rows=None):
    """The checks of one emulated forward (fwd_main.cpp's output), shared with
    the sweep of tests/test_emu_sweep.py."""
    assert rc == 0, out[-3000:]
    assert re.search(r"^errors 0$", out, re.M), out[-3000:]
    if routed is not None:
        assert int(re.search(r"routed (\d+)", out).group(1)) == routed, out
    if tile_rows is not None:
        assert int(re.search(r"plan tile_rows (\d+)", out).group(1)) == tile_rows, out
    if env.get("XS_FUSE_COMBINE") == "1":
        assert re.search(r"fused 1", out), out
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"^([\w ]+?) mismatches (\d+)", out, re.M)}
    router = args[8]
    poison = "EMU_POISON" in env
    assert c["own permutation"] == 0, out
    # a NaN key has no rank the reference defines (it has no MoE router, and the
    # oracle's scan keeps a NaN it starts from): poisoned tokens must only
    # route in range, to distinct experts, with a consistent permutation
    for n in () if poison else ("idx", "w", "counts", "offsets", "perm", "inv"):
        assert c[n] == 0, (n, out)
    if len(args) > 15:
        assert re.search(r"toggle plan .* fused 2", out), out
        assert c["toggle"] == 0, out
    if router in (1, 2) and not poison:
        assert c["ref idx"] == 0, out
    if router == 2:
        assert c["logit"] == 0, out     # NaN logits compare by their bits
    assert float(re.search(r"max-abs-rel (\S+)", out).group(1)) <= 2e-2, out
    assert int(re.search(r"idx out of range or repeated (\d+)", out).group(1)) == 0, out
    npz, pzf, cnf = map(int, re.search(r"poisoned rows (\d+): with a finite output element (\d+); "
                                       r"clean rows with a non-finite one (\d+)", out).groups())
    assert npz == (len({0, args[0] // 2, args[0] - 1}) if "EMU_POISON" in env else 0), out
    assert pzf == 0 and cnf == 0, out
    if args[11]:    # the pre-norm's row against the oracle's sequential-sum norm
        # bf16: 2 codes.  f32: two orders of a sum of H positive squares
        # differ by at most about 2H ulps of the sum, and inv and y add a few
        assert int(re.search(r"norm max code diff (\d+)", out).group(1)) <= (2 * args[1] + 8 if args[9] else 2), out
    if env.get("EMU_NOALLOC_SEQ"):
        assert int(re.search(r"noalloc sequence mismatches (\d+)", out).group(1)) == 0, out
    pairs, tokens = map(int, re.search(r"exact pass logits (\d+) tokens (\d+)", out).groups())
    if env.get("XS_ROUTER_MARGIN"):
        assert (pairs, tokens) == (args[0] * args[3], args[0]), out
        assert c["logit"] == 0, out     # every logit routed on is the oracle's gemm_cpu logit
    elif router != 1:
        assert (pairs, tokens) == (0, 0), out


def run_all(exe, cases, workers=4):
    """Every case's run, several at a time (most cases occupy a few host
    threads only); {name: (rc, out)}."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(workers) as ex:
        futs = {c[0]: ex.submit(run_forward, exe, c[1], c[2]) for c in cases}
        return {n: f.result() for n, f in futs.items()}


def test_empty_batch_emulated(fwd_emu, tmp_path):
    """T = 0: xs_moe_forward and xs_moe_forward_noalloc return XS_OK with no
    workspace and launch nothing (the emulator's launch log stays empty)."""
    log = tmp_path / "launches.txt"
    rc, out = run_forward(fwd_emu, {"EMU_KERNEL_LOG": str(log)}, (0, 256, 128, 8, 2, 5, 0, 1, 1, 0, 0, 0, 0, 0))
    assert rc == 0 and "empty batch forward 0 noalloc 0" in out and re.search(r"^errors 0$", out, re.M), out
    assert not log.exists() or log.read_text() == "", log.read_text()


@pytest.fixture(scope="module")
def forward_runs(fwd_emu):
    # the V4-Flash-shape cases hold 6-13 GB of weights each: two at a time then
    big = os.environ.get("XS_EMU_FULL") == "1" or os.environ.get("XS_EMU_HUGE") == "1"
    return run_all(fwd_emu, CASES, workers=2 if big else 4)


@pytest.mark.parametrize("name,env,args,routed", CASES, ids=[c[0] for c in CASES])
def test_forward_emulated(forward_runs, name, env, args, routed):
    rc, out = forward_runs[name]
    check_forward(rc, out, env, args, routed)
