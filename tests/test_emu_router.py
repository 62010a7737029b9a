"""Host emulation of the router kernels (moe_router.hip): the certified
router and the chain router run from the kernels' own source on the CPU (one
fiber per lane, tests/emu/router_emu.hpp) and are checked against the CPU
oracle (gemm_cpu-order logits, its routing).

Certified router: top-k indices equal the oracle's on its gemm_cpu logits,
weights equal the oracle's routing of the logits the kernels routed on, the
per-expert token masks match, every recomputed pair's logit is the oracle's
bit for bit, and with the margins widened (every token through the exact
pass) every logit is.  The MFMA is modelled six ways (exact sum rounded
once; k-order adds rounded or truncated; random-order adds rounded or
truncated; a pairwise tree); the bound must hold for each.
Covers decode (split-K MFMA kernel) and prefill (LDS-ring tile kernel) logits,
exact and near ties (duplicated router rows), group-limited routing, and E
not a multiple of 64, and both forms of the certified routing (one launch
with a block per token that routes, runs the exact pass and routes again;
routing, pair-parallel exact pass and second routing as three launches)."""
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


@pytest.fixture(scope="module")
def router_emu(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ not found")
    import oracle
    oracle.lib()          # builds oracle/_build/liboracle.so if needed
    d = tmp_path_factory.mktemp("router_emu")
    subprocess.run([sys.executable, os.path.join(EMU, "gen_router.py"), os.path.join(HIP, "moe_router.hip"),
                    os.path.join(HIP, "xs_device.hpp"), os.path.join(HIP, "moe_internal.hpp"),
                    str(d / "router_emu.inc")], check=True, cwd=EMU)
    build = os.path.join(ROOT, "oracle", "_build")
    exe = d / "router_emu"
    subprocess.run([CLANG, "-O2", "-std=c++20", "-pthread", "-Wno-psabi", "-ffp-contract=off", "-I", EMU,
                    "-I", str(d), "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle"),
                    os.path.join(EMU, "router_main.cpp"), "-o", str(exe), "-L", build, "-loracle", "-ldl",
                    f"-Wl,-rpath,{build}"], check=True)
    yield str(exe)
    shutil.rmtree(d, ignore_errors=True)


def _run(exe, *args, model=0):
    env = dict(os.environ, EMU_MFMA_MODEL=str(model))
    r = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert re.search(r"^errors 0$", out, re.M), out[-3000:]
    return out


def _counts(out):
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"^(\w+) mismatches (\d+)", out, re.M)}


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_chain_router_matches_gemm_cpu(router_emu, dtype):
    out = _run(router_emu, f"chain_{dtype}", 5, 200, 6, 1024, 3)
    assert _counts(out)["logit"] == 0, out


# mode T E k H seed nsplit margin bias_std zipf dup n_group topk_group path
CERT_CASES = [
    ("decode16", (16, 256, 6, 4096, 1, 16)),
    ("decode_skew", (32, 256, 6, 2048, 2, 8, 1, 0.1, 1.1)),
    ("prefill_tile", (300, 256, 6, 2048, 6, 4)),
    ("odd_E", (40, 72, 4, 1024, 5, 4)),
    ("ties", (32, 256, 6, 2048, 8, 8, 1, 0.1, 0, 16)),
    ("groups", (32, 256, 8, 2048, 9, 8, 1, 0.1, 0, 8, 8, 4)),
    ("all_exact", (16, 256, 6, 2048, 4, 16, 1e30)),
    ("all_exact_groups", (8, 256, 8, 1024, 9, 4, 1e30, 0.1, 0, 0, 8, 4)),
    ("e1024_top16", (24, 1024, 16, 512, 31, 4)),
    ("all_exact_e1024", (4, 1024, 16, 512, 32, 4, 1e30)),
    # the certified routing the other way than the forward picks for the
    # batch: separate routing, pair-parallel exact pass and second routing
    # launches at decode; one launch with a block per token at prefill
    ("decode16_pair_parallel", (16, 256, 6, 4096, 1, 16, 1, 0.1, 0, 0, 1, 1, 1)),
    ("all_exact_pair_parallel", (16, 256, 6, 2048, 4, 16, 1e30, 0.1, 0, 0, 1, 1, 1)),
    ("prefill_tile_route_blocks", (300, 256, 6, 2048, 6, 4, 1, 0.1, 0, 0, 1, 1, 2)),
]


ADVERSARIAL = ["decode16", "prefill_tile", "groups", "ties", "e1024_top16", "decode16_pair_parallel"]


@pytest.fixture(scope="module")
def cert_runs(router_emu):
    """Every (case, MFMA model) run of the two tests below, four at a time;
    {(name, model): output} (an AssertionError's message for a failed run)."""
    from concurrent.futures import ThreadPoolExecutor
    jobs = [(n, a, m) for n, a in CERT_CASES for m in (0, 1, 2) if not (m and n.startswith("all_exact"))]
    jobs += [(n, a, m) for n, a in CERT_CASES if n in ADVERSARIAL for m in (3, 4, 5)]

    def one(j):
        try:
            return _run(router_emu, "cert", *j[1], model=j[2])
        except AssertionError as e:
            return "RUN FAILED " + str(e)

    with ThreadPoolExecutor(4) as ex:
        return dict(zip([(n, m) for n, _, m in jobs], ex.map(one, jobs)))


@pytest.mark.parametrize("name,args", CERT_CASES, ids=[c[0] for c in CERT_CASES])
@pytest.mark.parametrize("model", [0, 1, 2])
def test_certified_router_matches_reference_routing(cert_runs, name, args, model):
    if model and name.startswith("all_exact"):
        pytest.skip("the exact pass does not read the MFMA results")
    out = cert_runs[(name, model)]
    assert not out.startswith("RUN FAILED"), out
    c = _counts(out)
    assert c == {"idx": 0, "w": 0, "mask": 0, "pair": 0, "exact": 0}, out
    pairs, flagged = map(int, re.search(r"pairs (\d+) flagged (\d+)", out).groups())
    if name.startswith("all_exact"):
        assert flagged == args[0] and pairs == args[0] * args[1]
    elif name == "ties":
        assert flagged > 0            # exact duplicates always need the exact pass


@pytest.mark.parametrize("name,args", [c for c in CERT_CASES if c[0] in ADVERSARIAL], ids=ADVERSARIAL)
@pytest.mark.parametrize("model", [3, 4, 5])
def test_certified_router_any_mfma_summation_order(cert_runs, name, args, model):
    """The bound assumes nothing about the order in which the MFMA adds its 32
    products and C: random orders with each add rounded (3) or truncated (4),
    and a pairwise tree (5), must route exactly like the reference too."""
    out = cert_runs[(name, model)]
    assert not out.startswith("RUN FAILED"), out
    assert _counts(out) == {"idx": 0, "w": 0, "mask": 0, "pair": 0, "exact": 0}, out


def test_certified_bound_is_what_keeps_the_routing_exact(router_emu):
    """Sensitivity of the checks above.  Inputs whose products cancel at
    magnitude 1000 (EMU_CANCEL) make the MFMA logits differ from gemm_cpu's by
    far more than the margins' fixed terms (2^-20 and the bias term), and near
    ties (dup) put experts within that error.  With the proven term removed
    (margin scale 0), a truncating random-order MFMA routes tokens wrongly;
    with it, every token is routed exactly.  So a bound missing its
    error terms fails these tests."""
    args = ("cert", 64, 256, 6, 2048, 8, 4)
    env = dict(os.environ, EMU_CANCEL="256", EMU_MFMA_MODEL="4")

    def run(margin):
        r = subprocess.run([router_emu, *map(str, args), str(margin), "0.1", "0", "32"], capture_output=True,
                           text=True, timeout=600, env=env)
        out = r.stdout + r.stderr
        assert r.returncode == 0 and re.search(r"^errors 0$", out, re.M), out[-3000:]
        return _counts(out), out

    c0, out0 = run(0)
    assert c0["idx"] > 0, out0
    c1, out1 = run(1)
    assert c1 == {"idx": 0, "w": 0, "mask": 0, "pair": 0, "exact": 0}, out1


def test_bf16_rounding_on_every_float(router_emu):
    """Row a9 by exhaustion: the kernels' bf16 rounding (xs_device.hpp), the
    oracle's and the reference's own bfloat16(float) (bfloat16.cpp:5-25,
    compiled into oracle/_ref when the reference tree is present) agree on all
    2^32 floats, NaN and infinities included (against the reference: every
    16th chunk of 65536 floats here, every float with XS_EMU_FULL=1, which
    takes about 4 minutes)."""
    ref = os.path.join(ROOT, "oracle", "_ref", "libxsref.so")
    full = os.environ.get("XS_EMU_FULL") == "1"
    args = ["bf16"] + ([ref, "1" if full else "16"] if os.path.exists(ref) else [])
    out = _run(router_emu, *args)
    assert int(re.search(r"bf16 device mismatches (\d+)", out).group(1)) == 0, out
    if os.path.exists(ref):
        assert int(re.search(r"bf16 reference mismatches (\d+)", out).group(1)) == 0, out


def test_software_encoders_on_every_float(router_emu):
    """The kernels' software e4m3 encoder (MXFP8 activations, FP8 weight
    quantization) and e2m1 encoder (MXFP4 weights) equal the oracle's: on
    every 61st bit pattern here, on all 2^32 floats with XS_EMU_FULL=1 (about
    3.5 minutes, clean): RNE, saturation, subnormals, NaN and infinities."""
    out = _run(router_emu, "codecs", 1 if os.environ.get("XS_EMU_FULL") == "1" else 61)
    assert int(re.search(r"e4m3 encode mismatches (\d+)", out).group(1)) == 0, out
    assert int(re.search(r"e2m1 encode mismatches (\d+)", out).group(1)) == 0, out


def test_route_sigmoid_error_bound(router_emu):
    """The certified router's margin assumes xs_sigmoid is within 2^-22 of the
    true sigmoid for every float: checked on every float but NaN (both signs,
    infinities) against the sigmoid in double.  The largest error is
    0.3746 x 2^-22, near x = 7.86.  The oracle's xo_sigmoid, the sigmoid of
    the reference keys in the bound, equals it bit for bit: on every 61st
    float pattern here, on every float with XS_EMU_FULL=1 (2 minutes)."""
    full = os.environ.get("XS_EMU_FULL") == "1"
    out = _run(router_emu, "sigmoid", 1 if full else 61)
    worst = float(re.search(r"sigmoid max error (\S+) x 2\^-22", out).group(1))
    assert worst < 0.5, out
    # the reference side of the bound: the oracle's sigmoid is the same function
    assert int(re.search(r"sigmoid oracle mismatches (\d+)", out).group(1)) == 0, out
