"""Randomised host emulation (opt-in: XS_EMU_FUZZ=N runs N cases of each
kind, XS_EMU_FUZZ_SEED picks the campaign).  Each case draws a shape, router,
routing options (group-limited, scaling, renormalisation), dtype, expert
format, pre-norm, residual, entry point, dispatch switches, NaN / Inf tokens,
the no-allocation forward twice in a row, and (a quarter of the cases)
fragment-packed weights on the weight-direct GEMMs.  It runs the whole
forward through the library's C ABI on the emulator (tests/emu/fwd_main.cpp)
or the certified router alone (tests/emu/router_main.cpp, with one of the
six MFMA summation models), and applies the same checks as the fixed cases:
routing, counts and permutation bit for bit, top-k from x for the certified
and chain routers, the chain router's logits bit for bit, the output within
2e-2 of the oracle's layer, the pre-norm's row within its bound."""
import os
import random
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from test_emu_forward import fwd_emu  # noqa: F401  (fixture)
from test_emu_router import router_emu  # noqa: F401  (fixture)

N = int(os.environ.get("XS_EMU_FUZZ", "0"))
SEED = int(os.environ.get("XS_EMU_FUZZ_SEED", "1"))
# a campaign runs in one test: about 10 s of CPU per forward case
pytestmark = [pytest.mark.skipif(N <= 0, reason="randomised emulation: set XS_EMU_FUZZ=N"),
              pytest.mark.timeout(max(1200, 30 * N))]


def _groups(r, E, k):
    divs = [g for g in range(2, 65) if E % g == 0 and E // g >= 2]
    if not divs:
        return 1, 1
    ng = r.choice(divs)
    return ng, r.choice([t for t in range(1, ng + 1) if t * (E // ng) >= k])


def _forward_case(exe, i):
    r = random.Random(SEED * 7919 + i)
    fp4 = r.random() < 0.25
    H = r.choice([256, 512, 768, 1024])
    I = r.choice([256, 512]) if fp4 else r.choice([128, 256, 384, 512])
    E = r.choice([1, 2, 4, 8, 16, 24, 64, 96, 256])
    k = r.randint(1, min(8, E))
    T = r.choice([1, 2, 7, 16, 33, 64, 100, 200, 256, 257, 300, 450])
    shared, router = r.choice([0, 1, 1]), r.choice([0, 1, 1, 2])
    xf32, norm, resid = r.random() < 0.2, r.random() < 0.3, r.random() < 0.3
    env = {}
    if r.random() < 0.3:
        env["XS_MOE_STREAM"] = r.choice(["0", "1"])
    if not fp4 and r.random() < 0.3:
        env["XS_MOE_GEMM"] = r.choice(["wide", "tiled"])
    if r.random() < 0.15:
        env["XS_FUSE_COMBINE"] = "1"
    if r.random() < 0.15:
        env["XS_ROUTER_MARGIN"] = r.choice(["1e30", "4"])
    if r.random() < 0.1:
        env["XS_FOLD_QUANT"] = "0"
    if r.random() < 0.3:
        ng, tg = _groups(r, E, k)
        env["EMU_ROUTE"] = f"{ng},{tg},{r.choice([0, 1])},{r.choice([1.0, 2.5])}"
    poison = r.random() < 0.1
    if poison:
        env["EMU_POISON"] = r.choice(["nan", "inf"])
    frag = 0
    if r.random() < 0.25:     # the weight-direct GEMMs on fragment-packed weights
        frag, H, I, E = r.choice([1, 2]), 1024, r.choice([512, 1024]), r.choice([4, 8, 16])
        k = min(k, E)
        env["XS_WEIGHT_DIRECT"] = "1"
        env.pop("EMU_ROUTE", None)
    if T * k * H * I > 300 * 8 * 1024 * 512:
        T = 64
    if T > 1 and r.random() < 0.15:   # the no-allocation forward twice, the second call smaller
        env["EMU_NOALLOC_SEQ"] = str(r.randint(1, T - 1))
    args = [T, H, I, E, k, r.randint(1, 10**6), int(fp4), shared, router, int(xf32), r.choice([0, 0, 1.1]),
            int(norm), int(resid), int(r.random() < 0.15), frag]
    if shared and r.random() < 0.2:
        args += ["XS_SHARED_COMBINE=1"]
    p = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=1200,
                       env=dict(os.environ, **env))
    out = p.stdout + p.stderr
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"^([\w ]+?) mismatches (\d+)", out, re.M)}
    bad = []
    if p.returncode != 0 or not re.search(r"^errors 0$", out, re.M):
        bad.append("run")
    bad += [n for n in ("own permutation", "toggle") if c.get(n, 1 if n == "own permutation" else 0)]
    bad += [] if poison else [n for n in ("idx", "w", "counts", "offsets", "perm", "inv") if c.get(n, 0)]
    m = re.search(r"idx out of range or repeated (\d+)", out)
    if not m or int(m.group(1)):
        bad.append("idx range")
    m = re.search(r"poisoned rows (\d+): with a finite output element (\d+); clean rows with a non-finite one (\d+)",
                  out)
    if not m or int(m.group(2)) or int(m.group(3)) or int(m.group(1)) != (len({0, T // 2, T - 1}) if poison else 0):
        bad.append("finiteness")
    if router in (1, 2) and not poison and c.get("ref idx", 0):
        bad.append("ref idx")
    if router == 2 and c.get("logit", 0):
        bad.append("logit")
    m = re.search(r"max-abs-rel (\S+)", out)
    if not m or float(m.group(1)) > 2e-2:
        bad.append("output")
    if "EMU_NOALLOC_SEQ" in env:
        m = re.search(r"noalloc sequence mismatches (\d+)", out)
        if not m or int(m.group(1)):
            bad.append("noalloc sequence")
    if norm:
        m = re.search(r"norm max code diff (\d+)", out)
        if not m or int(m.group(1)) > (2 * H + 8 if xf32 else 2):
            bad.append("norm")
    return bad, env, args, out


def _router_case(exe, i):
    r = random.Random(SEED * 100003 + i)
    E = r.choice([1, 2, 3, 8, 16, 32, 60, 64, 72, 96, 128, 200, 256, 384, 512, 1000, 1024])
    k = r.randint(1, min(16, E))
    H = r.choice([256, 512, 768, 1024, 2048, 4096])
    ns = r.choice([s for s in (1, 2, 4, 8, 16) if H % (128 * s) == 0])
    T = r.choice([1, 2, 3, 5, 16, 31, 64, 100, 255, 256, 257, 300, 513])
    if T > 300 and H > 1024:
        H, ns = 1024, min(ns, 8)
    dup = r.choice([0, 0, 0, r.randint(1, max(1, E // 2))]) if E >= 2 else 0
    ng, tg = _groups(r, E, k) if r.random() < 0.35 else (1, 1)
    args = ["cert", T, E, k, H, r.randint(1, 10**6), ns, r.choice([1, 1, 1, 1, 2, 1e30]),
            r.choice([0, 0.001, 0.1, 1.0, 5.0]), r.choice([0, 0, 1.1]), dup, ng, tg, r.choice([0, 1, 2])]
    model = r.choice([0, 1, 2, 3, 4, 5])
    p = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=900,
                       env=dict(os.environ, EMU_MFMA_MODEL=str(model)))
    out = p.stdout + p.stderr
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"^(\w+) mismatches (\d+)", out, re.M)}
    bad = [] if p.returncode == 0 and re.search(r"^errors 0$", out, re.M) and c else ["run"]
    if E == 1:
        c.pop("exact", None)   # one expert: no interval to meet, so no exact pass even at a huge margin
    bad += [n for n, v in c.items() if v]
    return bad, {"EMU_MFMA_MODEL": model}, args, out


def _campaign(fn, exe):
    with ThreadPoolExecutor(3) as ex:
        fails = [(b, e, a, o[-2000:]) for b, e, a, o in ex.map(lambda i: fn(exe, i), range(N)) if b]
    assert not fails, "\n\n".join(f"{b} {e} {' '.join(map(str, a))}\n{o}" for b, e, a, o in fails[:3])


def test_forward_fuzz(fwd_emu):  # noqa: F811
    _campaign(_forward_case, fwd_emu)


def test_certified_router_fuzz(router_emu):  # noqa: F811
    _campaign(_router_case, router_emu)
