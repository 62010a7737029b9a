#!/usr/bin/env python3
"""Benchmark of the MI355X MoE operator (one GPU).

Workload (the configuration the headline metric is
quoted on): one V4-Flash MoE layer forward at prefill, 8192 bf16 tokens,
hidden 4096, 256 routed experts top-6 + 1 shared, intermediate 2048, FP8 e4m3
weights with 128x128 block scales, sigmoid router with bias ~ N(0, 0.1) and
Zipf(1.1)-skewed popularity.  A step = one full layer forward (router, top-k,
permute, gate_up GEMM + SwiGLU, down GEMM, combine) with inputs resident in
HBM.  The same JSON line also carries the decode configuration (configs[3]:
T in {1, 16, 64, 256}, uniform routing, HBM GB/s), the single FP8 GEMM
(configs[1]) and the MXFP4 layer.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "xstar-infer_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, ROOT)

H, I, E, K_TOP = 4096, 2048, 256, 6
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
METRIC = "MoE-layer tokens/s + TFLOP/s (% FP8 MFMA peak) and decode HBM GB/s, hid4096"


PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "moe_gemm_prefill8192.md")


def measured_traffic():
    """HBM bytes per gate_up dispatch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a 1 GiB copy), or None."""
    try:
        for line in open(PROFILE_SUMMARY):
            if line.startswith("traffic_bytes_gate_up:"):
                return float(line.split(":")[1])
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_forward(layer, x, steps, warmup, profile=False):
    import torch
    import xs_moe_capi as X
    out = torch.empty_like(x)
    for _ in range(warmup):
        layer.forward(x, out=out)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        layer.forward(x, out=out)
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    stages = None
    if profile:
        # second pass with per-stage HIP events recorded by the library on its stream
        X.profile_enable(True)
        for _ in range(steps):
            layer.forward(x, out=out)
        torch.cuda.synchronize()
        tot, n = X.profile_read()
        X.profile_enable(False)
        stages = {kk: v / max(n, 1) for kk, v in tot.items()}
    return ms, stages


def routed_counts(layer, x):
    import torch
    dbg = dict(counts=torch.empty(layer.E, dtype=torch.int32, device="cuda"))
    layer.forward(x, debug=dbg)
    torch.cuda.synchronize()
    return dbg["counts"].cpu().numpy()


def routed_expert_count(layer, x):
    return int((routed_counts(layer, x) > 0).sum())


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _ref_f32_seconds(g, T0, T1, torch):
    """The reference's CPU path restated (oracle.moe_ref_f32: gemm_cpu i->kk->j
    order with transB strided reads, f32 mlp() per expert, weighted sum plus the
    shared expert; single thread) on tokens [T0, T1) of a synthetic layer, with
    the FP8 weights dequantized to f32 (as a reference user would load them).
    Returns (seconds, experts touched)."""
    import oracle

    x = g["x"][T0:T1].float().cpu().numpy()
    wr = g["router_w"].float().cpu().numpy()
    bias = g["bias"].cpu().numpy() if g["bias"] is not None else None
    idx, _ = oracle.route(oracle.router_logits(x, wr, False), bias, g["k"])
    touched = sorted(set(idx.ravel().tolist()))

    def deq(q, s_):
        v = q.view(torch.float8_e4m3fn).float()
        rep = s_.repeat_interleave(128, -2).repeat_interleave(128, -1)
        return (v * rep).cpu().numpy()

    w13 = {e: deq(g["w13"][e], g["s13"][e]) for e in touched}
    w2 = {e: deq(g["w2"][e], g["s2"][e]) for e in touched}
    sh = g["shared"]
    shared = (deq(sh[0], sh[1]), deq(sh[2], sh[3])) if sh is not None else None
    t0 = time.perf_counter()
    oracle.moe_ref_f32(x, wr, bias, w13, w2, g["k"], shared=shared)
    return time.perf_counter() - t0, len(touched)


def cpu_baseline(g_prefill, g_decode, torch, slice_tokens=64):
    """BASELINE protocol: one core (this thread pinned to one CPU), configs C1,
    C4 at T = 1 and 16, and a slice of C3; C3's tokens/s is the slice's rate, a
    per-token extrapolation of the full 8192-token layer."""
    cpus = sorted(os.sched_getaffinity(0))
    os.sched_setaffinity(0, {cpus[0]})
    try:
        runs = {}
        import numpy as np
        import oracle
        rng = np.random.default_rng(11)   # C1: f32, everything ~ N(0, 0.02), zero bias
        n = lambda *sh: (rng.standard_normal(sh) * 0.02).astype(np.float32)  # noqa: E731
        x1, wr1, w13, w2 = n(64, 256), n(8, 256), n(8, 256, 256), n(8, 256, 128)
        t0 = time.perf_counter()
        oracle.moe_ref_f32(x1, wr1, None, w13, w2, 2, shared=(n(256, 256), n(256, 128)))
        dt = time.perf_counter() - t0
        runs["C1_tiny_f32_64tok"] = {"s": dt, "tokens_per_s": 64 / dt, "experts_touched": 8}
        for Td in (1, 16):
            dt, ne = _ref_f32_seconds(g_decode, 0, Td, torch)
            runs[f"C4_decode_T{Td}"] = {"s": dt, "tokens_per_s": Td / dt, "experts_touched": ne}
        dt, ne = _ref_f32_seconds(g_prefill, 0, slice_tokens, torch)
        runs[f"C3_prefill_{slice_tokens}tok_slice"] = {"s": dt, "tokens_per_s": slice_tokens / dt,
                                                       "experts_touched": ne,
                                                       "extrapolated_8192tok_s": dt / slice_tokens * 8192}
    finally:
        os.sched_setaffinity(0, set(cpus))
    c3 = runs[f"C3_prefill_{slice_tokens}tok_slice"]
    return dict(value=c3["tokens_per_s"], unit="tokens/s", cores=1, kind="port",
                sample=(f"C3 value = first {slice_tokens} tokens of the prefill workload (per-token "
                        f"extrapolation to 8192 tokens: {c3['extrapolated_8192tok_s']:.0f} s); reference-path "
                        f"f32 restated (gemm_cpu i->kk->j order, mlp per expert), 1 pinned core of "
                        f"{len(cpus)} visible, CPU {_cpu_model()}"),
                cpu_model=_cpu_model(), nproc=os.cpu_count(), visible_cpus=len(cpus), configs=runs)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="prefill only, no extra configs")
    ap.add_argument("--sections", default="prefill,decode,gemm,fp4,norm,block",
                    help="comma list of prefill,decode,gemm,fp4,norm,block (the JSON line needs prefill)")
    ap.add_argument("--decode-tokens", default="1,16,64,256",
                    help="comma list of decode batch sizes (configs[3])")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=64, help="tokens of the C3 slice the CPU baseline times")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (the MoE operator is built and measured for a "
              f"single MI355X holding all experts of a layer); --gpus {a.gpus} is not supported.",
              file=sys.stderr)
        return 2

    import torch
    import xs_moe_capi as X
    from moe_synth import synth_layer, layer_from, expert_bytes, layer_flops

    dev_name = torch.cuda.get_device_name(0)
    log(f"device: {dev_name}")
    sections = set(a.sections.split(","))
    if a.quick:
        sections &= {"prefill"}
    res = {}
    if "prefill" in sections:
        res = prefill(a, X, torch)
    # the other configurations: a failure in one is recorded in its place and
    # does not take the headline line with it
    def leg(name, fn):
        try:
            res[name] = fn()
        except Exception as e:  # noqa: BLE001
            log(f"{name} failed: {e!r}")
            res[name] = {"error": repr(e)}
            torch.cuda.synchronize()
            torch.cuda.empty_cache()

    if "decode" in sections:
        leg("decode", lambda: decode(a, X, torch))
    if "gemm" in sections:
        leg("gemm_fp8_512x4096x4096", lambda: single_gemm(a, X, torch))
    if "fp4" in sections:
        leg("fp4_2048", lambda: fp4_layer(a, X, torch))
    if "norm" in sections or "block" in sections:
        leg("rmsnorm_8192x4096", lambda: norm_legs(a, X, torch, kernels="norm" in sections, block="block" in sections))
    print(json.dumps(res))
    return 0


# the gate_up kernel of each GEMM family at the prefill shape (the roofline's kernel)
GATE_UP_KERNEL = {
    "tall": "moe_gemm_wide_kernel<192, gate_up> (grouped FP8 gate_up GEMM + SwiGLU + requant)",
    "direct_prefill": "moe_gemm_wd_kernel<gate_up, 32> (weight-direct grouped FP8 gate_up GEMM + SwiGLU + requant)",
}


def safe_plan(layer, T):
    """layer.plan(T), or the error it raised (the measurement stands either way)."""
    try:
        return layer.plan(T)
    except Exception as e:  # noqa: BLE001
        return {"error": str(e)}


def bench_frag():
    """XS_BENCH_FRAG: 0 (default) row-major weights; 1 also fragment-packed
    copies (the weight-direct GEMMs); only: packed copies alone."""
    v = os.environ.get("XS_BENCH_FRAG", "0")
    if v != "0":
        os.environ["XS_WEIGHT_DIRECT"] = "1"   # the weight-direct GEMMs are opt-in
    return "only" if v == "only" else v == "1"


def prefill(a, X, torch):
    from moe_synth import synth_layer, layer_from, expert_bytes, layer_flops
    T = 8192
    g = synth_layer(T, H, I, E, K_TOP, seed=0, zipf=1.1)
    # XS_BENCH_FRAG=1 / only: fragment-packed weights, weight-direct GEMMs
    layer = layer_from(g, frag=bench_frag())
    ms, stages = time_forward(layer, g["x"], a.steps, a.warmup, profile=True)
    flops = layer_flops(T, H, I, E, K_TOP)
    counts = routed_counts(layer, g["x"])
    ne = int((counts > 0).sum())
    wbytes = (ne + 1) * expert_bytes(H, I, False) + E * H * 2
    act_bytes = T * H * 2 * 2 + T * H + (T * K_TOP + T) * (I + 2 * H)
    gu_ms = stages["gemm_gate_up"]
    # gate_up launch: algorithmic flops (k + shared rows x 2H x 2I) and bytes
    # (W13 of every expert it touches, FP8 activations read once, the requantized
    # act written once); its floors are 0.39 ms at the FP8 peak and 0.56 ms at the
    # HBM peak, so the bounding roofline is HBM
    gu_flops = (K_TOP + 1) * T * 2 * H * 2 * I
    gu_bytes = ((ne + 1) * (2 * I * H + 4 * (2 * I // 128) * (H // 128)) + T * H * (1 + 4 / 128)
                + (K_TOP + 1) * T * I * (1 + 4 / 128))
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (bf16 in/out, f32 accumulate)",
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) weights quantized on the GPU)",
        "config": {"workload": "V4-Flash MoE layer prefill, configs[2]", "tokens": T, "hidden": H,
                   "moe_intermediate": I, "experts": E, "top_k": K_TOP, "shared_experts": 1,
                   "weights": "e4m3 128x128 block scales", "routing": "sigmoid+bias, Zipf(1.1)",
                   "parallelism": "single GPU"},
        "routing_counts": {"experts_used": ne, "max": int(counts.max()), "min": int(counts.min()),
                           "top8": sorted(counts.tolist(), reverse=True)[:8]},
        "layer_tflops": flops / (ms * 1e-3) / 1e12,
        "layer_frac_fp8_peak": flops / (ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS,
        "layer_hbm_gbs": (wbytes + act_bytes) / (ms * 1e-3) / 1e9,
        "stage_ms": stages,
        "plan": safe_plan(layer, T),   # the kernels that ran (xs_moe_plan)
        "roofline": {"kernel": GATE_UP_KERNEL.get(safe_plan(layer, T).get("routed"), str(safe_plan(layer, T))),
                     "bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": measured_traffic(),
                     "algorithmic_bytes": gu_bytes, "launch_ms": gu_ms,
                     "mfma_tflops": gu_flops / (gu_ms * 1e-3) / 1e12,
                     "mfma_frac": gu_flops / (gu_ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS},
    }
    # the default (certified, bit-exact top-k) router against the approximate
    # MFMA router and the chain router (every logit in gemm_cpu order)
    try:
        res["router"] = router_report(layer, g["x"], T, ms, stages, a, layer_from, g)
    except Exception as e:  # noqa: BLE001
        log(f"router report failed: {e!r}")
        res["router"] = {"error": repr(e)}
    del layer
    if not a.no_cpu:
        log("cpu baseline ...")
        gdc = synth_layer(16, H, I, E, K_TOP, seed=1, bias_std=0.0)
        res["cpu_baseline"] = cpu_baseline(g, gdc, torch, a.cpu_tokens)
        del gdc
    del g
    torch.cuda.empty_cache()
    return res


def router_report(layer, x, T, ms, stages, a, layer_from, g):
    """The default certified router's share of the layer (its logits launch
    with the bound terms; route, exact pass and second route together make the
    route stage) and how much the exact pass did on this batch, next to the
    same layer with the approximate MFMA router and with the chain router."""
    layer.forward(x)
    pairs, tokens = layer.router_stats(T)
    rep = {"kind": "certified", "logits_ms": stages["router_logits"], "route_ms": stages["route"],
           "exact_pass": {"logits": pairs, "tokens": tokens, "token_frac": tokens / max(T, 1)}}
    for name, kind in (("mfma", 0), ("chain", 2)):
        lx = layer_from(g, router=kind)
        msx, stx = time_forward(lx, x, a.steps, a.warmup, profile=True)
        rep[name] = {"ms_per_step": msx, "logits_ms": stx["router_logits"], "route_ms": stx["route"],
                     "layer_ms_vs_certified": msx - ms}
        del lx
    return rep


def decode(a, X, torch):
    """T in {1, 16, 64, 256}, uniform routing; HBM bytes = weights of
    the experts touched + shared + router + activations."""
    from moe_synth import synth_layer, layer_from, expert_bytes
    dec = {}
    gd = synth_layer(256, H, I, E, K_TOP, seed=1, bias_std=0.0)
    # XS_BENCH_FRAG=1 / only: fragment-packed weights, weight-direct GEMMs
    L = layer_from(gd, frag=bench_frag())
    for Td in (int(t) for t in a.decode_tokens.split(",")):
        xd = gd["x"][:Td].contiguous()
        msd, st = time_forward(L, xd, max(a.steps, 50), a.warmup, profile=True)
        ned = routed_expert_count(L, xd)
        by = (ned + 1) * expert_bytes(H, I, False) + E * H * 2 + Td * H * 4
        a_dec = argparse.Namespace(**dict(vars(a), steps=max(a.steps, 50)))
        dec[str(Td)] = {"ms": msd, "experts_touched": ned + 1, "hbm_gbs": by / (msd * 1e-3) / 1e9,
                        "frac_hbm_peak": by / (msd * 1e-3) / 1e9 / PEAK_HBM_GBS,
                        "tokens_per_s": Td / (msd * 1e-3), "stage_ms": st, "plan": safe_plan(L, Td),
                        "router": router_report(L, xd, Td, msd, st, a_dec, layer_from, gd)}
    del gd
    torch.cuda.empty_cache()
    return dec


def single_gemm(a, X, torch):
    """one FP8 block-scaled GEMM 512 x 4096 x 4096 (bf16 A, e4m3 B)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2)
    A = torch.randn((512, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    Wt = torch.randn((4096, 4096), generator=gen, device="cuda", dtype=torch.bfloat16) * 0.02
    bq, bs = X.quant_weight_fp8_block(Wt)
    C_ = torch.empty((512, 4096), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(X.lib().xs_gemm_fp8_blockscale_workspace_size(512, 4096), dtype=torch.uint8, device="cuda")
    gfl = 2 * 512 * 4096 * 4096

    def timed(call):
        for _ in range(a.warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        n = 50
        for _ in range(n):
            call()
        e1.record()
        torch.cuda.synchronize()
        gms = e0.elapsed_time(e1) / n
        return {"ms": gms, "tflops": gfl / (gms * 1e-3) / 1e12,
                "frac_fp8_peak": gfl / (gms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS}

    res = timed(lambda: X.gemm_fp8_blockscale(A, bq, bs, out=C_, workspace=ws))
    res["kernel"] = "gemm_dense_fp8_kernel (row-major B through the LDS ring)"
    if bench_frag():
        # XS_BENCH_FRAG=1 / only: B also packed in fragment order, the
        # weight-direct kernel (the packing is a load-time step, outside the timing)
        bp = X.pack_weight_fp8_frag(bq)
        res["packed"] = timed(lambda: X.gemm_fp8_blockscale_packed(A, bp, bs, out=C_, workspace=ws))
        res["packed"]["kernel"] = "gemm_wd_dense_kernel (packed B straight into registers)"
    return res


def fp4_layer(a, X, torch):
    """MXFP4 routed experts (FP8 shared), 2048 tokens."""
    from moe_synth import synth_layer, layer_from, expert_bytes, layer_flops
    g4 = synth_layer(2048, H, I, E, K_TOP, seed=3, fp4=True)
    # XS_BENCH_FRAG=1 / only: packed MXFP4 weights and scales, weight-direct GEMMs
    L4 = layer_from(g4, frag=bench_frag())
    ms4, st4 = time_forward(L4, g4["x"], a.steps, a.warmup, profile=True)
    ne4 = routed_expert_count(L4, g4["x"])
    by4 = ne4 * expert_bytes(H, I, True) + expert_bytes(H, I, False) + E * H * 2
    fl4 = layer_flops(2048, H, I, E, K_TOP)
    return {"ms": ms4, "tokens_per_s": 2048 / (ms4 * 1e-3), "tflops": fl4 / (ms4 * 1e-3) / 1e12,
            "hbm_gbs_weights": by4 / (ms4 * 1e-3) / 1e9, "stage_ms": st4, "plan": safe_plan(L4, 2048)}



def norm_legs(a, X, torch, kernels=True, block=True):
    """RMSNorm at the prefill activation shape (8192 x 4096 bf16): alone, fused
    with the FP8 1x128 quant of its output, the separate quant for comparison,
    and the MoE layer with the pre-norm against the layer without it."""
    from moe_synth import synth_layer, layer_from
    T = 8192
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    x = torch.randn((T, H), generator=gen, device="cuda").to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=gen, device="cuda")).to(torch.bfloat16)
    y = torch.empty_like(x)
    q = torch.empty((T, H), dtype=torch.uint8, device="cuda")
    s = torch.empty((T, H // 128), dtype=torch.float32, device="cuda")
    st = X._stream()
    L = X.lib()

    def norm(quant):
        X.check(L.xs_rmsnorm(X._ptr(x), X._ptr(w), X.XS_BF16, T, H, 1e-6, X._ptr(y),
                             X._ptr(q) if quant else None, X._ptr(s) if quant else None, st))

    def quant_only():
        X.check(L.xs_quant_act_fp8(X._ptr(y), X.XS_BF16, T, H, X._ptr(q), X._ptr(s), st))

    def timed(fn, n=50):
        for _ in range(a.warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    out = {}
    b_norm = 2 * T * H * 2 + 2 * H
    b_fused = b_norm + T * H + 4 * T * (H // 128)
    b_quant = 2 * T * H + T * H + 4 * T * (H // 128)
    legs = (("rmsnorm", lambda: norm(False), b_norm), ("rmsnorm_fp8", lambda: norm(True), b_fused),
            ("quant_act_fp8", quant_only, b_quant))
    for name, fn, by in legs if kernels else ():
        ms = timed(fn)
        out[name] = {"ms": ms, "bytes": by, "gbs": by / (ms * 1e-3) / 1e9,
                     "frac_hbm_peak": by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}
    del x, y, q, s
    if not block:
        torch.cuda.empty_cache()
        return out
    # the MoE layer with and without the pre-norm (prefill and a decode batch)
    g = synth_layer(T, H, I, E, K_TOP, seed=0, zipf=1.1)
    for Tn in (T, 16):
        xn = g["x"][:Tn].contiguous()
        base = layer_from(g)
        ms0, _ = time_forward(base, xn, a.steps, a.warmup)
        del base
        pre = layer_from(g, norm_weight=w, norm_eps=1e-6)
        ms1, st1 = time_forward(pre, xn, a.steps, a.warmup, profile=True)
        # the block's FFN half, h + moe(rmsnorm(h)): fused (norm in the quant
        # pass, residual in the combine) against three separate calls
        res = torch.empty_like(xn)
        ms2 = timed(lambda: pre.forward(xn, out=res, residual=xn))
        plain = layer_from(g)
        xnn = torch.empty_like(xn)
        mo = torch.empty_like(xn)

        def unfused():
            X.check(L.xs_rmsnorm(X._ptr(xn), X._ptr(w), X.XS_BF16, Tn, H, 1e-6, X._ptr(xnn), None, None, st))
            plain.forward(xnn, out=mo)
            torch.add(xn, mo, out=res)
        ms3 = timed(unfused)
        del pre, plain, res, xnn, mo
        out[f"moe_T{Tn}"] = {"ms_without_norm": ms0, "ms_with_prenorm": ms1, "act_quant_stage_ms": st1["act_quant"],
                             "ms_block_ffn_fused": ms2, "ms_block_ffn_unfused": ms3}
    del g
    torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
