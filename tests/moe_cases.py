"""Seeded MoE test cases shared by the GPU parity tests and smoke().

Inputs follow the configurations of the benchmark description: x ~ N(0, 1)
(C2-C5) or N(0, 0.02) (C1), router weights and expert weights ~ N(0, 0.02),
router bias ~ N(0, 0.1) or zero.  Expert weights are quantized on the CPU by
the oracle (they are inputs here; the GPU quantizers are tested separately).
"""
from __future__ import annotations

import numpy as np

import oracle


def make_case(T, H, I, E, k, *, seed=0, x_std=1.0, bf16=True, shared=True, bias_std=0.1,
              fp4=False, zipf=None):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, H)) * x_std).astype(np.float32)
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(E) * bias_std).astype(np.float32) if bias_std else None
    if zipf is not None:
        # skewed popularity: add log of a Zipf(s) rank distribution (random
        # expert <-> rank assignment) to the bias
        ranks = rng.permutation(E) + 1
        p = ranks.astype(np.float64) ** (-zipf)
        p /= p.sum()
        bias = (bias if bias is not None else np.zeros(E, np.float32)) + np.log(p).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    c = dict(T=T, H=H, I=I, E=E, k=k, bias=bias)
    if bf16:
        c["x"] = oracle.bf16_from_f32(x)
        c["router_w"] = oracle.bf16_from_f32(wr)
    else:
        c["x"], c["router_w"] = x, wr
    if fp4:
        c["w13"], c["s13"] = oracle.quant_weight_mxfp4(w13)
        c["w2"], c["s2"] = oracle.quant_weight_mxfp4(w2)
    else:
        c["w13"], c["s13"] = oracle.quant_weight_fp8_block(w13)
        c["w2"], c["s2"] = oracle.quant_weight_fp8_block(w2)
    c["fp4"] = fp4
    if shared:
        sw13 = (rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32)
        sw2 = (rng.standard_normal((H, I)) * 0.02).astype(np.float32)
        q13, s13 = oracle.quant_weight_fp8_block(sw13)
        q2, s2 = oracle.quant_weight_fp8_block(sw2)
        c["shared"] = (q13, s13, q2, s2)
    else:
        c["shared"] = None
    return c


def to_device(c, device="cuda"):
    import torch

    def d(a):
        if a is None:
            return None
        t = torch.from_numpy(np.ascontiguousarray(a))
        if a.dtype == np.uint16:
            t = t.view(torch.bfloat16)
        return t.to(device)

    g = {k: d(v) if isinstance(v, np.ndarray) else v for k, v in c.items() if k != "shared"}
    g["shared"] = None if c["shared"] is None else tuple(d(a) for a in c["shared"])
    return g


def layer_for(c, g, router_exact=False, **kw):
    import xs_moe_capi as X
    return X.MoeLayer(g["router_w"], g["w13"], g["s13"], g["w2"], g["s2"], c["k"],
                      router_bias=g["bias"], shared=g["shared"],
                      routed_format=X.XS_FP4_E2M1X2 if c["fp4"] else X.XS_FP8_E4M3,
                      router_exact=router_exact, **kw)


def oracle_forward(c, logits_in=None, rows=None, **kw):
    x = c["x"] if rows is None else np.ascontiguousarray(c["x"][rows])
    return oracle.moe_forward(x, c["router_w"], c["bias"], c["w13"], c["s13"], c["w2"], c["s2"],
                              c["k"], shared=c["shared"], routed_fp4=c["fp4"], logits_in=logits_in,
                              **kw)


def max_abs_rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def make_case_gpu(T, H, I, E, k, *, seed=0, shared=True, bias_std=0.1, fp4=False, zipf=None,
                  host=True):
    """Large cases: the benchmark's GPU generator (moe_synth.synth_layer: weights
    drawn on the GPU and quantized by the library's GPU quantizers, which
    test_gpu_stages pins bit-exact against the oracle).  Returns (case dict of
    numpy arrays or None, device dict)."""
    import torch
    from moe_synth import synth_layer

    g = synth_layer(T, H, I, E, k, seed=seed, shared=shared, bias_std=bias_std, fp4=fp4, zipf=zipf)
    if not host:
        return None, g

    def h(t):
        if t is None:
            return None
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    c = {kk: (h(v) if isinstance(v, torch.Tensor) else v) for kk, v in g.items() if kk != "shared"}
    c["shared"] = None if g["shared"] is None else tuple(h(t) for t in g["shared"])
    return c, g
