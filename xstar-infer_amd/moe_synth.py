"""Synthetic MoE layers for benchmarking, drawn and quantized on the GPU.

Weights ~ N(0, 0.02) are drawn with a seeded torch generator and quantized by
the library's own quantizers (xs_quant_weight_fp8_block / xs_quant_weight_mxfp4)
-- there is no network for checkpoints.  Activations x ~ N(0, 1) in bf16,
router weights ~ N(0, 0.02), router bias ~ N(0, 0.1) (or zero for uniform
routing).

Zipf(s) expert popularity (zipf=s): each token ranks the experts by
log p_e + Gumbel noise, with p a Zipf(s) rank distribution under a random
expert <-> rank map (Plackett-Luce sampling, so the realised per-expert token
counts follow the Zipf profile: a few experts near T tokens, a tail of ~T*k*p_256
tokens, all experts used).  The router is built to reproduce that ranking:
router rows are orthonormal (entries ~ N(0, 1/H), close to the N(0, 0.02) of
the plain case), the logits are chosen so that sigmoid(logit) + bias is an
increasing function of the key, and x = logits . W_r + (noise orthogonal to the
router rows), so x . W_r^T gives back the logits.
"""
from __future__ import annotations

import numpy as np


def _zipf_router(T, H, E, gen, bias, zipf, seed, dev):
    import torch
    rng = np.random.default_rng(seed)
    p = (np.arange(E) + 1.0) ** (-zipf)
    p /= p.sum()
    logp = torch.from_numpy(np.log(p[rng.permutation(E)]).astype(np.float32)).to(dev)
    u = torch.rand((T, E), generator=gen, device=dev).clamp_(1e-12, 1.0 - 1e-7)
    key = logp + (-torch.log(-torch.log(u)))
    b = bias if bias is not None else torch.zeros(E, device=dev)
    s = (0.5 + 0.03 * key - b).clamp_(0.004, 0.996)
    logits = torch.log(s / (1.0 - s))
    q, _ = torch.linalg.qr(torch.randn((H, E), generator=gen, device=dev))
    wr = q.t().contiguous()                                  # [E, H], orthonormal rows
    z = torch.randn((T, H), generator=gen, device=dev)
    x = logits @ wr + (z - (z @ wr.t()) @ wr)
    return x.to(torch.bfloat16), wr.to(torch.bfloat16)


def synth_layer(T, H, I, E, k, *, seed=0, shared=True, bias_std=0.1, fp4=False, zipf=None,
                chunk=16):
    import torch
    import xs_moe_capi as X

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    dev = "cuda"
    bias = torch.randn((E,), generator=gen, device=dev) * bias_std if bias_std else None
    if zipf is not None:
        x, wr = _zipf_router(T, H, E, gen, bias, zipf, seed, dev)
    else:
        x = torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16)
        wr = (torch.randn((E, H), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    g = dict(T=T, H=H, I=I, E=E, k=k, x=x, router_w=wr, bias=bias, fp4=fp4)
    quant = X.quant_weight_mxfp4 if fp4 else X.quant_weight_fp8_block
    if fp4:
        w13q = torch.empty((E, 2 * I, H // 2), dtype=torch.uint8, device=dev)
        w13s = torch.empty((E, 2 * I, H // 32), dtype=torch.uint8, device=dev)
        w2q = torch.empty((E, H, I // 2), dtype=torch.uint8, device=dev)
        w2s = torch.empty((E, H, I // 32), dtype=torch.uint8, device=dev)
    else:
        w13q = torch.empty((E, 2 * I, H), dtype=torch.uint8, device=dev)
        w13s = torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32, device=dev)
        w2q = torch.empty((E, H, I), dtype=torch.uint8, device=dev)
        w2s = torch.empty((E, H // 128, I // 128), dtype=torch.float32, device=dev)
    for e0 in range(0, E, chunk):
        e1 = min(E, e0 + chunk)
        w = torch.randn((e1 - e0, 2 * I, H), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02
        q, s = quant(w)
        w13q[e0:e1].copy_(q)
        w13s[e0:e1].copy_(s)
        del w, q, s
        w = torch.randn((e1 - e0, H, I), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02
        q, s = quant(w)
        w2q[e0:e1].copy_(q)
        w2s[e0:e1].copy_(s)
        del w, q, s
    g["w13"], g["s13"], g["w2"], g["s2"] = w13q, w13s, w2q, w2s
    if shared:
        sw13 = torch.randn((2 * I, H), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02
        sw2 = torch.randn((H, I), generator=gen, device=dev, dtype=torch.bfloat16) * 0.02
        q13, s13 = X.quant_weight_fp8_block(sw13)
        q2, s2 = X.quant_weight_fp8_block(sw2)
        g["shared"] = (q13, s13, q2, s2)
    else:
        g["shared"] = None
    torch.cuda.synchronize()
    return g


def layer_from(g, **kw):
    import xs_moe_capi as X
    return X.MoeLayer(g["router_w"], g["w13"], g["s13"], g["w2"], g["s2"], g["k"],
                      router_bias=g["bias"], shared=g["shared"],
                      routed_format=X.XS_FP4_E2M1X2 if g["fp4"] else X.XS_FP8_E4M3, **kw)


def expert_bytes(H, I, fp4):
    """HBM bytes of one expert's weights + scales."""
    if fp4:
        return 3 * H * I // 2 + 3 * H * I // 32
    return 3 * H * I + 4 * (2 * I // 128) * (H // 128) + 4 * (H // 128) * (I // 128)


def layer_flops(T, H, I, E, k, shared=True):
    """Algorithmic FLOPs of one layer forward: router + (k + shared) experts."""
    return T * (2 * H * E + (k + (1 if shared else 0)) * (2 * H * 2 * I + 2 * I * H))
