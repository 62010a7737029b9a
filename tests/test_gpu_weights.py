"""Loading an MoE layer from safetensors onto the GPU (load_moe_layer).

FP8 checkpoints: the loaded layer's output through xstar_cpp.moe equals the
output of the same weights handed over directly (bit for bit), and is within
2e-2 of the oracle.  Dense BF16 checkpoints: the weights quantized while
loading equal the oracle's FP8 128x128 block quantization of [gate ; up] and
down, bit for bit."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import xs_moe_capi  # noqa: F401  (fails loudly when the library is missing)


def _t(a):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.view(torch.bfloat16) if a.dtype == np.uint16 else t


def _checkpoint(c, prefix):
    """The case's stacked weights written back as per-expert DeepSeek-style names."""
    E, I = c["E"], c["I"]
    t = {f"{prefix}.gate.weight": _t(c["router_w"]), f"{prefix}.gate.e_score_correction_bias": _t(c["bias"])}

    def expert(base, w13, s13, w2, s2):
        w13, w2 = _t(w13).view(torch.float8_e4m3fn), _t(w2).view(torch.float8_e4m3fn)
        t[f"{base}.gate_proj.weight"] = w13[:I].clone()
        t[f"{base}.up_proj.weight"] = w13[I:].clone()
        t[f"{base}.gate_proj.weight_scale_inv"] = _t(s13[: I // 128]).clone()
        t[f"{base}.up_proj.weight_scale_inv"] = _t(s13[I // 128:]).clone()
        t[f"{base}.down_proj.weight"] = w2.clone()
        t[f"{base}.down_proj.weight_scale_inv"] = _t(s2).clone()

    for e in range(E):
        expert(f"{prefix}.experts.{e}", c["w13"][e], c["s13"][e], c["w2"][e], c["s2"][e])
    sh = c["shared"]
    expert(f"{prefix}.shared_experts", sh[0], sh[1], sh[2], sh[3])
    return t


def test_fp8_checkpoint_drives_moe_bit_exact(tmp_path):
    import xstar_cpp
    from safetensors.torch import save_file
    from bridge import torch_to_cpp, cpp_to_torch
    from moe_cases import make_case, to_device, layer_for, oracle_forward, max_abs_rel
    T, H, I, E, k = 48, 512, 256, 16, 4
    c = make_case(T, H, I, E, k, seed=31)
    t = _checkpoint(c, "model.layers.1.mlp")
    keys = sorted(t)
    p1, p2 = str(tmp_path / "a.safetensors"), str(tmp_path / "b.safetensors")
    save_file({kk: t[kk] for kk in keys[: len(keys) // 2]}, p1)
    save_file({kk: t[kk] for kk in keys[len(keys) // 2:]}, p2)
    print("load_moe_layer fp8", flush=True)
    w = xstar_cpp.load_moe_layer([p1, p2], "model.layers.1.mlp", xstar_cpp.Device.CUDA)
    assert (w.E, w.H, w.I) == (E, H, I)
    xt = xstar_cpp.to_cuda(torch_to_cpp(_t(c["x"])))
    out = xstar_cpp.moe(xt, w.router_w, w.router_bias, w.w13, w.w13_scale, w.w2, w.w2_scale, w.shared_w13,
                        w.shared_w13_scale, w.shared_w2, w.shared_w2_scale, top_k=k)
    got = cpp_to_torch(xstar_cpp.to_cpu(out), (T, H))
    g = to_device(c)
    ref = layer_for(c, g, router_exact=None).forward(g["x"])   # both on the default (certified) router
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.cpu().view(torch.int16))
    logits = xstar_cpp.moe_router_logits(xt, w.router_w)
    r = oracle_forward(c, logits_in=cpp_to_torch(xstar_cpp.to_cpu(logits), (T, E)).numpy())
    assert max_abs_rel(got.float().numpy(), r["out_f32"]) <= 2e-2


def test_dense_checkpoint_is_quantized_like_the_oracle(tmp_path):
    import xstar_cpp
    from safetensors.torch import save_file
    from bridge import cpp_to_torch
    E, H, I = 3, 512, 256
    g = torch.Generator().manual_seed(3)
    t = {"m.gate.weight": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)}
    for b in [f"m.experts.{e}" for e in range(E)] + ["m.shared_experts"]:
        for proj, (n, kk) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"{b}.{proj}.weight"] = (torch.randn(n, kk, generator=g) * 0.02).to(torch.bfloat16)
    t["m.experts.1.up_proj.weight"][:128, :128] = 0          # an all-zero block: scale 1, codes 0
    p = str(tmp_path / "d.safetensors")
    save_file(t, p)
    print("load_moe_layer dense bf16", flush=True)
    w = xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CUDA)
    w13 = cpp_to_torch(xstar_cpp.to_cpu(w.w13), (E, 2 * I, H)).numpy()
    s13 = cpp_to_torch(xstar_cpp.to_cpu(w.w13_scale), (E, 2 * I // 128, H // 128)).numpy()
    w2 = cpp_to_torch(xstar_cpp.to_cpu(w.w2), (E, H, I)).numpy()
    s2 = cpp_to_torch(xstar_cpp.to_cpu(w.w2_scale), (E, H // 128, I // 128)).numpy()
    for e in range(E):
        b = f"m.experts.{e}"
        dense13 = torch.cat([t[f"{b}.gate_proj.weight"], t[f"{b}.up_proj.weight"]]).float().numpy()
        rq, rs = oracle.quant_weight_fp8_block(dense13)
        assert np.array_equal(w13[e], rq) and np.array_equal(s13[e], rs)
        rq, rs = oracle.quant_weight_fp8_block(t[f"{b}.down_proj.weight"].float().numpy())
        assert np.array_equal(w2[e], rq) and np.array_equal(s2[e], rs)
    sw2 = cpp_to_torch(xstar_cpp.to_cpu(w.shared_w2), (H, I)).numpy()
    rq, _ = oracle.quant_weight_fp8_block(t["m.shared_experts.down_proj.weight"].float().numpy())
    assert np.array_equal(sw2, rq)
