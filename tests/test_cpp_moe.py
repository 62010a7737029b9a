"""The pybind11 drop-in (xstar_cpp.moe and stage ops): argument validation with
the reference's error messages (CPU), raw-byte bridges (CPU), and on the GPU
equality with the C-ABI path and parity with the oracle."""
import numpy as np
import pytest
import torch

import xstar_cpp
from bridge import torch_to_cpp, cpp_to_torch

D = xstar_cpp.DType


def _weights(E=4, H=256, I=128, seed=0, fp4=False):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    x = r(8, H).to(torch.bfloat16)
    wr = (r(E, H) * 0.02).to(torch.bfloat16)
    if fp4:
        w13 = torch.zeros(E, 2 * I, H // 2, dtype=torch.uint8)
        s13 = torch.full((E, 2 * I, H // 32), 127, dtype=torch.uint8)
        w2 = torch.zeros(E, H, I // 2, dtype=torch.uint8)
        s2 = torch.full((E, H, I // 32), 127, dtype=torch.uint8)
        return x, wr, (torch_to_cpp(w13, D.Float4E2M1x2), torch_to_cpp(s13, D.Float8E8M0),
                       torch_to_cpp(w2, D.Float4E2M1x2), torch_to_cpp(s2, D.Float8E8M0))
    w13 = torch.zeros(E, 2 * I, H, dtype=torch.uint8)
    s13 = torch.ones(E, 2 * I // 128, H // 128)
    w2 = torch.zeros(E, H, I, dtype=torch.uint8)
    s2 = torch.ones(E, H // 128, I // 128)
    return x, wr, (torch_to_cpp(w13, D.Float8E4M3), torch_to_cpp(s13), torch_to_cpp(w2, D.Float8E4M3),
                   torch_to_cpp(s2))


def test_raw_bridge_roundtrip_bitexact():
    x = torch.randn(3, 5).to(torch.bfloat16)
    assert torch.equal(cpp_to_torch(torch_to_cpp(x), x.shape).view(torch.int16), x.view(torch.int16))
    y = torch.randn(7)
    assert torch.equal(cpp_to_torch(torch_to_cpp(y), y.shape), y)
    q = torch.randint(0, 255, (4, 6), dtype=torch.uint8)
    t = torch_to_cpp(q, D.Float8E4M3)
    assert t.dtype() == D.Float8E4M3 and t.nbytes() == 24
    assert torch.equal(cpp_to_torch(t, q.shape), q)


def test_from_numpy_raw_checks_itemsize():
    with pytest.raises(RuntimeError, match="itemsize mismatch"):
        xstar_cpp.from_numpy_raw(np.zeros(4, np.float32), [4], D.BFloat16)
    with pytest.raises(RuntimeError, match="byte count mismatch"):
        xstar_cpp.from_numpy_raw(np.zeros(4, np.float32), [5], D.Float32)


def test_moe_on_cpu_tensors_is_unsupported_device():
    """No CPU fallback: the product path runs only on the GPU."""
    x, wr, (w13, s13, w2, s2) = _weights()
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.moe(torch_to_cpp(x), torch_to_cpp(wr), None, w13, s13, w2, s2, top_k=2)


def test_moe_dtype_rank_shape_errors():
    x, wr, (w13, s13, w2, s2) = _weights()
    xt, wrt = torch_to_cpp(x), torch_to_cpp(wr)
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        xstar_cpp.moe(xt, torch_to_cpp(wr.float()), None, w13, s13, w2, s2, top_k=2)
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        xstar_cpp.moe(xt, wrt, None, w13, s13, w2, torch_to_cpp(torch.ones(4, 2, 1, dtype=torch.int32)), top_k=2)
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        xstar_cpp.moe(torch_to_cpp(torch.ones(8, 256, dtype=torch.int32)), wrt, None, w13, s13, w2, s2, top_k=2)
    with pytest.raises(RuntimeError, match="rank mismatch"):
        xstar_cpp.moe(xt, torch_to_cpp(wr.flatten()), None, w13, s13, w2, s2, top_k=2)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.moe(xt, torch_to_cpp(wr[:, :128].contiguous()), None, w13, s13, w2, s2, top_k=2)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.moe(xt, wrt, None, w13, s13, w2, s2, top_k=5)        # top_k > E
    with pytest.raises(RuntimeError, match="shape mismatch"):        # partial shared expert
        xstar_cpp.moe(xt, wrt, None, w13, s13, w2, s2, shared_w13=w13, top_k=2)


def test_moe_fp4_signature_validates():
    x, wr, (w13, s13, w2, s2) = _weights(fp4=True)
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.moe(torch_to_cpp(x), torch_to_cpp(wr), None, w13, s13, w2, s2, top_k=2)
    _, _, (f13, fs13, f2, fs2) = _weights()
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        xstar_cpp.moe(torch_to_cpp(x), torch_to_cpp(wr), None, w13, fs13, w2, s2, top_k=2)


def test_stage_ops_validate_on_cpu():
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.moe_route(torch_to_cpp(torch.zeros(4, 8)), None, 2)
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        xstar_cpp.moe_route(torch_to_cpp(torch.zeros(4, 8).to(torch.bfloat16)), None, 2)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.quant_act_fp8(torch_to_cpp(torch.zeros(4, 100)))
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.moe_permute(torch_to_cpp(torch.zeros(4, 2, dtype=torch.int32)), 8)


@pytest.mark.gpu
def test_cpp_moe_matches_capi_and_oracle():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from moe_cases import make_case, to_device, layer_for, oracle_forward, max_abs_rel
    c = make_case(40, 512, 256, 16, 4, seed=77)
    g = to_device(c)
    ref_gpu = layer_for(c, g, router_exact=None).forward(g["x"])   # both on the default (certified) router
    torch.cuda.synchronize()
    cu = lambda a, d=None: xstar_cpp.to_cuda(torch_to_cpp(torch.from_numpy(np.ascontiguousarray(a)), d))  # noqa: E731
    xt = xstar_cpp.to_cuda(torch_to_cpp(g["x"]))
    wrt = xstar_cpp.to_cuda(torch_to_cpp(g["router_w"]))
    bt = xstar_cpp.to_cuda(torch_to_cpp(g["bias"]))
    sh = c["shared"]
    out = xstar_cpp.moe(xt, wrt, bt, cu(c["w13"], D.Float8E4M3), cu(c["s13"]), cu(c["w2"], D.Float8E4M3), cu(c["s2"]),
                        cu(sh[0], D.Float8E4M3), cu(sh[1]), cu(sh[2], D.Float8E4M3), cu(sh[3]), top_k=4)
    got = cpp_to_torch(xstar_cpp.to_cpu(out), (40, 512))
    assert torch.equal(got.view(torch.int16), ref_gpu.cpu().view(torch.int16))   # same kernels, same bits
    logits = cpp_to_torch(xstar_cpp.to_cpu(xstar_cpp.moe_router_logits(xt, wrt)), (40, 16)).numpy()
    r = oracle_forward(c, logits_in=logits)
    assert max_abs_rel(got.float().numpy(), r["out_f32"]) <= 2e-2
    idx, w = xstar_cpp.moe_route(xstar_cpp.to_cuda(torch_to_cpp(torch.from_numpy(logits))), bt, 4)
    assert np.array_equal(cpp_to_torch(xstar_cpp.to_cpu(idx), (40, 4)).numpy(), r["idx"])
    counts, offsets, perm, inv = xstar_cpp.moe_permute(idx, 16)
    assert np.array_equal(cpp_to_torch(xstar_cpp.to_cpu(perm), (160,)).numpy(), r["perm"])


# ------------------------------------------------------------------ rmsnorm
def test_rmsnorm_validation_messages():
    """Checks and messages of xstar_cpp/src/ops/rmsnorm.cpp:9-16, raised before
    any device work; CPU tensors are an unsupported device (no CPU compute)."""
    x = torch_to_cpp(torch.randn(4, 32))
    w = torch_to_cpp(torch.randn(32))
    wb = torch_to_cpp(torch.randn(32).to(torch.bfloat16))
    with pytest.raises(RuntimeError, match="x and weight must have the same dtype"):
        xstar_cpp.rmsnorm(x, wb, 1e-5)
    with pytest.raises(RuntimeError, match="rank >= 1 and weight 1D"):
        xstar_cpp.rmsnorm(x, torch_to_cpp(torch.randn(2, 16)), 1e-5)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.rmsnorm(x, torch_to_cpp(torch.randn(31)), 1e-5)
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.rmsnorm(x, w, 1e-5)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.rmsnorm_quant_fp8(torch_to_cpp(torch.randn(4, 96)), torch_to_cpp(torch.randn(96)), 1e-5)


def test_moe_norm_weight_validation():
    x, wr, (w13, s13, w2, s2) = _weights()
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        xstar_cpp.moe(torch_to_cpp(x), torch_to_cpp(wr), None, w13, s13, w2, s2, top_k=2,
                      norm_weight=torch_to_cpp(torch.ones(256)))
    with pytest.raises(RuntimeError, match="shape mismatch"):
        xstar_cpp.moe(torch_to_cpp(x), torch_to_cpp(wr), None, w13, s13, w2, s2, top_k=2,
                      norm_weight=torch_to_cpp(torch.ones(128).to(torch.bfloat16)))
