"""Weight-direct decode GEMMs (moe_gemm_wdd.hip, fragment-packed FP8 weights
loaded into registers) against the one-block-per-tile kernels of the same
16-row tiles: the same per-row arithmetic in the same order, so the same bits;
and the whole layer against the oracle at the V4-Flash decode shape."""
import pytest
import torch

import numpy as np

from moe_cases import make_case_gpu, layer_for, oracle_forward, max_abs_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    # the weight-direct GEMMs are opt-in; these tests are theirs
    mp = pytest.MonkeyPatch()
    mp.setenv("XS_WEIGHT_DIRECT", "1")
    yield
    mp.undo()


def _debug_rows(R, I, H):
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    return dict(act_q=z((R, I), torch.uint8), act_s=z((R, I // 128), torch.float32), y_rows=z((R, H), torch.float32))


@pytest.mark.parametrize("T,H,I,E,k,zipf,seed,shared", [
    (1, 1024, 512, 32, 4, None, 51, True),       # one row per expert
    (5, 512, 1024, 16, 4, None, 52, False),      # no shared expert
    (16, 2048, 1024, 64, 6, None, 53, True),
    (40, 1024, 512, 8, 2, 1.1, 54, True),        # experts of several 16-row tiles, ragged last tiles
    (1, 4096, 2048, 256, 6, None, 55, True),     # V4-Flash decode, T = 1
    (16, 4096, 2048, 256, 6, None, 56, True),    # T = 16
    (256, 4096, 2048, 256, 6, None, 57, True),   # T = 256 (16-row tiles, shared expert in 16 tiles)
])
def test_decode_weight_direct_matches_tiled(T, H, I, E, k, zipf, seed, shared, monkeypatch):
    print(f"case T={T} H={H} I={I} E={E} k={k} shared={shared}", flush=True)
    monkeypatch.setenv("XS_MOE_STREAM", "0")      # the reference path: one block per 16-row tile
    monkeypatch.setenv("XS_MOE_GEMM", "tiled")
    c, g = make_case_gpu(T, H, I, E, k, seed=seed, zipf=zipf, shared=shared, host=False)
    R = T * k + (T if shared else 0)
    tiled = layer_for({"k": k, "fp4": False}, g)
    direct = layer_for({"k": k, "fp4": False}, g, frag=True)
    d0, d1 = _debug_rows(R, I, H), _debug_rows(R, I, H)
    monkeypatch.setenv("XS_DECODE_DIRECT", "0")
    a = tiled.forward(g["x"], debug=d0)
    monkeypatch.setenv("XS_DECODE_DIRECT", "1")
    b = direct.forward(g["x"], debug=d1)
    b2 = direct.forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(d0["act_q"], d1["act_q"]) and torch.equal(d0["act_s"], d1["act_s"])
    assert torch.equal(d0["y_rows"], d1["y_rows"])
    assert torch.equal(a, b) and torch.equal(b, b2)


@pytest.mark.parametrize("T", [1, 16])
def test_decode_weight_direct_v4_oracle(T, monkeypatch):
    """C4 at full shape (zero router bias) through the weight-direct decode
    GEMMs: routing bit-exact given the GPU's logits, output within 2e-2 of the
    oracle's dequantize-then-f32 layer."""
    monkeypatch.setenv("XS_DECODE_DIRECT", "1")
    c, g = make_case_gpu(T, 4096, 2048, 256, 6, seed=60 + T, bias_std=0)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    dbg = dict(logits=z((T, 256), torch.float32), topk_idx=z((T, 6), torch.int32), inv=z((T * 6,), torch.int32))
    out = layer_for(c, g, frag=True).forward(g["x"], debug=dbg)
    torch.cuda.synchronize()
    d = {n: t.cpu().numpy() for n, t in dbg.items()}
    r = oracle_forward(c, logits_in=d["logits"])
    assert np.array_equal(d["topk_idx"], r["idx"]) and np.array_equal(d["inv"], r["inv"])
    err = max_abs_rel(out.float().cpu().numpy(), r["out_f32"])
    print(f"T={T} max-abs-rel={err:.3e}")
    assert err <= 2e-2, err


@pytest.mark.parametrize("T,H,I,E,k", [
    (8, 512, 512, 16, 4),      # 16-row tiles: the decode GEMMs
    (300, 1024, 512, 8, 2),    # tall tiles: the prefill GEMMs
])
def test_cpp_block_ffn_packed_weights(T, H, I, E, k, tmp_path):
    """xstar_cpp.moe_block_ffn after pack_moe_layer_frag(w) gives the bits it
    gave before packing."""
    import xstar_cpp
    from safetensors.torch import save_file
    from bridge import torch_to_cpp, cpp_to_torch
    from moe_cases import make_case
    from test_gpu_weights import _checkpoint
    print(f"case T={T} H={H} I={I} E={E} k={k}", flush=True)
    c = make_case(T, H, I, E, k, seed=9)
    p = str(tmp_path / "l.safetensors")
    save_file(_checkpoint(c, "blk.mlp"), p)
    w = xstar_cpp.load_moe_layer([p], "blk.mlp")
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)  # noqa: E731
    ht = xstar_cpp.to_cuda(torch_to_cpp(bf(c["x"])))
    ln = xstar_cpp.to_cuda(torch_to_cpp(bf(np.full(H, 0x3f80, np.uint16))))   # ones
    before = cpp_to_torch(xstar_cpp.to_cpu(xstar_cpp.moe_block_ffn(ht, ln, 1e-6, w, top_k=k)), (T, H))
    assert w.w13_frag is None
    xstar_cpp.pack_moe_layer_frag(w)
    assert w.w13_frag is not None and w.shared_w2_frag is not None
    after = cpp_to_torch(xstar_cpp.to_cpu(xstar_cpp.moe_block_ffn(ht, ln, 1e-6, w, top_k=k)), (T, H))
    assert torch.equal(before.view(torch.int16), after.view(torch.int16))
