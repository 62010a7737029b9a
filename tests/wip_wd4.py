"""Weight-direct MXFP4 GEMMs (moe_gemm_wd4.hip, fragment-packed e2m1 weights
and e8m0 scales loaded into registers) against the MXFP4 tiles of
moe_gemm.hip at the same tile height: the same MFMA sequence in K order and
the same epilogue, so the same bits; and C5 at full size against the oracle."""
import numpy as np
import pytest
import torch

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


def test_pack_weight_mxfp4_frag():
    import xs_moe_capi as X
    rng = np.random.default_rng(3)
    b, n, k = 2, 48, 512
    w = rng.integers(0, 256, size=(b, n, k // 2), dtype=np.uint8)
    s = rng.integers(0, 256, size=(b, n, k // 32), dtype=np.uint8)
    gw, gs = X.pack_weight_mxfp4_frag(torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda())
    # [b][n/16][k/128][lane 16 g + r][16 B] = w[b][16 t + r][64 ks + 16 g ...]
    ew = w.reshape(b, n // 16, 16, k // 128, 4, 16).transpose(0, 1, 3, 4, 2, 5).reshape(b, n, k // 2)
    # [b][n/16][k/128][lane 16 g + r] = s[b][16 t + r][4 ks + g]
    es = s.reshape(b, n // 16, 16, k // 128, 4).transpose(0, 1, 3, 4, 2).reshape(b, n, k // 32)
    assert np.array_equal(gw.cpu().numpy(), ew) and np.array_equal(gs.cpu().numpy(), es)


def _debug_rows(R, I, H):
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    return dict(act_q=z((R, I), torch.uint8), act_s=z((R, I // 32), torch.uint8), y_rows=z((R, H), torch.float32))


@pytest.mark.parametrize("T,H,I,E,k,zipf,seed", [
    (300, 1024, 512, 16, 4, None, 71),     # 64-row tiles, ragged last tiles
    (300, 1024, 512, 4, 2, 1.1, 72),       # experts of several tiles
    (900, 1024, 512, 8, 2, None, 73),      # 128-row tiles
    (2048, 4096, 2048, 256, 6, None, 74),  # C5 shape
])
def test_fp4_weight_direct_matches_tiled(T, H, I, E, k, zipf, seed, monkeypatch):
    print(f"case T={T} H={H} I={I} E={E} k={k}", flush=True)
    monkeypatch.setenv("XS_MOE_STREAM", "0")      # the reference path: one block per tile
    _, g = make_case_gpu(T, H, I, E, k, seed=seed, zipf=zipf, fp4=True, host=False)
    R = T * k + T
    tiled = layer_for({"k": k, "fp4": True}, g)
    direct = layer_for({"k": k, "fp4": True}, g, frag=True)
    d0, d1 = _debug_rows(R, I, H), _debug_rows(R, I, H)
    monkeypatch.setenv("XS_FP4_DIRECT", "0")
    a = tiled.forward(g["x"], debug=d0)
    monkeypatch.setenv("XS_FP4_DIRECT", "1")
    b = direct.forward(g["x"], debug=d1)
    b2 = direct.forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(d0["act_q"], d1["act_q"]) and torch.equal(d0["act_s"], d1["act_s"])
    assert torch.equal(d0["y_rows"], d1["y_rows"])
    assert torch.equal(a, b) and torch.equal(b, b2)


def test_fp4_weight_direct_c5_oracle(monkeypatch):
    """C5 (2048 tokens, 256 MXFP4 experts top-6 + FP8 shared) through the
    weight-direct MXFP4 GEMMs: routing bit-exact given the GPU's logits, the
    sampled rows within 2e-2 of the oracle's dequantize-then-f32 layer."""
    monkeypatch.setenv("XS_FP4_DIRECT", "1")
    T = 2048
    c, g = make_case_gpu(T, 4096, 2048, 256, 6, seed=75, fp4=True)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    dbg = dict(logits=z((T, 256), torch.float32), topk_idx=z((T, 6), torch.int32))
    out = layer_for(c, g, frag=True).forward(g["x"], debug=dbg)
    torch.cuda.synchronize()
    d = {n: t.cpu().numpy() for n, t in dbg.items()}
    rows = np.array([0, 1, 2, 517, 1023, 1500, 2046, 2047])
    r = oracle_forward(c, logits_in=np.ascontiguousarray(d["logits"][rows]), rows=rows)
    assert np.array_equal(d["topk_idx"][rows], r["idx"])
    err = max_abs_rel(out.float().cpu().numpy()[rows], r["out_f32"])
    print(f"C5 rows={rows.tolist()} max-abs-rel={err:.3e}")
    assert err <= 2e-2, err
