"""The single FP8 GEMM from fragment-packed B (xs_gemm_fp8_blockscale_packed,
the weight-direct kernel) against a float64 reference on the same quantized
operands, and against xs_gemm_fp8_blockscale on the row-major B."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    # the weight-direct GEMMs are opt-in; these tests are theirs
    mp = pytest.MonkeyPatch()
    mp.setenv("XS_WEIGHT_DIRECT", "1")
    yield
    mp.undo()


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (1, 256, 512), (100, 512, 1024), (130, 768, 1536),
                                   (2100, 1024, 2048), (64, 256, 512)])
def test_gemm_fp8_blockscale_packed(M, N, K):
    import xs_moe_capi as X
    print(f"case M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    a = oracle.bf16_from_f32(rng.standard_normal((M, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bq, bs = oracle.quant_weight_fp8_block(w)
    ad_ = torch.from_numpy(a).view(torch.bfloat16).cuda()
    bq_d, bs_d = torch.from_numpy(bq).cuda(), torch.from_numpy(bs).cuda()
    bp = X.pack_weight_fp8_frag(bq_d)
    out = X.gemm_fp8_blockscale_packed(ad_, bp, bs_d)
    row = X.gemm_fp8_blockscale(ad_, bq_d, bs_d)
    again = X.gemm_fp8_blockscale_packed(ad_, bp, bs_d)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    aq, as_ = oracle.quant_act_fp8(oracle.f32_from_bf16(a))
    ad = oracle.e4m3_table()[aq].astype(np.float64) * np.repeat(as_, 128, 1)
    bd = oracle.dequant_weight_fp8_block(bq, bs).astype(np.float64)
    ref = ad @ bd.T
    err = np.abs(got - ref).max() / np.abs(ref).max()
    print(f"max-abs-rel vs float64 {err:.3e}")
    assert err < 4e-3, err
    # against the LDS-ring kernel: the same products, summed in another order
    d = np.abs(got - row.float().cpu().numpy()).max() / np.abs(ref).max()
    assert d < 4e-3, d
    # deterministic: no K split, every output summed in K order
    assert torch.equal(again, out)


def test_gemm_fp8_blockscale_packed_rejects_shapes():
    import xs_moe_capi as X
    a = torch.zeros((8, 384), dtype=torch.bfloat16, device="cuda")
    b = torch.zeros((256, 384), dtype=torch.uint8, device="cuda")
    s = torch.ones((2, 3), dtype=torch.float32, device="cuda")
    with pytest.raises(X.XsError, match="multiple of 256 and K of 512"):
        X.gemm_fp8_blockscale_packed(a, b, s)
