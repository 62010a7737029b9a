"""GPU parity of the individual stages against the CPU oracle, through the C ABI.

Bit-exact: activation/weight quantizers, exact router logits, routing
(indices and weights, given the same logits), permutation.  Tolerance: MFMA
router logits and the single FP8 block-scaled GEMM."""
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


def _bf16_dev(a_u16):
    return torch.from_numpy(a_u16).view(torch.bfloat16).cuda()


def _cases_act(rng):
    x = rng.standard_normal((37, 512)).astype(np.float32)
    x[3, :128] = 0.0                       # all-zero group
    x[4, 384:] = -0.0                      # all-zero group of negative zeros (FP8: code 0)
    x[5, 128:256] *= 1e4                   # large
    x[6, 256:384] *= 1e-30                 # tiny (subnormal after scaling)
    x[7, 0] = 3.0e38                       # near f32 max
    return x


def test_quant_act_fp8_bitexact():
    import xs_moe_capi as X
    rng = np.random.default_rng(1)
    x = _cases_act(rng)
    # f32 input
    q, s = X.quant_act_fp8(torch.from_numpy(x).cuda())
    rq, rs = oracle.quant_act_fp8(x)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)
    # bf16 input
    xb = oracle.bf16_from_f32(x)
    q, s = X.quant_act_fp8(_bf16_dev(xb))
    rq, rs = oracle.quant_act_fp8(oracle.f32_from_bf16(xb))
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


def test_quant_act_mxfp8_bitexact():
    import xs_moe_capi as X
    rng = np.random.default_rng(2)
    x = _cases_act(rng)
    q, s = X.quant_act_mxfp8(torch.from_numpy(x).cuda())
    rq, rs = oracle.quant_act_mxfp8(x)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)


def test_quant_weight_fp8_and_mxfp4_bitexact():
    import xs_moe_capi as X
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((3, 256, 384)) * 0.02).astype(np.float32)
    w[1, :128, :128] = 0.0
    q, s = X.quant_weight_fp8_block(torch.from_numpy(w).cuda())
    rq, rs = oracle.quant_weight_fp8_block(w)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    wb = oracle.bf16_from_f32(w)
    q, s = X.quant_weight_fp8_block(_bf16_dev(wb))
    rq, rs = oracle.quant_weight_fp8_block(oracle.f32_from_bf16(wb))
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    q4, s4 = X.quant_weight_mxfp4(torch.from_numpy(w).cuda())
    rq4, rs4 = oracle.quant_weight_mxfp4(w)
    assert np.array_equal(s4.cpu().numpy(), rs4) and np.array_equal(q4.cpu().numpy(), rq4)


def test_hw_fp8_pack_matches_software_rne():
    """The activation quantizer and the GEMM epilogue pack with the hardware
    converter (after clamping to +-448): pin it against the software RNE
    encoder of the oracle over every e4m3 code boundary (midpoints and
    neighbours, subnormals included) in [-448, 448]."""
    import xs_moe_capi as X
    tab = oracle.e4m3_table()
    fin = np.unique(np.abs(tab[np.isfinite(tab)]))
    mids = (fin[1:] + fin[:-1]) / 2
    near = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), fin])
    vals = np.concatenate([near, -near]).astype(np.float32)
    vals = vals[np.abs(vals) <= 448.0]
    rows = (vals.size + 127) // 128
    x = np.zeros(rows * 128, np.float32)
    x[:vals.size] = vals
    # quant with amax forced to 448 (scale 1): prepend nothing; each row's amax
    # is <= 448, so compare the library's GEMM-free encoder path via the act
    # quantizer at scale 1 by building rows whose amax is exactly 448
    x = x.reshape(rows, 128)
    x[:, 0] = 448.0
    q, s = X.quant_act_fp8(torch.from_numpy(x).cuda())
    rq, rs = oracle.quant_act_fp8(x)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.all(rs == 1.0)


@pytest.mark.parametrize("bf16", [False, True])
def test_router_logits_exact_bitexact(bf16):
    import xs_moe_capi as X
    rng = np.random.default_rng(4)
    T, E, H = 70, 24, 512
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    if bf16:
        xb, wb = oracle.bf16_from_f32(x), oracle.bf16_from_f32(w)
        got = X.router_logits(_bf16_dev(xb), _bf16_dev(wb), exact=True).cpu().numpy()
        ref = oracle.router_logits(xb, wb, True)
    else:
        got = X.router_logits(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), exact=True).cpu().numpy()
        ref = oracle.router_logits(x, w, False)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T,E,H", [(130, 256, 4096), (1000, 256, 4096), (2048, 198, 1024), (300, 130, 512)])
def test_router_logits_mfma_tolerance(T, E, H):
    """Decode (T <= 256: fragments from global memory) and prefill (LDS-tiled
    kernel, ragged token and expert tiles) bf16 MFMA router logits."""
    import xs_moe_capi as X
    rng = np.random.default_rng(5 + T)
    xb = oracle.bf16_from_f32(rng.standard_normal((T, H)).astype(np.float32))
    wb = oracle.bf16_from_f32((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    got = X.router_logits(_bf16_dev(xb), _bf16_dev(wb), exact=False).cpu().numpy()
    ref = (oracle.f32_from_bf16(xb).astype(np.float64) @ oracle.f32_from_bf16(wb).astype(np.float64).T)
    # f32 accumulation of 4096 exact bf16 products: |err| <= ~K * eps * sum|x w|
    bound = 4096 * 2 ** -24 * (np.abs(oracle.f32_from_bf16(xb)) @ np.abs(oracle.f32_from_bf16(wb)).T)
    assert np.all(np.abs(got - ref) <= bound + 1e-6)


@pytest.mark.parametrize("E,k,ng,tg,scale,renorm", [
    (8, 2, 1, 1, 1.0, True), (256, 6, 1, 1, 1.0, True), (256, 8, 8, 4, 2.5, True),
    (64, 6, 1, 1, 1.0, False), (1024, 16, 1, 1, 1.0, True), (96, 4, 32, 8, 1.5, True)])
def test_route_bitexact(E, k, ng, tg, scale, renorm):
    import xs_moe_capi as X
    rng = np.random.default_rng(E * 10 + k)
    T = 301
    logits = rng.standard_normal((T, E)).astype(np.float32) * 2
    logits[0, :] = 0.5                              # all tied
    logits[1, : E // 2] = logits[1, E // 2:]        # pairwise ties
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    idx, w = X.route(torch.from_numpy(logits).cuda(), torch.from_numpy(bias).cuda(), k, ng, tg,
                     renorm, scale)
    ridx, rw = oracle.route(logits, bias, k, ng, tg, renorm, scale)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(w.cpu().numpy(), rw)
    idx, w = X.route(torch.from_numpy(logits).cuda(), None, k, ng, tg, renorm, scale)
    ridx, rw = oracle.route(logits, None, k, ng, tg, renorm, scale)
    assert np.array_equal(idx.cpu().numpy(), ridx) and np.array_equal(w.cpu().numpy(), rw)


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (64, 8, 2), (16, 256, 6), (1000, 256, 6), (8192, 256, 6), (33, 1024, 16)])
def test_permute_bitexact(T, E, k):
    import xs_moe_capi as X
    rng = np.random.default_rng(T + E)
    if E >= 64:
        # skewed: most tokens pick from the first experts
        pref = np.argsort(rng.random((T, E)) * (np.arange(E) + 1) ** 1.5, axis=1)
        idx = pref[:, :k].astype(np.int32)
    else:
        idx = np.array([rng.permutation(E)[:k] for _ in range(T)], np.int32)
    counts, offsets, perm, inv = X.permute(torch.from_numpy(idx).cuda(), E)
    rc, ro, rp, ri = oracle.permute(idx, E)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(offsets.cpu().numpy(), ro)
    assert np.array_equal(perm.cpu().numpy(), rp)
    assert np.array_equal(inv.cpu().numpy(), ri)


@pytest.mark.parametrize("case", ["out_of_range", "negative", "duplicate"])
def test_permute_rejects_invalid_idx(case):
    """The public permute checks its precondition (experts in [0, E), distinct
    within a row) and fails with the documented error; a valid call after it
    still matches the oracle (the error leaves no state behind)."""
    import xs_moe_capi as X
    rng = np.random.default_rng(7)
    T, E, k = 100, 16, 4
    idx = np.array([rng.permutation(E)[:k] for _ in range(T)], np.int32)
    bad = idx.copy()
    if case == "out_of_range":
        bad[37, 2] = E
    elif case == "negative":
        bad[99, 3] = -1
    else:
        bad[5, 3] = bad[5, 0]
    msg = "outside" if case != "duplicate" else "twice"
    with pytest.raises(X.XsError, match=msg):
        X.permute(torch.from_numpy(bad).cuda(), E)
    counts, offsets, perm, inv = X.permute(torch.from_numpy(idx).cuda(), E)
    rc, ro, rp, ri = oracle.permute(idx, E)
    assert np.array_equal(counts.cpu().numpy(), rc) and np.array_equal(perm.cpu().numpy(), rp)
    assert np.array_equal(inv.cpu().numpy(), ri) and np.array_equal(offsets.cpu().numpy(), ro)


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (40, 256, 384), (1, 128, 128), (2100, 512, 1024),
                                   (200, 1024, 4096), (130, 384, 2048), (33000, 256, 256)])
def test_gemm_fp8_blockscale(M, N, K):
    """C = dequant(quant1x128(A)) . dequant(B)^T vs a float64 reference on the
    same quantized operands (the activation quantizer is bit-exact, so the
    difference is accumulation order and the bf16 output cast)."""
    import xs_moe_capi as X
    rng = np.random.default_rng(M + N + K)
    a = oracle.bf16_from_f32(rng.standard_normal((M, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bq, bs = oracle.quant_weight_fp8_block(w)
    out = X.gemm_fp8_blockscale(_bf16_dev(a), torch.from_numpy(bq).cuda(), torch.from_numpy(bs).cuda())
    got = out.float().cpu().numpy()
    aq, as_ = oracle.quant_act_fp8(oracle.f32_from_bf16(a))
    ad = oracle.e4m3_table()[aq].astype(np.float64) * np.repeat(as_, 128, 1)
    bd = oracle.dequant_weight_fp8_block(bq, bs).astype(np.float64)
    ref = ad @ bd.T
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 4e-3, err
    # split-K partials are summed in split order: a second call gives the same bits
    again = X.gemm_fp8_blockscale(_bf16_dev(a), torch.from_numpy(bq).cuda(), torch.from_numpy(bs).cuda())
    assert torch.equal(again, out)
