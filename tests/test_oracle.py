"""Pins the CPU oracle (oracle/) against library answers, the reference's own
code (golden vectors from oracle/_ref) and mathematics.  CPU only."""
import math
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def codecs():
    return np.load(os.path.join(GOLD, "codecs.npz"))


@pytest.fixture(scope="module")
def refv():
    return np.load(os.path.join(GOLD, "ref_vectors.npz"))


# ------------------------------------------------------------------ codecs
def test_e4m3_decode_matches_torch_table(codecs):
    ours = oracle.e4m3_table()
    ref = codecs["e4m3_table"]
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(ours[fin], ref[fin])


def test_e4m3_encode_matches_torch_rne(codecs):
    x = codecs["e4m3_enc_in"]
    got = oracle.e4m3_encode(x)
    assert np.array_equal(got, codecs["e4m3_enc_out"])


def test_e4m3_encode_saturates_and_bruteforce():
    tab = oracle.e4m3_table()
    assert oracle.e4m3_encode(np.array([1e6, -1e6, 500.0, 448.0], np.float32)).tolist() == [0x7E, 0xFE, 0x7E, 0x7E]
    # brute force nearest-even over the finite positive codes
    fin = np.array([c for c in range(127)], dtype=np.int64)
    vals = tab[fin]
    rng = np.random.default_rng(0)
    xs = rng.uniform(0, 448, 3000).astype(np.float32)
    got = oracle.e4m3_encode(xs)
    for x, g in zip(xs, got):
        d = np.abs(vals.astype(np.float64) - float(x))
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
        assert g == want


def test_e2m1_table_and_encode_bruteforce():
    # OCP MX v1.0 E2M1: bias 1, subnormal 0.5
    want = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    tab = oracle.e2m1_table()
    assert tab[:8].tolist() == want and tab[8:].tolist() == [-v for v in want]
    L = oracle.lib()
    vals = np.array(want, np.float64)
    for x in np.concatenate([np.linspace(0, 7, 2801), np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])]):
        d = np.abs(vals - x)
        best = np.flatnonzero(d == d.min())
        code = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
        if x > 6:
            code = 7
        assert L.xo_e2m1_encode(float(x)) == code, x
        assert L.xo_e2m1_encode(float(-x)) == (code | 8 if x != 0 else L.xo_e2m1_encode(-0.0))


def test_e8m0_matches_torch(codecs):
    ours = oracle.e8m0_table()
    ref = codecs["e8m0_table"]
    assert np.isnan(ours[255]) and np.isnan(ref[255])
    assert np.array_equal(ours[:255], ref[:255])


def test_bf16_rne_matches_torch_and_reference(codecs, refv):
    L = oracle.lib()
    x = codecs["bf16_in"]
    assert np.array_equal(oracle.bf16_from_f32(x), codecs["bf16_out"])
    sample = x[:2000]
    assert [L.xo_bf16_from_f32(float(v)) for v in sample] == codecs["bf16_out"][:2000].tolist()
    # the reference's own bfloat16(float) (xstar_cpp/src/bfloat16.cpp:5-25)
    assert np.array_equal(oracle.bf16_from_f32(refv["bf16_in"]), refv["bf16_out"])


# ------------------------------------------------------------- scalar math
def test_expf_accuracy():
    L = oracle.lib()
    xs = np.concatenate([np.linspace(-103.9, 88.7, 20011), np.linspace(-1, 1, 2001)]).astype(np.float32)
    for x in xs:
        got = np.float32(L.xo_expf(float(x)))
        ref = math.exp(float(x))
        if ref < 1.2e-38:   # subnormal results: absolute check
            assert abs(float(got) - ref) <= 2 ** -149 * 1.01
            continue
        ulp = np.spacing(np.float32(ref))
        assert abs(float(got) - ref) <= 2 * ulp, (x, got, ref)
    assert L.xo_expf(0.0) == 1.0
    assert L.xo_expf(-200.0) == 0.0 and math.isinf(L.xo_expf(100.0))


def test_sigmoid_silu_vs_reference(refv):
    """Against the reference's own sigmoid/silu (mlp.cpp:10-26, libm expf):
    within 2 ulp (the oracle uses its own reproducible exp)."""
    L = oracle.lib()
    xs = refv["act_x"]
    for i in range(0, xs.size, 7):
        x = float(xs[i])
        s = np.float32(L.xo_sigmoid(x))
        r = refv["sigmoid"][i]
        assert abs(float(s) - float(r)) <= 2 * np.spacing(np.float32(r)) + 2.0 ** -148
        sl = np.float32(L.xo_silu(x))
        rs = refv["silu"][i]
        # subnormal sigmoid values (x < -87) carry an absolute error of ~2^-149 times |x|
        assert abs(float(sl) - float(rs)) <= 3 * np.spacing(np.float32(abs(rs))) + abs(x) * 2.0 ** -147
    # branched form: no overflow at large |x|
    assert L.xo_sigmoid(-1000.0) == 0.0 and L.xo_sigmoid(1000.0) == 1.0


# ------------------------------------------------------------------ router
def test_router_logits_bitexact_vs_reference_gemm(refv):
    for name in ("g1", "g2", "g3"):
        A, B, Cm = refv[f"{name}_A"], refv[f"{name}_B"], refv[f"{name}_C"]
        got = oracle.router_logits(A, B, is_bf16=False)
        assert np.array_equal(got, Cm), name
        # bf16 inputs: the reference casts the f32 accumulator to bf16 once
        Ab, Bb, Cb = refv[f"{name}_Ab"], refv[f"{name}_Bb"], refv[f"{name}_Cb"]
        gotb = oracle.router_logits(Ab, Bb, is_bf16=True)
        assert np.array_equal(oracle.bf16_from_f32(gotb), Cb), name


def test_router_logits_vs_torch_matmul():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 512)).astype(np.float32)
    w = rng.standard_normal((16, 512)).astype(np.float32) * 0.02
    got = oracle.router_logits(x, w, False)
    ref = (torch.from_numpy(x).double() @ torch.from_numpy(w).double().T).numpy()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def _brute_route(logits, bias, k, n_group=1, topk_group=1, renorm=True, scaling=1.0):
    L = oracle.lib()
    T, E = logits.shape
    idx = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        s = np.array([L.xo_sigmoid(float(v)) for v in logits[t]], np.float32)
        key = s + (bias if bias is not None else np.float32(0))
        allowed = np.ones(E, bool)
        if n_group > 1:
            gs = E // n_group
            gsc = [np.float32(np.sort(key[g * gs:(g + 1) * gs])[-1]) + np.float32(np.sort(key[g * gs:(g + 1) * gs])[-2]) for g in range(n_group)]
            order = sorted(range(n_group), key=lambda g: (-gsc[g], g))[:topk_group]
            allowed[:] = False
            for g in order:
                allowed[g * gs:(g + 1) * gs] = True
        cand = sorted([e for e in range(E) if allowed[e]], key=lambda e: (-key[e], e))[:k]
        idx[t] = cand
        sel = s[cand]
        den = np.float32(0)
        for v in sel:
            den = np.float32(den + v)
        w[t] = [np.float32(np.float32(v / den) * np.float32(scaling)) if renorm else np.float32(v * np.float32(scaling)) for v in sel]
    return idx, w


@pytest.mark.parametrize("E,k,ng,tg", [(8, 2, 1, 1), (16, 6, 1, 1), (64, 6, 8, 3), (256, 6, 1, 1)])
def test_route_vs_bruteforce(E, k, ng, tg):
    rng = np.random.default_rng(E + k)
    T = 37
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    idx, w = oracle.route(logits, bias, k, ng, tg, True, 2.5)
    bidx, bw = _brute_route(logits, bias, k, ng, tg, True, 2.5)
    assert np.array_equal(idx, bidx)
    assert np.array_equal(w, bw)
    for t in range(T):
        assert len(set(idx[t].tolist())) == k
    assert np.allclose(w.sum(1), 2.5, rtol=1e-5)


def test_route_ties_go_to_lower_index_and_bias_free_is_topk_of_logits():
    logits = np.zeros((3, 8), np.float32)
    logits[1, [2, 5, 6]] = 1.0
    idx, w = oracle.route(logits, None, 2)
    assert idx[0].tolist() == [0, 1]
    assert idx[1].tolist() == [2, 5]
    assert np.allclose(w, 0.5)
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((50, 32)).astype(np.float32)
    idx, _ = oracle.route(lg, None, 4)
    ref = np.argsort(-lg, axis=1, kind="stable")[:, :4]   # sigmoid is monotonic
    assert np.array_equal(idx, ref)


def test_route_unnormalized_weights_are_scores():
    rng = np.random.default_rng(6)
    lg = rng.standard_normal((10, 16)).astype(np.float32)
    idx, w = oracle.route(lg, None, 3, renormalize=False, scaling=1.0)
    L = oracle.lib()
    for t in range(10):
        for j in range(3):
            assert w[t, j] == np.float32(L.xo_sigmoid(float(lg[t, idx[t, j]])))


# ----------------------------------------------------------------- permute
@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (64, 8, 2), (100, 256, 6), (0, 4, 2)])
def test_permute_vs_lexsort(T, E, k):
    rng = np.random.default_rng(T)
    idx = np.array([rng.permutation(E)[:k] for _ in range(T)], dtype=np.int32).reshape(T, k)
    counts, offsets, perm, inv = oracle.permute(idx, E)
    flat = idx.ravel()
    assert counts.tolist() == np.bincount(flat, minlength=E).tolist()
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    ref = np.lexsort((np.arange(T * k), flat)) if T else np.zeros(0, np.int64)
    assert np.array_equal(perm, ref)
    assert np.array_equal(inv[perm], np.arange(T * k))


# -------------------------------------------------------------- quantizers
def test_quant_act_fp8_roundtrip_and_scale():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    x[1, :128] = 0
    q, s = oracle.quant_act_fp8(x)
    tab = oracle.e4m3_table()
    deq = tab[q] * np.repeat(s, 128, axis=1)
    amax = np.abs(x.reshape(4, 4, 128)).max(-1)
    assert s[1, 0] == 1.0 and (q[1, :128] == 0).all()
    nz = amax > 0
    assert np.array_equal(s[nz], (amax[nz] / np.float32(448)).astype(np.float32))
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 of the group amax-scaled value
    assert np.all(np.abs(deq - x) <= np.repeat(amax / 448 * 2.0 ** -9 * 448 / 8 + 1e-30, 128, 1) + np.abs(x) * 2 ** -4)
    # the group max is representable: it round-trips to amax (within one rounding)
    for r in range(4):
        for g in range(4):
            if amax[r, g] > 0:
                j = np.argmax(np.abs(x[r, g * 128:(g + 1) * 128])) + g * 128
                assert abs(abs(deq[r, j]) - amax[r, g]) <= amax[r, g] * 1e-6


def test_quant_weight_blocks_and_mx():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    q, s = oracle.quant_weight_fp8_block(w)
    assert q.shape == (256, 384) and s.shape == (2, 3)
    deq = oracle.dequant_weight_fp8_block(q, s)
    assert np.max(np.abs(deq - w)) <= np.max(np.abs(w)) / 448 * 16 + 1e-9
    assert np.abs(deq - w).mean() < 0.02 * 0.03
    q4, s4 = oracle.quant_weight_mxfp4(w)
    assert q4.shape == (256, 192) and s4.shape == (256, 12)
    d4 = oracle.dequant_weight_mxfp4(q4, s4)
    # per 32-block: scale 2^(floor(log2 amax) - 2) so amax/scale in [4, 8): max |v| maps to 4..6
    amax = np.abs(w.reshape(256, 12, 32)).max(-1)
    sc = oracle.e8m0_table()[s4]
    assert np.all((amax / sc >= 4) & (amax / sc < 8))
    assert np.abs(d4 - w).mean() < 0.02 * 0.15
    qa, sa = oracle.quant_act_mxfp8(w)
    amax32 = np.abs(w.reshape(256, 12, 32)).max(-1)
    sca = oracle.e8m0_table()[sa]
    assert np.all((amax32 / sca >= 256) & (amax32 / sca < 512))


# ------------------------------------------------------------- full layer
def _mk(T, H, I, E, seed, std=0.02):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, H)) * std).astype(np.float32)
    wr = (rng.standard_normal((E, H)) * std).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * I, H)) * std).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * std).astype(np.float32)
    return x, wr, w13, w2


def test_ref_path_reduces_to_reference_mlp(refv):
    """E = 1, k = 1, no shared: MoE(x) = mlp(x) bit for bit (reference mlp() golden)."""
    x, w13, w2 = refv["mlp_x"], refv["mlp_w13"], refv["mlp_w2"]
    wr = np.ones((1, x.shape[1]), np.float32)
    got = oracle.moe_ref_f32(x, wr, None, w13[None], w2[None], k=1)
    assert np.array_equal(got, refv["mlp_y"])


def test_ref_path_identical_experts_with_shared_is_twice_mlp(refv):
    x, w13, w2 = refv["mlp_x"], refv["mlp_w13"], refv["mlp_w2"]
    E = 8
    rng = np.random.default_rng(11)
    wr = (rng.standard_normal((E, x.shape[1])) * 0.02).astype(np.float32)
    got = oracle.moe_ref_f32(x, wr, None, np.repeat(w13[None], E, 0), np.repeat(w2[None], E, 0), k=2,
                             shared=(w13, w2))
    assert np.allclose(got, 2 * refv["mlp_y"], rtol=1e-5, atol=1e-9)


def test_gate_up_order_known_answer():
    """tests/ops/test_cpp_mlp.py:129-153 of the reference: x = 1, gate rows 0.125,
    up rows 1.25 -> gate = 1, up = 10, act = silu(1)*10 = 7.3105857...; swapping
    the halves gives silu(10)*1 = 9.9995."""
    H, I = 8, 6
    x = np.ones((2, H), np.float32)
    w13 = np.ones((2 * I, H), np.float32)
    w13[:I] = 0.125
    w13[I:] = 1.25
    w2 = np.zeros((H, I), np.float32)
    w2[0, :] = 1.0
    y = oracle.moe_ref_f32(x, np.ones((1, H), np.float32), None, w13[None], w2[None], k=1)
    assert abs(y[0, 0] - 6 * 7.310585786300049) < 1e-4
    assert np.all(y[:, 1:] == 0)


def test_quant_path_close_to_f32_path_and_torch():
    """Quantized oracle vs (a) torch f32 on the dequantized operands with the same
    routing, (b) the unquantized reference path (FP8 error budget)."""
    torch = pytest.importorskip("torch")
    T, H, I, E, k = 64, 256, 128, 8, 2
    x, wr, w13, w2 = _mk(T, H, I, E, 21)
    sw13 = w13[0] * 1.1
    sw2 = w2[0] * 0.9
    q13, s13 = oracle.quant_weight_fp8_block(w13)
    q2, s2 = oracle.quant_weight_fp8_block(w2)
    qs13, ss13 = oracle.quant_weight_fp8_block(sw13)
    qs2, ss2 = oracle.quant_weight_fp8_block(sw2)
    r = oracle.moe_forward(x, wr, None, q13, s13, q2, s2, k, shared=(qs13, ss13, qs2, ss2))
    # (a) torch f32 with identical quantized activations and routing
    d13 = torch.from_numpy(oracle.dequant_weight_fp8_block(q13, s13)).double()
    d2 = torch.from_numpy(oracle.dequant_weight_fp8_block(q2, s2)).double()
    ds13 = torch.from_numpy(oracle.dequant_weight_fp8_block(qs13, ss13)).double()
    ds2 = torch.from_numpy(oracle.dequant_weight_fp8_block(qs2, ss2)).double()
    xq, xs = oracle.quant_act_fp8(x)
    a = torch.from_numpy(oracle.e4m3_table()[xq] * np.repeat(xs, 128, 1)).double()

    def expert(av, W13, W2):
        gu = av @ W13.T
        g, u = gu[:, :I], gu[:, I:]
        act = (g * torch.sigmoid(g) * u).float().numpy()
        aq, as_ = oracle.quant_act_fp8(act)
        a2 = torch.from_numpy(oracle.e4m3_table()[aq] * np.repeat(as_, 128, 1)).double()
        return a2 @ W2.T

    out = expert(a, ds13, ds2)
    for t in range(T):
        for j in range(k):
            out[t] += float(r["w"][t, j]) * expert(a[t:t + 1], d13[r["idx"][t, j]], d2[r["idx"][t, j]])[0]
    ref = out.numpy()
    err = np.abs(r["out_f32"] - ref).max() / np.abs(ref).max()
    assert err < 2e-3, err
    # (b) vs the unquantized f32 reference path
    ref32 = oracle.moe_ref_f32(x, wr, None, w13, w2, k=k, shared=(sw13, sw2))
    err32 = np.abs(r["out_f32"] - ref32).max() / np.abs(ref32).max()
    assert err32 < 0.1, err32


def test_quant_path_fp4_vs_torch():
    torch = pytest.importorskip("torch")
    T, H, I, E, k = 16, 256, 128, 8, 2
    x, wr, w13, w2 = _mk(T, H, I, E, 22)
    q13, s13 = oracle.quant_weight_mxfp4(w13)
    q2, s2 = oracle.quant_weight_mxfp4(w2)
    r = oracle.moe_forward(x, wr, None, q13, s13, q2, s2, k, routed_fp4=True)
    d13 = torch.from_numpy(oracle.dequant_weight_mxfp4(q13, s13)).double()
    d2 = torch.from_numpy(oracle.dequant_weight_mxfp4(q2, s2)).double()
    xq, xs = oracle.quant_act_mxfp8(x)
    e8 = oracle.e8m0_table()
    a = torch.from_numpy(oracle.e4m3_table()[xq] * np.repeat(e8[xs], 32, 1)).double()
    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = r["idx"][t, j]
            gu = a[t:t + 1] @ d13[e].T
            g, u = gu[:, :I], gu[:, I:]
            act = (g * torch.sigmoid(g) * u).float().numpy()
            aq, as_ = oracle.quant_act_mxfp8(act)
            a2 = torch.from_numpy(oracle.e4m3_table()[aq] * np.repeat(e8[as_], 32, 1)).double()
            ref[t] += float(r["w"][t, j]) * (a2 @ d2[e].T).numpy()[0]
    err = np.abs(r["out_f32"] - ref).max() / np.abs(ref).max()
    assert err < 2e-3, err


# ------------------------------------------------------------------ RMSNorm
def _torch_rmsnorm_layer(x, w, eps, ieee=True):
    """The reference's Python layer (xstar/layers/rmsnorm.py:44-58): f32
    statistics, normalise in f32, cast back, multiply by the weight in the
    input dtype.  ieee=True writes its rsqrt as 1 / sqrt, the form of the C++
    CPU path (rmsnorm.cpp:44,67)."""
    import torch
    xf = x.to(torch.float32)
    ms = xf.pow(2).mean(-1, keepdim=True) + eps
    rms = 1.0 / torch.sqrt(ms) if ieee else torch.rsqrt(ms)
    return w * (xf * rms).to(x.dtype)


def _bits(t):
    import torch
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("shape,eps", [((4, 32), 1e-5), ((3, 1024), 1e-6), ((5, 2048), 1e-5), ((2, 1), 1e-5)])
def test_rmsnorm_bitexact_on_exact_sums(bf16, shape, eps):
    """x on a 1/8 grid in [-1, 1]: every square and partial sum is exact in f32,
    so torch's reduction order cannot matter and the reference layer's steps
    (mean, + eps, sqrt, divide, normalise, cast, weight) give the oracle's bits.
    Pins eps inside the sqrt, the division by hidden, (x * inv) * w in f32 and
    the two bf16 roundings."""
    import torch
    g = torch.Generator().manual_seed(shape[-1])
    dt = torch.bfloat16 if bf16 else torch.float32
    x = (torch.randint(-8, 9, shape, generator=g).float() / 8).to(dt)
    w = torch.randn(shape[-1], generator=g).to(dt)
    ref = _torch_rmsnorm_layer(x, w, eps)
    got = oracle.rmsnorm(_bits(x), _bits(w), eps, bf16=bf16)
    assert np.array_equal(got, _bits(ref))


def test_rmsnorm_bf16_double_rounding_is_visible():
    """The bf16 path rounds x * inv to bf16 before the weight multiply
    (rmsnorm.cpp:72).  Find inputs where one rounding of x * inv * w gives
    another bf16 value and check the oracle keeps the two roundings."""
    import torch
    g = torch.Generator().manual_seed(7)
    x = (torch.randint(-8, 9, (64, 32), generator=g).float() / 8).to(torch.bfloat16)
    w = torch.randn(32, generator=g).to(torch.bfloat16)
    xf = x.float()
    inv = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)
    single = (xf * inv * w.float()).to(torch.bfloat16)
    double = _torch_rmsnorm_layer(x, w, 1e-5)
    assert not torch.equal(single, double)
    got = oracle.rmsnorm(_bits(x), _bits(w), 1e-5, bf16=True)
    assert np.array_equal(got, _bits(double))


@pytest.mark.parametrize("bf16,shape,rtol,atol", [(False, (4, 32), 0, 1e-6), (False, (16,), 0, 1e-6),
                                                  (False, (4, 1024), 0, 1e-4), (True, (4, 32), 0, 1e-2),
                                                  (True, (8, 7168), 1e-2, 1e-2)])
def test_rmsnorm_vs_reference_layer(bf16, shape, rtol, atol):
    """randn inputs against the reference layer as written (torch.rsqrt), to the
    tolerances of tests/ops/test_cpp_rmsnorm.py:30,51,140 and
    tests/ops/test_cpp_cuda_rmsnorm.py:111-116."""
    import torch
    g = torch.Generator().manual_seed(11)
    dt = torch.bfloat16 if bf16 else torch.float32
    x = torch.randn(shape, generator=g).to(dt)
    w = torch.randn(shape[-1], generator=g).to(dt)
    ref = _torch_rmsnorm_layer(x, w, 1e-5, ieee=False).float().numpy()
    got = oracle.rmsnorm(_bits(x), _bits(w), 1e-5, bf16=bf16)
    got = oracle.f32_from_bf16(got) if bf16 else got
    assert np.allclose(got, ref, rtol=rtol, atol=atol)


def test_rmsnorm_closed_forms():
    """Zero rows give exact zeros (eps keeps them finite,
    tests/ops/test_cpp_rmsnorm.py:76-95); hidden = 1 gives x / sqrt(x^2 + eps) * w;
    a constant row c gives c / sqrt(c^2 + eps) * w."""
    z = oracle.rmsnorm(np.zeros((4, 32), np.float32), np.ones(32, np.float32), 1e-5)
    assert np.array_equal(z, np.zeros((4, 32), np.float32))
    x = np.array([[3.0], [-0.5], [1e-3], [0.0]], np.float32)
    w = np.array([1.5], np.float32)
    h1 = oracle.rmsnorm(x, w, 1e-5)
    ref = x.astype(np.float64) / np.sqrt(x.astype(np.float64) ** 2 + np.float64(np.float32(1e-5))) * 1.5
    assert np.allclose(h1, ref, rtol=3e-7, atol=0)
    c = np.full((1, 256), 0.75, np.float32)
    wc = np.linspace(-2, 2, 256, dtype=np.float32)
    yc = oracle.rmsnorm(c, wc, 1e-6)
    ref = 0.75 / math.sqrt(0.5625 + float(np.float32(1e-6))) * wc.astype(np.float64)
    assert np.allclose(yc[0], ref, rtol=3e-7, atol=1e-12)
