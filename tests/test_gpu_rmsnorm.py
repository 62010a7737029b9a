"""GPU parity of RMSNorm and its fused FP8 output (xs_rmsnorm) and of the MoE
layer's pre-norm, through the C ABI, against the CPU oracle.

Bars:
  - x on a 1/8 grid: every partial sum of squares is exact, so the GPU's
    reduction order cannot matter and y is bit-exact with the oracle;
  - randn x: the tolerances of the reference's own tests
    (tests/ops/test_cpp_rmsnorm.py:30,51 and tests/ops/test_cpp_cuda_rmsnorm.py:30-35,
    111-116: f32 atol 1e-6, bf16 rtol = atol = 1e-2), plus at most two bf16 codes;
  - fused FP8 output: bit-exact with the oracle's quantization of the GPU's y
    (same values in, same codes out);
  - MoE with has_norm: bit-exact with the layer run on xs_rmsnorm's output, and
    within 2e-2 max-abs-rel of the oracle chain."""
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


def _dev(a):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t.view(torch.bfloat16) if a.dtype == np.uint16 else t).cuda()


def _host(t):
    t = t.cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _inputs(shape, bf16, seed, grid=False):
    rng = np.random.default_rng(seed)
    if grid:
        x = rng.integers(-8, 9, shape).astype(np.float32) / 8
    else:
        x = rng.standard_normal(shape).astype(np.float32)
    w = rng.standard_normal(shape[-1]).astype(np.float32)
    if bf16:
        return oracle.bf16_from_f32(x), oracle.bf16_from_f32(w)
    return x, w


def _run(x, w, eps, quant=False):
    import xs_moe_capi as X
    print(f"rmsnorm x{list(x.shape)} {x.dtype} eps={eps} quant={quant}", flush=True)
    r = X.rmsnorm(_dev(x), _dev(w), eps, quant=quant)
    torch.cuda.synchronize()
    return tuple(_host(t) for t in r) if quant else _host(r)


# shapes: the wave kernel at 1..14 chunks per lane and its partial last chunk
# (896 = 1.75 chunks), the one-block-per-row kernel (hidden % 8 != 0, > 8192)
SHAPES = [(4, 32), (16,), (3, 1), (5, 7), (4, 896), (2, 3, 1024), (6, 4096), (9, 7168), (8, 8192), (3, 10000)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm_bitexact_on_exact_sums(shape, bf16):
    x, w = _inputs(shape, bf16, seed=sum(shape), grid=True)
    y = _run(x, w, 1e-5)
    assert np.array_equal(y, oracle.rmsnorm(x, w, 1e-5, bf16=bf16))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm_randn_within_reference_tolerance(shape, bf16):
    x, w = _inputs(shape, bf16, seed=3 + sum(shape))
    y = _run(x, w, 1e-6)
    ref = oracle.rmsnorm(x, w, 1e-6, bf16=bf16)
    if bf16:
        yf, rf = oracle.f32_from_bf16(y), oracle.f32_from_bf16(ref)
        assert np.allclose(yf, rf, rtol=1e-2, atol=1e-2)
        # one ulp of inv moves bf16(x * inv) by at most one code, and the
        # weight multiply's rounding then by at most one more
        assert np.abs(y.astype(np.int32) - ref.astype(np.int32)).max() <= 2
    else:
        assert np.allclose(y, ref, rtol=0, atol=1e-6 * max(1.0, float(np.abs(ref).max())))


@pytest.mark.parametrize("hidden", [1, 8, 24])
def test_rmsnorm_sqrt_and_division_rounding(hidden):
    """65536 rows of grid values and spread magnitudes: sum / hidden + eps takes
    many distinct values, so an approximate sqrt or division shows as one-ulp
    differences in f32 y (hidden 1: block kernel; 8, 24: wave kernel)."""
    rng = np.random.default_rng(hidden)
    x = (rng.integers(-8, 9, (65536, hidden)).astype(np.float32) / 8)
    x *= np.exp2(rng.integers(-20, 20, (65536, 1))).astype(np.float32)
    w = rng.standard_normal(hidden).astype(np.float32)
    y = _run(x, w, 1e-5)
    assert np.array_equal(y, oracle.rmsnorm(x, w, 1e-5))


@pytest.mark.parametrize("bf16", [False, True])
def test_rmsnorm_zero_rows_and_empty(bf16):
    x, w = _inputs((4, 512), bf16, seed=5, grid=True)
    x[1] = 0
    y = _run(x, w, 1e-5)
    yv = oracle.f32_from_bf16(y[1]) if bf16 else y[1]
    assert np.all(yv == 0)                       # eps keeps the zero row finite and zero (+-0)
    assert np.array_equal(y, oracle.rmsnorm(x, w, 1e-5, bf16=bf16))
    # zero rows: no work, no error
    import xs_moe_capi as X
    X.check(X.lib().xs_rmsnorm(None, None, X.XS_BF16 if bf16 else X.XS_F32, 0, 512, 1e-5, None, None, None,
                               X._stream()))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("shape,grid", [((37, 512), True), ((37, 512), False), ((8, 7168), False),
                                        ((5, 10240), False), ((3, 896 + 128), False)])
def test_rmsnorm_fused_fp8_bitexact(shape, grid, bf16):
    """q, s equal the oracle's FP8 1x128 quantization of the GPU's y."""
    x, w = _inputs(shape, bf16, seed=11, grid=grid)
    x[2, :128] = 0                              # an all-zero group
    y, q, s = _run(x, w, 1e-6, quant=True)
    yf = oracle.f32_from_bf16(y) if bf16 else y
    rq, rs = oracle.quant_act_fp8(yf)
    assert np.array_equal(q, rq)
    assert np.array_equal(s, rs)
    assert np.array_equal(y, _run(x, w, 1e-6))  # the fused kernel's y is the plain kernel's y
    if grid:
        assert np.array_equal(y, oracle.rmsnorm(x, w, 1e-6, bf16=bf16))


def test_rmsnorm_misaligned_rows_take_the_block_kernel():
    """A base pointer off the 16-byte grid goes to the one-block-per-row kernel;
    results are the same bits on exact sums."""
    import xs_moe_capi as X
    x, w = _inputs((6, 1024), True, seed=9, grid=True)
    big = torch.zeros(6 * 1024 + 1, dtype=torch.bfloat16, device="cuda")
    big[1:] = _dev(x).reshape(-1)
    xv = big[1:].view(6, 1024)
    yv = torch.empty(6 * 1024 + 1, dtype=torch.bfloat16, device="cuda")[1:].view(6, 1024)
    X.check(X.lib().xs_rmsnorm(X._ptr(xv), X._ptr(_dev(w)), X.XS_BF16, 6, 1024, 1e-5, X._ptr(yv), None, None,
                               X._stream()))
    torch.cuda.synchronize()
    assert np.array_equal(_host(yv), oracle.rmsnorm(x, w, 1e-5, bf16=True))


def test_rmsnorm_full_size_c3():
    """8192 x 7168 bf16 (the prefill shape): randn within two bf16 codes of the
    oracle, fused FP8 equal to the oracle's quantization of y."""
    x, w = _inputs((8192, 7168), True, seed=21)
    y, q, s = _run(x, w, 1e-6, quant=True)
    ref = oracle.rmsnorm(x, w, 1e-6, bf16=True)
    d = np.abs(y.astype(np.int32) - ref.astype(np.int32))
    assert d.max() <= 2 and (d > 0).mean() < 1e-3
    rows = np.arange(0, 8192, 97)
    rq, rs = oracle.quant_act_fp8(oracle.f32_from_bf16(y[rows]))
    assert np.array_equal(q[rows], rq) and np.array_equal(s[rows], rs)


def test_cpp_rmsnorm_matches_capi():
    import xstar_cpp
    from bridge import torch_to_cpp, cpp_to_torch
    x, w = _inputs((4, 896), True, seed=4)
    xt, wt = torch.from_numpy(x).view(torch.bfloat16), torch.from_numpy(w).view(torch.bfloat16)
    yc = xstar_cpp.rmsnorm(xstar_cpp.to_cuda(torch_to_cpp(xt)), xstar_cpp.to_cuda(torch_to_cpp(wt)), 1e-6)
    got = cpp_to_torch(xstar_cpp.to_cpu(yc), (4, 896)).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, _run(x, w, 1e-6))
    with pytest.raises(RuntimeError, match="device mismatch"):
        xstar_cpp.rmsnorm(xstar_cpp.to_cuda(torch_to_cpp(xt)), torch_to_cpp(wt), 1e-6)


# ------------------------------------------------------------ MoE pre-norm
@pytest.mark.parametrize("T,fp4,shared", [(64, False, True), (300, False, True), (48, True, True), (40, True, False)])
def test_moe_prenorm_equals_norm_then_moe(T, fp4, shared):
    """moe(x, norm_weight) = moe(rmsnorm(x)) bit for bit (same kernels downstream),
    and within 2e-2 of the oracle's rmsnorm -> MoE chain."""
    from moe_cases import make_case, to_device, layer_for, oracle_forward, max_abs_rel
    import xs_moe_capi as X
    H, I, E, k = 512, 256, 16, 4
    c = make_case(T, H, I, E, k, seed=T, fp4=fp4, shared=shared)
    g = to_device(c)
    nw = oracle.bf16_from_f32((1.0 + 0.1 * np.random.default_rng(T).standard_normal(H)).astype(np.float32))
    nwd = _dev(nw)
    print(f"moe prenorm T={T} fp4={fp4} shared={shared}", flush=True)
    logits = torch.empty((T, E), dtype=torch.float32, device="cuda")
    out_n = layer_for(c, g, norm_weight=nwd, norm_eps=1e-6).forward(g["x"], debug={"logits": logits})
    xn = X.rmsnorm(g["x"], nwd, 1e-6)
    out_ref = layer_for(c, g).forward(xn)
    torch.cuda.synchronize()
    assert torch.equal(out_n.view(torch.int16), out_ref.view(torch.int16))
    cn = dict(c)
    cn["x"] = _host(xn)
    rn = oracle.rmsnorm(c["x"], nw, 1e-6, bf16=True)
    assert np.abs(cn["x"].astype(np.int32) - rn.astype(np.int32)).max() <= 2
    r = oracle_forward(cn, logits_in=logits.cpu().numpy())
    assert max_abs_rel(out_n.float().cpu().numpy(), r["out_f32"]) <= 2e-2


# ------------------------------------------------- residual / block FFN half
def _f32_copy(c):
    """The same case with x and router_w as f32 (the bf16 values widened)."""
    cf = dict(c)
    cf["x"] = oracle.f32_from_bf16(c["x"])
    cf["router_w"] = oracle.f32_from_bf16(c["router_w"])
    return cf


@pytest.mark.parametrize("T,shared", [(64, True), (300, False)])
def test_moe_residual_is_added_before_the_one_rounding(T, shared):
    """f32 layer: out(residual=h) == h + out() in f32, bit for bit (also in place).
    bf16 layer: out(residual=h) == bf16(f32(h) + out_f32), the f32 layer's output
    being the combine's f32 sum (exact routers on both sides)."""
    from moe_cases import make_case, to_device, layer_for
    H, I, E, k = 512, 256, 16, 4
    c = make_case(T, H, I, E, k, seed=7 + T, shared=shared)
    cf = _f32_copy(c)
    gf = to_device(cf)
    print(f"moe residual T={T} shared={shared}", flush=True)
    Lf = layer_for(cf, gf, router_exact=True)
    base = Lf.forward(gf["x"])
    h = torch.randn((T, H), generator=torch.Generator(device="cuda").manual_seed(T), device="cuda")
    withr = Lf.forward(gf["x"], residual=h)
    inplace = h.clone()
    Lf.forward(gf["x"], out=inplace, residual=inplace)
    torch.cuda.synchronize()
    ref = h.cpu().numpy() + base.cpu().numpy()
    assert np.array_equal(withr.cpu().numpy(), ref)
    assert np.array_equal(inplace.cpu().numpy(), ref)
    g = to_device(c)
    hb = h.to(torch.bfloat16)
    outb = layer_for(c, g, router_exact=True).forward(g["x"], residual=hb)
    torch.cuda.synchronize()
    want = oracle.bf16_from_f32(oracle.f32_from_bf16(_host(hb)) + base.cpu().numpy())
    assert np.array_equal(_host(outb), want)


def test_moe_block_ffn_from_a_checkpoint(tmp_path):
    """xstar_cpp.moe_block_ffn(h, ln2_w, eps, load_moe_layer(...)) equals the
    layer with pre-norm and residual through the C ABI, bit for bit, and the
    unfused h + moe(rmsnorm(h)) within two bf16 codes of the output."""
    import xstar_cpp
    from safetensors.torch import save_file
    from bridge import torch_to_cpp, cpp_to_torch
    from moe_cases import make_case, to_device, layer_for
    from test_gpu_weights import _checkpoint
    import xs_moe_capi as X
    T, H, I, E, k = 96, 512, 256, 16, 4
    c = make_case(T, H, I, E, k, seed=5)
    p = str(tmp_path / "l.safetensors")
    save_file(_checkpoint(c, "blk.mlp"), p)
    w = xstar_cpp.load_moe_layer([p], "blk.mlp")
    ln = oracle.bf16_from_f32((1 + 0.1 * np.random.default_rng(1).standard_normal(H)).astype(np.float32))
    print("moe_block_ffn", flush=True)
    ht = xstar_cpp.to_cuda(torch_to_cpp(_t_bf16(c["x"])))
    out = xstar_cpp.moe_block_ffn(ht, xstar_cpp.to_cuda(torch_to_cpp(_t_bf16(ln))), 1e-6, w, top_k=k)
    got = cpp_to_torch(xstar_cpp.to_cpu(out), (T, H))
    g = to_device(c)
    lnd = _dev(ln)
    # the C ABI layers on the C++ op's default (certified) router
    fused = layer_for(c, g, router_exact=None, norm_weight=lnd, norm_eps=1e-6).forward(g["x"], residual=g["x"])
    moe_out = layer_for(c, g, router_exact=None).forward(X.rmsnorm(g["x"], lnd, 1e-6))
    unfused = g["x"].float() + moe_out.float()
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), fused.cpu().view(torch.int16))
    # the unfused path rounds the MoE output to bf16 before the add: the two
    # differ by at most half an ulp of that output plus one rounding of the sum
    # each (value-based: where h + moe cancels, the first term dominates)
    def ulp(v):
        return np.exp2(np.floor(np.log2(np.maximum(np.abs(v), 1e-30))) - 7)
    a = fused.float().cpu().numpy()
    b = unfused.to(torch.bfloat16).float().cpu().numpy()
    m = moe_out.float().cpu().numpy()
    assert np.all(np.abs(a - b) <= ulp(np.maximum(np.abs(a), np.abs(b))) + ulp(m) / 2)


def _t_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)
