"""Whole-layer GPU parity (xs_moe_forward through the C ABI) against the CPU
oracle's dequantize-then-f32 path.

Contract: router indices, weights, per-expert counts, offsets and the
permutation are bit-exact (with the exact router, or given the GPU's own
logits with the MFMA router); outputs are within max-abs-rel 2e-2 (max |gpu -
oracle| / max |oracle|), the tolerance the benchmark description states."""
import numpy as np
import pytest

import oracle
from moe_cases import make_case, make_case_gpu, to_device, layer_for, oracle_forward, max_abs_rel

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _debug(T, E, k):
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    return dict(logits=z((T, E), torch.float32), topk_idx=z((T, k), torch.int32),
                topk_w=z((T, k), torch.float32), counts=z((E,), torch.int32),
                offsets=z((E + 1,), torch.int32), perm=z((T * k,), torch.int32),
                inv=z((T * k,), torch.int32))


def _run_and_check(c, g, router_exact, tol=TOL, rows=None):
    T, E, k = c["T"], c["E"], c["k"]
    layer = layer_for(c, g, router_exact=router_exact)
    dbg = _debug(T, E, k)
    out = layer.forward(g["x"], debug=dbg)
    torch.cuda.synchronize()
    d = {n: t.cpu().numpy() for n, t in dbg.items()}
    r = oracle_forward(c, logits_in=None if router_exact else d["logits"])
    if router_exact:
        assert np.array_equal(d["logits"], r["logits"])
    assert np.array_equal(d["topk_idx"], r["idx"])
    assert np.array_equal(d["topk_w"], r["w"])
    assert np.array_equal(d["counts"], r["counts"])
    assert np.array_equal(d["offsets"], r["offsets"])
    assert np.array_equal(d["perm"], r["perm"])
    assert np.array_equal(d["inv"], r["inv"])
    got = out.float().cpu().numpy()
    err = max_abs_rel(got, r["out_f32"])
    print(f"T={T} H={c['H']} I={c['I']} E={E} k={k} fp4={c['fp4']} max-abs-rel={err:.3e}")
    assert err <= tol, err
    return err


def test_moe_c1_tiny_f32():
    """BASELINE config C1 shape: f32, H=256, I=128, E=8, top-2 + shared, 64
    tokens, x and weights ~ N(0, 0.02), zero bias."""
    c = make_case(64, 256, 128, 8, 2, seed=11, x_std=0.02, bf16=False, bias_std=0)
    _run_and_check(c, to_device(c), router_exact=True)


@pytest.mark.parametrize("T,H,I,E,k,shared", [
    (1, 256, 128, 8, 2, True), (5, 512, 256, 16, 4, False), (128, 512, 256, 32, 6, True),
    (600, 512, 256, 16, 2, True), (2048, 512, 256, 8, 1, True)])
def test_moe_bf16_shapes(T, H, I, E, k, shared):
    """Tile heights 16..128 (rows per expert from 0.6 to 512), ragged tiles,
    with and without the shared expert; exact and MFMA routers."""
    c = make_case(T, H, I, E, k, seed=T + E, shared=shared)
    g = to_device(c)
    _run_and_check(c, g, router_exact=True)
    _run_and_check(c, g, router_exact=False)


@pytest.mark.parametrize("T,E,k,zipf,seed", [(700, 16, 4, 1.1, 21), (40, 4, 4, None, 22), (1000, 8, 2, 0.6, 23)])
def test_moe_wide_tiles(T, E, k, zipf, seed):
    """192 x 256-tile FP8 GEMMs (H, I multiples of 1024; experts averaging 32+
    rows): skewed routing gives segments of 1..6 32-row subtiles, multi-tile
    experts and the shared segment; exact and MFMA routers."""
    c = make_case(T, 1024, 1024, E, k, seed=seed, zipf=zipf)
    g = to_device(c)
    _run_and_check(c, g, router_exact=True)
    _run_and_check(c, g, router_exact=False)


@pytest.mark.parametrize("T,H,I,E,k,zipf,seed", [
    (1, 512, 512, 8, 2, None, 31),      # 12 items over 48 K steps and 48 blocks: every item split 4 ways
    (3, 1024, 1024, 16, 4, None, 32),
    (100, 2048, 512, 64, 2, 1.1, 33),   # multi-tile experts and 7 shared tiles (slab-major order)
    (40, 1536, 1024, 8, 6, None, 34),   # 30 rows / expert: 32-row tiles; H % 256 == 0, not % 512
    (16, 1024, 2048, 32, 6, 0.8, 35)])
def test_moe_stream_decode(T, H, I, E, k, zipf, seed, monkeypatch):
    """Persistent (stream-K) decode GEMMs against the oracle, and against the
    one-block-per-tile kernels on the same inputs."""
    c = make_case(T, H, I, E, k, seed=seed, zipf=zipf)
    g = to_device(c)
    outs = []
    for mode in ("1", "0"):
        monkeypatch.setenv("XS_MOE_STREAM", mode)
        _run_and_check(c, g, router_exact=True)
        layer = layer_for(c, g, router_exact=True)
        outs.append(layer.forward(g["x"]).float().cpu().numpy())
        outs.append(layer.forward(g["x"]).float().cpu().numpy())
    assert np.array_equal(outs[0], outs[1])      # repeatable (counters re-armed each call)
    assert max_abs_rel(outs[0], outs[2]) <= 1e-2


def test_moe_group_limited_and_scaling():
    c = make_case(96, 512, 128, 32, 4, seed=3)
    g = to_device(c)
    import xs_moe_capi as X
    layer = X.MoeLayer(g["router_w"], g["w13"], g["s13"], g["w2"], g["s2"], 4, router_bias=g["bias"],
                       shared=g["shared"], n_group=8, topk_group=2, routed_scaling=2.5, router_exact=True)
    out = layer.forward(g["x"])
    r = oracle_forward(c, n_group=8, topk_group=2, scaling=2.5)
    assert max_abs_rel(out.float().cpu().numpy(), r["out_f32"]) <= TOL


@pytest.mark.parametrize("mode", ["0", "1"])
@pytest.mark.parametrize("T", [48, 80, 160, 300])
def test_moe_fp4_small(T, mode, monkeypatch):
    """C5 structure at small size: MXFP4 routed experts, FP8 shared expert;
    18 / 30 / 60 / 112 rows per expert select 16- to 128-row tiles; the
    one-block-per-tile kernels (mode 0) and the persistent ones (mode 1, 16- to
    64-row tiles; K steps in pairs, so H and I are multiples of 512)."""
    monkeypatch.setenv("XS_MOE_STREAM", mode)
    c = make_case(T, 512, 512, 16, 6, seed=5 + T, fp4=True)
    g = to_device(c)
    _run_and_check(c, g, router_exact=True)
    _run_and_check(c, g, router_exact=False)


@pytest.mark.parametrize("T", [1, 16, 64, 256])
def test_moe_v4_decode_full_shape(T):
    """C4 at full V4-Flash shape: H=4096, I=2048, 256 experts top-6 + shared."""
    c, g = make_case_gpu(T, 4096, 2048, 256, 6, seed=40 + T)
    _run_and_check(c, g, router_exact=False)


def test_moe_fp4_full_shape():
    """C5 shape (H=4096, I=2048, 256 MXFP4 experts top-6 + FP8 shared) at 32 tokens."""
    c, g = make_case_gpu(32, 4096, 2048, 256, 6, seed=7, fp4=True)
    _run_and_check(c, g, router_exact=False)


def test_moe_prefill_full_size_properties():
    """C3 at full size (8192 tokens, Zipf(1.1) popularity): routing, counts and
    permutation bit-exact against the oracle on the GPU logits; outputs of a
    sample of tokens against the oracle run on those tokens alone."""
    T, E, k = 8192, 256, 6
    c, g = make_case_gpu(T, 4096, 2048, E, k, seed=8, zipf=1.1)
    layer = layer_for(c, g)
    dbg = _debug(T, E, k)
    out = layer.forward(g["x"], debug=dbg)
    torch.cuda.synchronize()
    d = {n: t.cpu().numpy() for n, t in dbg.items()}
    ridx, rw = oracle.route(d["logits"], c["bias"], k)
    assert np.array_equal(d["topk_idx"], ridx) and np.array_equal(d["topk_w"], rw)
    rc, ro, rp, ri = oracle.permute(ridx, E)
    assert np.array_equal(d["counts"], rc) and np.array_equal(d["offsets"], ro[:E + 1])
    assert np.array_equal(d["perm"], rp) and np.array_equal(d["inv"], ri)
    # Zipf(1.1) profile: a head of experts with thousands of tokens, every expert used
    assert rc.max() > 16 * rc.mean() and (rc > 0).all()
    rows = np.array([0, 1, 777, 4096, 5000, 8191])
    r = oracle_forward(c, logits_in=np.ascontiguousarray(d["logits"][rows]), rows=rows)
    got = out.float().cpu().numpy()[rows]
    assert max_abs_rel(got, r["out_f32"]) <= TOL
    # sum of the routed weights per token is 1 (renormalised)
    assert np.allclose(d["topk_w"].sum(1), 1.0, rtol=1e-5)


def _golden_mlp_case(E, k, shared):
    """The reference's own mlp() test vectors (tests/golden/ref_vectors.npz,
    written by the compiled reference) as an MoE layer: every routed expert and
    the shared expert carry the same FP8-quantized [gate; up] and down weights,
    and a zero router ties every expert (top-k takes the lowest indices with
    renormalised weights 1/k)."""
    import os
    r = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
    x, w13, w2 = r["mlp_x"], r["mlp_w13"], r["mlp_w2"]
    T, H = x.shape
    I = w2.shape[1]
    q13, s13 = oracle.quant_weight_fp8_block(w13[None])
    q2, s2 = oracle.quant_weight_fp8_block(w2[None])
    c = dict(T=T, H=H, I=I, E=E, k=k, bias=None, x=x, router_w=np.zeros((E, H), np.float32),
             w13=np.repeat(q13, E, 0), s13=np.repeat(s13, E, 0), w2=np.repeat(q2, E, 0),
             s2=np.repeat(s2, E, 0), fp4=False,
             shared=(q13[0], s13[0], q2[0], s2[0]) if shared else None)
    return c


def test_moe_reduces_to_reference_mlp_closed_forms():
    """E = 1, top-1, no shared expert: the layer is mlp(x) (checked against the
    oracle, which test_oracle pins to the reference mlp() golden).  E = 4
    identical experts, top-2, plus the same shared expert: the combine sums
    y + y/2 + y/2 of bit-identical expert rows, which is exactly 2 y in f32 and
    in the output cast, so the output is twice the E = 1 output bit for bit."""
    c1 = _golden_mlp_case(1, 1, False)
    g1 = to_device(c1)
    _run_and_check(c1, g1, router_exact=True)
    y1 = layer_for(c1, g1, router_exact=True).forward(g1["x"]).cpu().numpy()
    c4 = _golden_mlp_case(4, 2, True)
    g4 = to_device(c4)
    _run_and_check(c4, g4, router_exact=True)
    y4 = layer_for(c4, g4, router_exact=True).forward(g4["x"]).cpu().numpy()
    assert np.array_equal(y4, 2 * y1)


def test_moe_empty_input():
    """T = 0: the layer returns an empty output and launches nothing."""
    c = make_case(4, 256, 128, 8, 2, seed=5)
    g = to_device(c)
    layer = layer_for(c, g)
    x0 = g["x"][:0]
    out = layer.forward(x0)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (0, 256)


def test_moe_max_experts_and_topk():
    """The C ABI's limits E = 1024 and top_k = 16 through the whole layer
    (permute, tile tables, GEMMs, combine) plus the shared expert, against the
    oracle; exact and MFMA routers."""
    c = make_case(48, 256, 128, 1024, 16, seed=41)
    g = to_device(c)
    _run_and_check(c, g, router_exact=True)
    _run_and_check(c, g, router_exact=False)


def test_moe_prefill_32k_tokens_properties():
    """4x the C3 batch (32768 tokens, 196608 routed rows: beyond the 16-bit row
    tokens of the persistent GEMMs, so the tall-tile path): routing, counts and
    permutation bit-exact against the oracle on the GPU logits, sampled output
    rows against the oracle, routed weights summing to 1."""
    T, E, k = 32768, 256, 6
    c, g = make_case_gpu(T, 4096, 2048, E, k, seed=9, zipf=1.1)
    layer = layer_for(c, g)
    dbg = _debug(T, E, k)
    out = layer.forward(g["x"], debug=dbg)
    torch.cuda.synchronize()
    d = {n: t.cpu().numpy() for n, t in dbg.items()}
    ridx, rw = oracle.route(d["logits"], c["bias"], k)
    assert np.array_equal(d["topk_idx"], ridx) and np.array_equal(d["topk_w"], rw)
    rc, ro, rp, ri = oracle.permute(ridx, E)
    assert np.array_equal(d["counts"], rc) and np.array_equal(d["offsets"], ro[:E + 1])
    assert np.array_equal(d["perm"], rp) and np.array_equal(d["inv"], ri)
    rows = np.array([0, 3, 12345, 16384, 30000, 32767])
    r = oracle_forward(c, logits_in=np.ascontiguousarray(d["logits"][rows]), rows=rows)
    got = out.float().cpu().numpy()[rows]
    assert max_abs_rel(got, r["out_f32"]) <= TOL
    assert np.allclose(d["topk_w"].sum(1), 1.0, rtol=1e-5)
