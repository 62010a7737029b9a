"""xs_moe_forward_noalloc (the forward on the library's static per-GPU scratch,
for callers that cannot allocate) against xs_moe_forward with a workspace:
identical outputs bit for bit, on two calls in a row with the second call on a
smaller input (the scratch keeps the first call's contents), for FP8 decode,
FP8 prefill-shaped tiles and MXFP4; oversized params are rejected."""
import pytest

from moe_cases import make_case, make_case_gpu, to_device, layer_for

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _both(layer, x):
    out_ws = layer.forward(x)
    out_na = torch.empty_like(out_ws)
    layer.forward_noalloc(x, out_na)
    torch.cuda.synchronize()
    return out_ws, out_na


@pytest.mark.parametrize("T1,T2,H,I,E,k,fp4", [
    (256, 16, 4096, 2048, 256, 6, False),    # V4-Flash shape: the scratch limit's design point, then decode
    (700, 100, 1024, 1024, 16, 4, False),    # tall tiles, then the smaller tiled GEMMs
    (160, 48, 512, 512, 16, 6, True)])       # MXFP4 routed experts + FP8 shared
def test_noalloc_matches_workspace_forward(T1, T2, H, I, E, k, fp4):
    if H == 4096:
        c, g = make_case_gpu(T1, H, I, E, k, seed=71, fp4=fp4, host=False)
        c = {"k": k, "fp4": fp4}
    else:
        c = make_case(T1, H, I, E, k, seed=72, fp4=fp4, zipf=1.1)
        g = to_device(c)
    layer = layer_for(c, g)
    x1 = g["x"]
    x2 = x1[:T2].clone()
    a1, b1 = _both(layer, x1)
    a2, b2 = _both(layer, x2)
    assert torch.equal(a1, b1)
    assert torch.equal(a2, b2)
    assert not torch.equal(a1[:T2], torch.zeros_like(a1[:T2]))


def test_noalloc_rejects_params_beyond_the_scratch():
    import xs_moe_capi as X
    c, g = make_case_gpu(1, 4096, 2048, 256, 6, seed=73, host=False)
    layer = layer_for({"k": 6, "fp4": False}, g)
    x = torch.zeros((4096, 4096), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(x)
    with pytest.raises(X.XsError, match="static scratch"):
        layer.forward_noalloc(x, out)


@pytest.mark.parametrize("env,T1,T2,H,I,E,k", [
    # stream-K counters and partial tiles (zeroed by the preceding launches)
    ({"XS_MOE_GEMM": "tiled", "XS_MOE_STREAM": "1", "XS_STREAM_GROUPED": "0"}, 256, 40, 1024, 1024, 64, 4),
    # the fused combine's per-(token, slab) counters on the tall tiles
    ({"XS_MOE_GEMM": "wide", "XS_FUSE_COMBINE": "1"}, 700, 300, 1024, 1024, 16, 4),
    # the certified router's pair and token counters, every token through the exact pass
    ({"XS_ROUTER_MARGIN": "1e30"}, 200, 20, 1024, 512, 32, 6),
])
def test_noalloc_counters_are_rearmed(env, T1, T2, H, I, E, k, monkeypatch):
    """State that must start at zero in every forward (stream-K counters, the
    fused combine's counters, the certified router's list counters) lives in
    the shared scratch: a larger forward and then a smaller one through the
    scratch equal the workspace forward bit for bit."""
    for n, v in env.items():
        monkeypatch.setenv(n, v)
    c = make_case(T1, H, I, E, k, seed=74, zipf=1.1)
    g = to_device(c)
    layer = layer_for(c, g, router_exact=None)
    plan = layer.plan(T1)
    if "XS_MOE_STREAM" in env:
        assert plan["routed"] == "stream"
    if "XS_FUSE_COMBINE" in env:
        assert plan["fused_combine"]
    x1 = g["x"]
    x2 = x1[:T2].clone()
    a1, b1 = _both(layer, x1)
    a2, b2 = _both(layer, x2)
    assert torch.equal(a1, b1)
    assert torch.equal(a2, b2)
