"""The MoE forward under HIP graph capture (torch.cuda.CUDAGraph): every replay
equals the eager output bit for bit, with the program's own eager forwards and
synchronisations between the replays.  The forward records no memset (its
persistent-GEMM counters are cleared by the permute kernel), so a captured
graph replays the same work each time; the certified router's list
counters are cleared by its logits launch the same way.  Also: the
activation quant folded into the decode router launch equals the separate
quant pass."""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import xs_moe_capi  # noqa: F401  (fails loudly when the library is missing)


@pytest.mark.parametrize("T,stream,norm,router,margin", [
    (16, "1", False, "mfma", None), (16, "0", True, "mfma", None), (200, "1", True, "mfma", None),
    (64, "0", False, "mfma", None),
    # the default certified router: the one route launch at decode, the three
    # launches at prefill, and with every token through the exact pass
    (16, "1", False, "certified", None), (300, "0", False, "certified", None),
    (16, "1", False, "certified", "1e30"), (300, "0", True, "certified", "1e30")])
def test_graph_replays_equal_eager(monkeypatch, T, stream, norm, router, margin):
    from moe_cases import make_case, to_device, layer_for
    monkeypatch.setenv("XS_MOE_STREAM", stream)
    if margin:
        monkeypatch.setenv("XS_ROUTER_MARGIN", margin)
    H, I, E, k = 512, 256, 16, 4
    c = make_case(max(T, 40), H, I, E, k, seed=T)
    g = to_device(c)
    kw = {}
    if norm:
        kw = dict(norm_weight=torch.ones(H, dtype=torch.bfloat16, device="cuda"), norm_eps=1e-6)
    if router == "certified":
        kw["router_exact"] = None
    L = layer_for(c, g, **kw)
    x = g["x"][:T].contiguous()
    other = g["x"][T // 2:T // 2 + 7].contiguous()
    print(f"graph T={T} XS_MOE_STREAM={stream} norm={norm} router={router} margin={margin}", flush=True)
    eager = L.forward(x).clone()
    out = torch.empty_like(eager)
    res = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on the capture stream (workspace allocated here)
        L.forward(x, out=out, residual=res if norm else None)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        L.forward(x, out=out, residual=res if norm else None)
    want = L.forward(x, residual=res).clone() if norm else eager
    for rep in range(4):
        out.zero_()
        L.forward(other)            # eager work between replays, same workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {rep}"


@pytest.mark.parametrize("T", [1, 16, 100, 256])
def test_router_folded_quant_equals_separate_quant(monkeypatch, T):
    """Decode batches quantize the activations inside the router launch; the
    layer output equals the one with the separate quant pass, bit for bit."""
    from moe_cases import make_case, to_device, layer_for
    H, I, E, k = 1024, 256, 32, 4
    c = make_case(T, H, I, E, k, seed=100 + T)
    g = to_device(c)
    L = layer_for(c, g)
    print(f"fold quant T={T}", flush=True)
    monkeypatch.setenv("XS_FOLD_QUANT", "1")
    a = L.forward(g["x"]).clone()
    monkeypatch.setenv("XS_FOLD_QUANT", "0")
    b = L.forward(g["x"]).clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
