"""Weight-direct prefill GEMMs (fragment-packed FP8 weights loaded into
registers): the packing against its definition, and whole layers with and
without the packed copies, which must give the same bits (the same per-row
arithmetic in the same order)."""
import numpy as np
import pytest
import torch

from moe_cases import make_case_gpu
from moe_synth import layer_from

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


def _pack_ref(w):
    """[batch, n, k] u8 -> the fragment order of xs_pack_weight_fp8_frag:
    [batch][n/16][k/128][h][lane][16 B] = w[b][16 t + lane % 16][128 kb + 64 h + 16 (lane // 16) ...]."""
    b, n, k = w.shape
    x = w.reshape(b, n // 16, 16, k // 128, 2, 4, 16)          # b, t, r, kb, h, g, byte
    x = x.transpose(0, 1, 3, 4, 5, 2, 6)                       # b, t, kb, h, g, r, byte (lane = 16 g + r)
    return np.ascontiguousarray(x).reshape(b, n, k)


@pytest.mark.parametrize("b,n,k", [(1, 16, 128), (2, 48, 384), (3, 256, 1024)])
def test_pack_weight_fp8_frag(b, n, k):
    import xs_moe_capi as X
    rng = np.random.default_rng(b * n + k)
    w = rng.integers(0, 256, size=(b, n, k), dtype=np.uint8)
    got = X.pack_weight_fp8_frag(torch.from_numpy(w).cuda()).cpu().numpy()
    assert np.array_equal(got, _pack_ref(w))


def _debug_rows(T, k, I, H, shared):
    R = T * k + (T if shared else 0)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device="cuda")  # noqa: E731
    return dict(act_q=z((R, I), torch.uint8), act_s=z((R, I // 128), torch.float32), y_rows=z((R, H), torch.float32))


@pytest.mark.parametrize("T,H,I,E,k,zipf,seed,shared", [
    (2048, 1024, 512, 32, 6, 1.1, 31, True),     # skewed: full, partial and one-row tiles
    (1500, 1024, 1024, 16, 4, None, 32, False),  # ragged last tiles, no shared expert
])
def test_moe_weight_direct_matches_lds_ring(T, H, I, E, k, zipf, seed, shared, monkeypatch):
    monkeypatch.setenv("XS_MOE_GEMM", "wide")
    _, g = make_case_gpu(T, H, I, E, k, seed=seed, zipf=zipf, shared=shared, host=False)
    ring = layer_from(g)
    direct = layer_from(g, frag=True)
    d0, d1 = _debug_rows(T, k, I, H, shared), _debug_rows(T, k, I, H, shared)
    a = ring.forward(g["x"], debug=d0)
    b = direct.forward(g["x"], debug=d1)
    b2 = direct.forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(d0["act_q"], d1["act_q"]) and torch.equal(d0["act_s"], d1["act_s"])
    assert torch.equal(d0["y_rows"], d1["y_rows"])
    assert torch.equal(a, b) and torch.equal(b, b2)
    # the switch back to the LDS-ring kernels gives the same bits as well
    monkeypatch.setenv("XS_WIDE_DIRECT", "0")
    c = direct.forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(a, c)


def test_moe_weight_direct_full_size_c3():
    """The bench's prefill layer (8192 tokens, 256 experts top-6 + shared,
    Zipf(1.1)): identical output with the packed weights."""
    _, g = make_case_gpu(8192, 4096, 2048, 256, 6, seed=0, zipf=1.1, host=False)
    a = layer_from(g).forward(g["x"])
    b = layer_from(g, frag=True).forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(a, b)
