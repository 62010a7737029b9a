"""Packed-only layers: the routed (and shared) expert weights given only in
fragment order, every GEMM a weight-direct one.  Against the same layer with
row-major weights on the one-block-per-tile kernels (stream-K off: it splits
K), the outputs are the same bits at every batch size, including the
mid-size batches that a packed-only layer sends to the 128-row prefill kernel."""
import pytest
import torch

from moe_cases import make_case_gpu, layer_for

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


@pytest.mark.parametrize("T,fp4", [
    (1, False), (16, False),          # 16-row decode tiles
    (100, False), (600, False),       # mid-size: 32/64-row tiles row-major, 128-row packed-only
    (4096, False),                    # tall tiles
    (16, True), (300, True), (2048, True),
])
def test_packed_only_matches_row_major(T, fp4, monkeypatch):
    H, I, E, k = (1024, 512, 64, 6) if T < 2048 else (4096, 2048, 256, 6)
    print(f"case T={T} fp4={fp4} H={H} I={I} E={E}", flush=True)
    monkeypatch.setenv("XS_MOE_STREAM", "0")
    _, g = make_case_gpu(T, H, I, E, k, seed=80 + T, fp4=fp4, host=False)
    ref = layer_for({"k": k, "fp4": fp4}, g)
    only = layer_for({"k": k, "fp4": fp4}, g, frag="only")
    assert only.w13 is None and only.w2 is None
    a = ref.forward(g["x"])
    b = only.forward(g["x"])
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_cpp_block_ffn_packed_only(tmp_path):
    """pack_moe_layer_frag(w, packed_only=True) drops the row-major weights;
    moe_block_ffn then gives the bits it gave before."""
    import numpy as np
    import xstar_cpp
    from safetensors.torch import save_file
    from bridge import torch_to_cpp, cpp_to_torch
    from moe_cases import make_case
    from test_gpu_weights import _checkpoint
    T, H, I, E, k = 40, 512, 512, 16, 4
    c = make_case(T, H, I, E, k, seed=11)
    p = str(tmp_path / "l.safetensors")
    save_file(_checkpoint(c, "blk.mlp"), p)
    w = xstar_cpp.load_moe_layer([p], "blk.mlp")
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)  # noqa: E731
    ht = xstar_cpp.to_cuda(torch_to_cpp(bf(c["x"])))
    ln = xstar_cpp.to_cuda(torch_to_cpp(bf(np.full(H, 0x3f80, np.uint16))))
    before = cpp_to_torch(xstar_cpp.to_cpu(xstar_cpp.moe_block_ffn(ht, ln, 1e-6, w, top_k=k)), (T, H))
    xstar_cpp.pack_moe_layer_frag(w, packed_only=True)
    assert w.w13 is None and w.w2 is None and w.shared_w13 is None and w.w13_frag is not None
    after = cpp_to_torch(xstar_cpp.to_cpu(xstar_cpp.moe_block_ffn(ht, ln, 1e-6, w, top_k=k)), (T, H))
    assert torch.equal(before.view(torch.int16), after.view(torch.int16))
