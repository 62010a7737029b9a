"""The C-ABI library loads on a machine without a GPU and exports every entry
point include/xs_moe.h declares (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "xs_moe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(xs_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_stage_entry_points():
    names = declared_functions()
    for n in ("xs_moe_forward", "xs_moe_route", "xs_moe_permute", "xs_moe_router_logits",
              "xs_quant_act_fp8", "xs_gemm_fp8_blockscale", "xs_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import xs_moe_capi
    if not os.path.exists(xs_moe_capi.LIB_PATH):
        pytest.fail("libxs_moe.so not built (run python xstar-infer_amd/build.py)")
    lib = ctypes.CDLL(xs_moe_capi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers the same set
    assert set(xs_moe_capi.EXPORTS) == set(declared_functions())


def test_argument_validation_without_gpu():
    import xs_moe_capi as X
    L = X.lib()
    p = X.MoeParams(16, 100, 128, 8, 2, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 0, 0)
    assert L.xs_moe_workspace_size(ctypes.byref(p)) == 0          # H % 256 != 0
    p.H = 256
    assert L.xs_moe_workspace_size(ctypes.byref(p)) > 0
    # 32-bit row offsets in the GEMMs: T x H and T x (k + 1) x I below 2^32
    big = X.MoeParams(1 << 20, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 0)
    assert L.xs_moe_workspace_size(ctypes.byref(big)) == 0
    big.T = 299000    # 299000 x 7 x 2048 < 2^32
    assert L.xs_moe_workspace_size(ctypes.byref(big)) > 0
    big.T = 300000
    assert L.xs_moe_workspace_size(ctypes.byref(big)) == 0
    # the router's (token, expert) pair counters are 32-bit: T x E below 2^31
    wide = X.MoeParams(1 << 23, 256, 128, 256, 1, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 0, 0)
    assert L.xs_moe_workspace_size(ctypes.byref(wide)) == 0
    wide.T = (1 << 23) - 1
    assert L.xs_moe_workspace_size(ctypes.byref(wide)) > 0
    rc = L.xs_moe_route(ctypes.c_void_p(16), None, 1 << 23, 256, 6, 1, 1, 1, 1.0, ctypes.c_void_p(16),
                        ctypes.c_void_p(16), None)
    assert rc == 1 and b"T x E" in L.xs_last_error()
    rc = L.xs_moe_route(ctypes.c_void_p(16), None, -1, 8, 2, 1, 1, 1, 1.0, ctypes.c_void_p(16), ctypes.c_void_p(16),
                        None)
    assert rc == 1
    rc = L.xs_moe_router_logits(ctypes.c_void_p(16), ctypes.c_void_p(16), X.XS_BF16, 1 << 22, 512, 128, 1,
                                ctypes.c_void_p(16), None)
    assert rc == 1 and b"T x E" in L.xs_last_error()
    rc = L.xs_moe_route(None, None, 4, 8, 2, 1, 1, 1, 1.0, None, None, None)
    assert rc == 1 and b"null" in L.xs_last_error()
    rc = L.xs_quant_act_fp8(ctypes.c_void_p(16), X.XS_BF16, 4, 100, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == 1 and b"128" in L.xs_last_error()
    rc = L.xs_quant_act_fp8(ctypes.c_void_p(18), X.XS_BF16, 4, 128, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == 1 and b"misaligned" in L.xs_last_error()
    rc = L.xs_rmsnorm(ctypes.c_void_p(16), ctypes.c_void_p(16), X.XS_BF16, 4, 128, 1e-6, ctypes.c_void_p(18),
                      ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == 1 and b"misaligned" in L.xs_last_error()
    rc = L.xs_rmsnorm(ctypes.c_void_p(16), ctypes.c_void_p(16), X.XS_BF16, 4, 96, 1e-6, ctypes.c_void_p(16),
                      ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == 1 and b"hidden % 128" in L.xs_last_error()


def test_packed_weight_validation_without_gpu():
    """The forward's checks of packed-only layers and of the packing entry
    points, which all run before anything touches a GPU."""
    import xs_moe_capi as X
    L = X.lib()
    v = ctypes.c_void_p(4096)   # an aligned stand-in pointer: never dereferenced here
    p = X.MoeParams(16, 256, 256, 8, 2, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 0)
    names = [f[0] for f in X.MoeTensors._fields_]
    def tensors(**given):
        t = X.MoeTensors()
        for n in ("x", "router_w", "out", "w13_scale", "w2_scale", "shared_w13_scale", "shared_w2_scale"):
            setattr(t, n, v)
        for n, val in given.items():
            assert n in names
            setattr(t, n, val)
        return t
    # no row-major weights and no packed copies
    rc = L.xs_moe_forward(ctypes.byref(p), ctypes.byref(tensors()), v, 1 << 30, None)
    assert rc == 1 and b"packed copies" in L.xs_last_error()
    # packed routed weights, but the shared expert's missing
    rc = L.xs_moe_forward(ctypes.byref(p), ctypes.byref(tensors(w13_frag=v, w2_frag=v)), v, 1 << 30, None)
    assert rc == 1 and b"shared expert's packed" in L.xs_last_error()
    # MXFP4 packed-only layers also need the packed scales
    p4 = X.MoeParams(16, 256, 256, 8, 2, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP4_E2M1X2, 0, 0)
    rc = L.xs_moe_forward(ctypes.byref(p4), ctypes.byref(tensors(w13_frag=v, w2_frag=v)), v, 1 << 30, None)
    assert rc == 1 and b"packed copies" in L.xs_last_error()
    # misaligned packed copies
    rc = L.xs_moe_forward(ctypes.byref(p), ctypes.byref(tensors(w13_frag=ctypes.c_void_p(4104), w2_frag=v,
                                                                shared_w13_frag=v, shared_w2_frag=v)),
                          v, 1 << 30, None)
    assert rc == 1 and b"packed weights need 16-byte alignment" in L.xs_last_error()
    # the packing entry points
    rc = L.xs_pack_weight_mxfp4_frag(v, v, 1, 24, 256, ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20), None)
    assert rc == 1 and b"multiple of 16" in L.xs_last_error()
    rc = L.xs_pack_weight_mxfp4_frag(ctypes.c_void_p(4100), v, 1, 16, 256, ctypes.c_void_p(1 << 20),
                                     ctypes.c_void_p(2 << 20), None)
    assert rc == 1 and b"misaligned" in L.xs_last_error()
    rc = L.xs_pack_weight_mxfp4_frag(v, v, 1, 16, 256, v, ctypes.c_void_p(2 << 20), None)
    assert rc == 1 and b"overlap" in L.xs_last_error()
    rc = L.xs_pack_weight_fp8_frag(v, 1, 16, 200, ctypes.c_void_p(1 << 20), None)
    assert rc == 1 and b"multiple of 16" in L.xs_last_error()


def _stand_in_tensors(X, row_major=True, frag=False, fp4=False, shared=True):
    v = ctypes.c_void_p(4096)   # aligned stand-in pointers: xs_moe_plan reads none of them
    t = X.MoeTensors()
    for n in ("x", "router_w", "out", "w13_scale", "w2_scale"):
        setattr(t, n, v)
    if row_major:
        t.w13 = t.w2 = v
    if shared:
        t.shared_w13_scale = t.shared_w2_scale = v
        if row_major:
            t.shared_w13 = t.shared_w2 = v
    if frag:
        t.w13_frag = t.w2_frag = v
        if shared:
            t.shared_w13_frag = t.shared_w2_frag = v
        if fp4:
            t.w13_scale_frag = t.w2_scale_frag = v
    return t


@pytest.mark.parametrize("T,fmt,row_major,frag,want", [
    # row-major FP8 (V4-Flash shape): tiled decode, stream-K from 16 tokens, tall tiles for prefill
    (1, "fp8", True, False, (16, "tiled")),
    (16, "fp8", True, False, (16, "stream")),
    (8192, "fp8", True, False, (192, "tall")),
    # with packed copies: the weight-direct kernels where they apply
    (1, "fp8", True, True, (16, "direct_decode")),
    (16, "fp8", True, True, (16, "direct_decode")),
    (1200, "fp8", True, True, (32, "stream")),
    (1500, "fp8", True, True, (128, "direct_prefill")),   # 9000 rows >= 32 E: tall tiles
    (8192, "fp8", True, True, (128, "direct_prefill")),
    # packed-only: every launch weight-direct, mid-size batches on 128-row tiles
    (16, "fp8", False, True, (16, "direct_decode")),
    (1200, "fp8", False, True, (128, "direct_prefill")),
    (8192, "fp8", False, True, (128, "direct_prefill")),
    # MXFP4
    (2048, "fp4", True, False, (64, "stream")),
    (2048, "fp4", True, True, (64, "direct_mxfp4")),
    (16, "fp4", True, True, (16, "stream")),
    (16, "fp4", False, True, (64, "direct_mxfp4")),
])
def test_kernel_plan_without_gpu(T, fmt, row_major, frag, want, monkeypatch):
    """The forward's dispatch (xs_moe_plan, the same decision the forward
    takes): tile height and kernel family per batch size and weight form."""
    import xs_moe_capi as X
    for n in ("XS_MOE_STREAM", "XS_WIDE_DIRECT", "XS_DECODE_DIRECT", "XS_FP4_DIRECT", "XS_FUSE_COMBINE",
              "XS_MOE_GEMM"):
        monkeypatch.delenv(n, raising=False)
    monkeypatch.setenv("XS_WEIGHT_DIRECT", "1")
    f = X.XS_FP4_E2M1X2 if fmt == "fp4" else X.XS_FP8_E4M3
    p = X.MoeParams(T, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, f, 1, 0)
    got = X.plan(p, _stand_in_tensors(X, row_major, frag, fmt == "fp4"))
    assert (got["tile_rows"], got["routed"]) == want, got
    if fmt == "fp8":
        assert got["shared"] == got["routed"]       # one launch for routed and shared tiles
    else:
        assert got["shared"] == ("direct_prefill" if frag and got["routed"] == "direct_mxfp4" else "tiled")
    assert not got["fused_combine"]


def test_weight_direct_is_opt_in(monkeypatch):
    """Without XS_WEIGHT_DIRECT=1 the packed copies are ignored, and packed-only
    layers and the packed single GEMM are refused."""
    import xs_moe_capi as X
    for n in ("XS_WEIGHT_DIRECT", "XS_MOE_STREAM", "XS_MOE_GEMM", "XS_DECODE_DIRECT"):
        monkeypatch.delenv(n, raising=False)
    p = X.MoeParams(16, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 0)
    assert X.plan(p, _stand_in_tensors(X, True, True))["routed"] == "stream"
    p.T = 8192
    assert X.plan(p, _stand_in_tensors(X, True, True))["routed"] == "tall"
    with pytest.raises(X.XsError, match="weight-direct GEMMs are off"):
        X.plan(p, _stand_in_tensors(X, False, True))
    L = X.lib()
    v = ctypes.c_void_p(4096)
    ws = L.xs_gemm_fp8_blockscale_workspace_size(512, 4096)
    assert L.xs_gemm_fp8_blockscale_packed(v, v, v, 512, 4096, 4096, v, v, ws, None) == 3   # XS_ERR_UNSUPPORTED
    assert b"weight-direct GEMMs are off" in L.xs_last_error()
    monkeypatch.setenv("XS_WEIGHT_DIRECT", "0")
    assert X.plan(p, _stand_in_tensors(X, True, True))["routed"] == "tall"


def test_wide_switch_is_read_per_call(monkeypatch):
    """XS_MOE_GEMM is read on every call: a test that forces a family gets it
    even after an earlier call planned without it."""
    import xs_moe_capi as X
    monkeypatch.delenv("XS_MOE_GEMM", raising=False)
    monkeypatch.setenv("XS_MOE_STREAM", "0")
    p = X.MoeParams(64, 256, 128, 8, 2, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 0)
    assert X.plan(p, _stand_in_tensors(X))["routed"] == "tiled"
    monkeypatch.setenv("XS_MOE_GEMM", "wide")
    assert X.plan(p, _stand_in_tensors(X))["routed"] == "tall"
    monkeypatch.setenv("XS_MOE_GEMM", "tiled")
    p.T = 8192
    assert X.plan(p, _stand_in_tensors(X))["routed"] == "tiled"


def test_kernel_plan_switches_and_refusals(monkeypatch):
    import xs_moe_capi as X
    monkeypatch.setenv("XS_WEIGHT_DIRECT", "1")
    p = X.MoeParams(16, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 0)
    monkeypatch.setenv("XS_DECODE_DIRECT", "0")
    assert X.plan(p, _stand_in_tensors(X, True, True))["routed"] == "stream"
    monkeypatch.setenv("XS_MOE_STREAM", "0")
    assert X.plan(p, _stand_in_tensors(X, True, True))["routed"] == "tiled"
    # the switches do not apply to a packed-only layer: it has no other kernels
    assert X.plan(p, _stand_in_tensors(X, False, True))["routed"] == "direct_decode"
    # no shared expert
    p.has_shared = 0
    assert X.plan(p, _stand_in_tensors(X, True, False, shared=False))["shared"] is None
    # a packed-only layer whose shape the weight-direct kernels do not take
    q = X.MoeParams(16, 256, 256, 8, 2, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 0, 0)
    with pytest.raises(X.XsError, match="no weight-direct GEMM"):
        X.plan(q, _stand_in_tensors(X, False, True, shared=False))


def test_layer_plan_on_host_tensors():
    """MoeLayer.plan passes the layer's own pointers (never dereferenced): it
    runs on CPU tensors too."""
    import torch
    import xs_moe_capi as X
    H, I, E, k = 1024, 512, 32, 4
    u8 = lambda *s: torch.zeros(s, dtype=torch.uint8)  # noqa: E731
    f32 = lambda *s: torch.ones(s, dtype=torch.float32)  # noqa: E731
    layer = X.MoeLayer(torch.zeros((E, H), dtype=torch.bfloat16), u8(E, 2 * I, H), f32(E, 2 * I // 128, H // 128),
                       u8(E, H, I), f32(E, H // 128, I // 128), k,
                       shared=(u8(2 * I, H), f32(2 * I // 128, H // 128), u8(H, I), f32(H // 128, I // 128)))
    assert layer.plan(1)["routed"] == "tiled" and layer.plan(1)["tile_rows"] == 16
    assert layer.plan(4096)["routed"] == "tall" and layer.plan(4096)["shared"] == "tall"


def test_packed_gemm_validation_without_gpu(monkeypatch):
    """xs_gemm_fp8_blockscale_packed refuses shapes and pointers before any
    GPU call: N a multiple of 256, K of 512, aligned operands, a workspace."""
    import xs_moe_capi as X
    monkeypatch.setenv("XS_WEIGHT_DIRECT", "1")
    L = X.lib()
    v = ctypes.c_void_p(4096)
    ws = L.xs_gemm_fp8_blockscale_workspace_size(512, 4096)
    rc = L.xs_gemm_fp8_blockscale_packed(v, v, v, 512, 4096, 4096, v, None, 0, None)
    assert rc != 0 and b"workspace too small" in L.xs_last_error()
    for N, K in ((384, 4096), (4096, 384), (4096, 1152), (128, 512)):
        rc = L.xs_gemm_fp8_blockscale_packed(v, v, v, 512, N, K, v, v, ws, None)
        assert rc == 1 and b"multiple of 256 and K of 512" in L.xs_last_error()
    rc = L.xs_gemm_fp8_blockscale_packed(v, ctypes.c_void_p(4104), v, 512, 4096, 4096, v, v, ws, None)
    assert rc == 1 and b"misaligned" in L.xs_last_error()
    rc = L.xs_gemm_fp8_blockscale_packed(None, v, v, 512, 4096, 4096, v, v, ws, None)
    assert rc == 1 and b"null" in L.xs_last_error()
    # M = 0: nothing to do, nothing launched
    assert L.xs_gemm_fp8_blockscale_packed(v, v, v, 0, 4096, 4096, v, v, ws, None) == 0


def test_router_stats_without_gpu():
    """xs_moe_router_stats validates its params and reports 0, 0 for routers
    other than the certified one without touching a GPU."""
    import xs_moe_capi as X
    L = X.lib()
    out = (ctypes.c_int64 * 2)(7, 7)
    p = X.MoeParams(16, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, X.XS_ROUTER_MFMA)
    assert L.xs_moe_router_stats(ctypes.byref(p), ctypes.c_void_p(4096), out, None) == 0
    assert list(out) == [0, 0]
    p.router_exact = X.XS_ROUTER_CHAIN
    assert L.xs_moe_router_stats(ctypes.byref(p), ctypes.c_void_p(4096), out, None) == 0 and list(out) == [0, 0]
    p.router_exact = 3
    assert L.xs_moe_router_stats(ctypes.byref(p), ctypes.c_void_p(4096), out, None) == 1
    assert b"router_exact must be" in L.xs_last_error()
    assert L.xs_moe_router_stats(ctypes.byref(p), ctypes.c_void_p(4096), None, None) == 1


def test_certified_router_workspace_grows_with_its_lists():
    """The certified router's workspace regions (bound terms per slice, logit
    rows and pair list of the listed tokens, the token list with pair ranges)
    are there only when it is the router."""
    import xs_moe_capi as X
    L = X.lib()
    sizes = {}
    for r in (X.XS_ROUTER_MFMA, X.XS_ROUTER_CERTIFIED, X.XS_ROUTER_CHAIN):
        p = X.MoeParams(16, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, r)
        sizes[r] = L.xs_moe_workspace_size(ctypes.byref(p))
    T, E, nsplit = 16, 256, 16
    extra = 4 * T * E * nsplit + 4 * T * E + 8 * T * E + 3 * 4 * T + 8
    assert sizes[X.XS_ROUTER_CERTIFIED] - sizes[X.XS_ROUTER_MFMA] >= extra
    assert sizes[X.XS_ROUTER_CHAIN] < sizes[X.XS_ROUTER_MFMA]       # one logit slice instead of 16


def test_shared_combine_plan(monkeypatch):
    """XS_SHARED_COMBINE=1 moves the combine into the shared expert's down
    launch on the tall tiles only, and never when the y_rows inspection output
    (which needs the shared rows stored) is asked for."""
    import xs_moe_capi as X
    for n in ("XS_MOE_GEMM", "XS_FUSE_COMBINE", "XS_WEIGHT_DIRECT"):
        monkeypatch.delenv(n, raising=False)
    p = X.MoeParams(8192, 4096, 2048, 256, 6, 1, 1, 1, 1.0, X.XS_BF16, X.XS_FP8_E4M3, 1, 1)
    assert not X.plan(p, _stand_in_tensors(X))["shared_combine"]
    monkeypatch.setenv("XS_SHARED_COMBINE", "1")
    got = X.plan(p, _stand_in_tensors(X))
    assert got["shared_combine"] and not got["fused_combine"] and got["routed"] == "tall"
    t = _stand_in_tensors(X)
    t.y_rows = ctypes.c_void_p(4096)
    assert not X.plan(p, t)["shared_combine"]
    p.T = 16                                   # decode: not the tall tiles
    assert not X.plan(p, _stand_in_tensors(X))["shared_combine"]
    p.T, p.has_shared = 8192, 0                # no shared expert
    assert not X.plan(p, _stand_in_tensors(X, shared=False))["shared_combine"]


def test_router_logits_validation_without_gpu():
    """xs_moe_router_logits refuses bad shapes and misaligned operands before
    any GPU call."""
    import xs_moe_capi as X
    L = X.lib()
    v = ctypes.c_void_p(4096)
    assert L.xs_moe_router_logits(v, v, X.XS_BF16, 4, 8, 200, 1, v, None) == 1
    assert b"H % 128" in L.xs_last_error()
    assert L.xs_moe_router_logits(ctypes.c_void_p(4098), v, X.XS_BF16, 4, 8, 256, 1, v, None) == 1
    assert b"misaligned" in L.xs_last_error()
    assert L.xs_moe_router_logits(v, v, 7, 4, 8, 256, 1, v, None) == 1
    assert b"unsupported dtype" in L.xs_last_error()
