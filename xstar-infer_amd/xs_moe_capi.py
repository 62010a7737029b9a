"""ctypes binding of the C ABI in include/xs_moe.h (libxs_moe.so).

This is the binding a Python caller adds to use the library without the
pybind11 module; the tests and bench.py call the kernels through it.  Device
buffers are torch CUDA tensors (device memory and streams only); every compute
call goes to the HIP library.  Importing fails loudly when libxs_moe.so has not
been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "xstar_cpp_py", "libxs_moe.so")

XS_F32, XS_BF16, XS_FP8_E4M3, XS_FP4_E2M1X2, XS_E8M0, XS_I32 = range(6)
XS_ROUTER_MFMA, XS_ROUTER_CERTIFIED, XS_ROUTER_CHAIN = range(3)

P = C.c_void_p
I64 = C.c_int64


class MoeParams(C.Structure):
    _fields_ = [("T", I64), ("H", I64), ("I", I64), ("E", I64), ("top_k", I64),
                ("n_group", I64), ("topk_group", I64), ("renormalize", C.c_int),
                ("routed_scaling", C.c_float), ("x_dtype", C.c_int), ("routed_format", C.c_int),
                ("has_shared", C.c_int), ("router_exact", C.c_int),
                ("has_norm", C.c_int), ("norm_eps", C.c_float)]


class MoeTensors(C.Structure):
    _fields_ = [(n, P) for n in (
        "x", "router_w", "router_bias", "w13", "w13_scale", "w2", "w2_scale",
        "shared_w13", "shared_w13_scale", "shared_w2", "shared_w2_scale", "out",
        "logits", "topk_idx", "topk_w", "counts", "offsets", "perm", "inv", "norm_weight", "residual",
        "act_q", "act_s", "y_rows", "w13_frag", "w2_frag", "shared_w13_frag", "shared_w2_frag",
        "w13_scale_frag", "w2_scale_frag")]


class MoePlan(C.Structure):
    _fields_ = [("tile_rows", C.c_int), ("routed_gemm", C.c_int), ("shared_gemm", C.c_int),
                ("fused_combine", C.c_int)]


GEMM_KINDS = ("tiled", "stream", "tall", "direct_prefill", "direct_decode", "direct_mxfp4")


EXPORTS = {
    "xs_last_error": (C.c_char_p, []),
    "xs_device_count": (C.c_int, [P]),
    "xs_malloc": (C.c_int, [P, C.c_size_t]),
    "xs_free": (C.c_int, [P]),
    "xs_memcpy_h2d": (C.c_int, [P, P, C.c_size_t]),
    "xs_memcpy_d2h": (C.c_int, [P, P, C.c_size_t]),
    "xs_memcpy_d2d": (C.c_int, [P, P, C.c_size_t]),
    "xs_free_bytes": (C.c_int, [P]),
    "xs_stream_synchronize": (C.c_int, [P]),
    "xs_moe_router_logits": (C.c_int, [P, P, C.c_int, I64, I64, I64, C.c_int, P, P]),
    "xs_moe_route": (C.c_int, [P, P, I64, I64, I64, I64, I64, C.c_int, C.c_float, P, P, P]),
    "xs_moe_permute_workspace_size": (C.c_size_t, [I64, I64]),
    "xs_moe_permute": (C.c_int, [P, I64, I64, I64, P, P, P, P, P, C.c_size_t, P]),
    "xs_quant_act_fp8": (C.c_int, [P, C.c_int, I64, I64, P, P, P]),
    "xs_quant_act_mxfp8": (C.c_int, [P, C.c_int, I64, I64, P, P, P]),
    "xs_rmsnorm": (C.c_int, [P, P, C.c_int, I64, I64, C.c_float, P, P, P, P]),
    "xs_quant_weight_fp8_block": (C.c_int, [P, C.c_int, I64, I64, I64, P, P, P]),
    "xs_quant_weight_mxfp4": (C.c_int, [P, C.c_int, I64, I64, I64, P, P, P]),
    "xs_pack_weight_fp8_frag": (C.c_int, [P, I64, I64, I64, P, P]),
    "xs_pack_weight_mxfp4_frag": (C.c_int, [P, P, I64, I64, I64, P, P, P]),
    "xs_gemm_fp8_blockscale_workspace_size": (C.c_size_t, [I64, I64]),
    "xs_gemm_fp8_blockscale": (C.c_int, [P, P, P, I64, I64, I64, P, P, C.c_size_t, P]),
    "xs_gemm_fp8_blockscale_packed": (C.c_int, [P, P, P, I64, I64, I64, P, P, C.c_size_t, P]),
    "xs_moe_workspace_size": (C.c_size_t, [P]),
    "xs_moe_plan": (C.c_int, [P, P, P]),
    "xs_moe_router_stats": (C.c_int, [P, P, P, P]),
    "xs_moe_forward": (C.c_int, [P, P, P, C.c_size_t, P]),
    "xs_moe_noalloc_scratch_bytes": (C.c_size_t, []),
    "xs_moe_forward_noalloc": (C.c_int, [P, P, P]),
    "xs_moe_profile_enable": (C.c_int, [C.c_int]),
    "xs_moe_profile_read": (C.c_int, [P, C.c_int, P]),
}

STAGES = ("act_quant", "router_logits", "route", "permute", "gemm_gate_up", "gemm_down", "combine")


def profile_enable(on=True):
    check(lib().xs_moe_profile_enable(int(on)))


def profile_read():
    """-> (dict stage -> summed ms, number of forwards) since the last read."""
    ms = (C.c_float * len(STAGES))()
    n = C.c_int(0)
    check(lib().xs_moe_profile_read(ms, len(STAGES), C.byref(n)))
    return {s: float(ms[i]) for i, s in enumerate(STAGES)}, n.value

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python xstar-infer_amd/build.py`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class XsError(RuntimeError):
    pass


def check(rc: int) -> None:
    if rc != 0:
        raise XsError(f"xs_moe error {rc}: {lib().xs_last_error().decode()}")


# ---------------------------------------------------------------- torch glue
def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_code(t):
    import torch
    if t.dtype == torch.bfloat16:
        return XS_BF16
    if t.dtype == torch.float32:
        return XS_F32
    raise XsError("unsupported dtype")


def _u8(t):
    """Raw-byte view of a quantized tensor (uint8 or torch float8 / float4 dtypes)."""
    import torch
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def router_logits(x, router_w, exact=False):
    import torch
    T, H = x.shape
    E = router_w.shape[0]
    out = torch.empty((T, E), dtype=torch.float32, device=x.device)
    check(lib().xs_moe_router_logits(_ptr(x), _ptr(router_w), _dtype_code(x), T, E, H, int(exact),
                                     _ptr(out), _stream()))
    return out


def route(logits, bias, k, n_group=1, topk_group=1, renormalize=True, scaling=1.0):
    import torch
    T, E = logits.shape
    idx = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    check(lib().xs_moe_route(_ptr(logits), _ptr(bias), T, E, k, n_group, topk_group,
                             int(renormalize), float(scaling), _ptr(idx), _ptr(w), _stream()))
    return idx, w


def permute(idx, E):
    import torch
    T, k = idx.shape
    dev = idx.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    nb = lib().xs_moe_permute_workspace_size(T, E)
    ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
    check(lib().xs_moe_permute(_ptr(idx), T, E, k, _ptr(counts), _ptr(offsets), _ptr(perm), _ptr(inv),
                               _ptr(ws), ws.numel(), _stream()))
    return counts, offsets, perm, inv


def quant_act_fp8(x):
    import torch
    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, cols // 128), dtype=torch.float32, device=x.device)
    check(lib().xs_quant_act_fp8(_ptr(x), _dtype_code(x), rows, cols, _ptr(q), _ptr(s), _stream()))
    return q, s


def quant_act_mxfp8(x):
    import torch
    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, cols // 32), dtype=torch.uint8, device=x.device)
    check(lib().xs_quant_act_mxfp8(_ptr(x), _dtype_code(x), rows, cols, _ptr(q), _ptr(s), _stream()))
    return q, s


def rmsnorm(x, weight, eps, quant=False):
    """RMSNorm over the last axis -> y (dtype of x); quant=True also returns the
    FP8 1x128 quantization of y as (y, q uint8, s f32 [rows, H/128])."""
    import torch
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    y = torch.empty_like(x)
    q = s = None
    if quant:
        q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        s = torch.empty((*x.shape[:-1], hidden // 128), dtype=torch.float32, device=x.device)
    check(lib().xs_rmsnorm(_ptr(x), _ptr(weight), _dtype_code(x), rows, hidden, float(eps), _ptr(y),
                           _ptr(q), _ptr(s), _stream()))
    return (y, q, s) if quant else y


def quant_weight_fp8_block(w):
    """w [..., n, k] (bf16/f32, CUDA) -> (q uint8 [..., n, k], s f32 [..., n/128, k/128])."""
    import torch
    *lead, n, k = w.shape
    b = 1
    for d in lead:
        b *= d
    q = torch.empty(w.shape, dtype=torch.uint8, device=w.device)
    s = torch.empty((*lead, n // 128, k // 128), dtype=torch.float32, device=w.device)
    check(lib().xs_quant_weight_fp8_block(_ptr(w), _dtype_code(w), b, n, k, _ptr(q), _ptr(s), _stream()))
    return q, s


def quant_weight_mxfp4(w):
    import torch
    *lead, n, k = w.shape
    b = 1
    for d in lead:
        b *= d
    q = torch.empty((*lead, n, k // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty((*lead, n, k // 32), dtype=torch.uint8, device=w.device)
    check(lib().xs_quant_weight_mxfp4(_ptr(w), _dtype_code(w), b, n, k, _ptr(q), _ptr(s), _stream()))
    return q, s


def gemm_fp8_blockscale(a, bq, bs, out=None, workspace=None):
    import torch
    M, K = a.shape
    N = bq.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    nb = lib().xs_gemm_fp8_blockscale_workspace_size(M, K)
    if workspace is None:
        workspace = torch.empty(nb, dtype=torch.uint8, device=a.device)
    check(lib().xs_gemm_fp8_blockscale(_ptr(a), _ptr(_u8(bq)), _ptr(bs), M, N, K, _ptr(out),
                                       _ptr(workspace), workspace.numel(), _stream()))
    return out


def gemm_fp8_blockscale_packed(a, bp, bs, out=None, workspace=None):
    """xs_gemm_fp8_blockscale_packed: bp is pack_weight_fp8_frag(B) of B [N, K]."""
    import torch
    M, K = a.shape
    N = bp.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    nb = lib().xs_gemm_fp8_blockscale_workspace_size(M, K)
    if workspace is None:
        workspace = torch.empty(nb, dtype=torch.uint8, device=a.device)
    check(lib().xs_gemm_fp8_blockscale_packed(_ptr(a), _ptr(_u8(bp)), _ptr(bs), M, N, K, _ptr(out),
                                              _ptr(workspace), workspace.numel(), _stream()))
    return out


def pack_weight_fp8_frag(w):
    """[..., n, k] e4m3 (uint8 or float8 view) -> a tensor of the same shape and
    bytes in MFMA fragment order (xs_pack_weight_fp8_frag)."""
    import torch
    w = _u8(w).contiguous()
    n, k = w.shape[-2], w.shape[-1]
    batch = w.numel() // (n * k)
    out = torch.empty_like(w)
    check(lib().xs_pack_weight_fp8_frag(_ptr(w), batch, n, k, _ptr(out), _stream()))
    return out


def pack_weight_mxfp4_frag(w, s):
    """MXFP4 [..., n, k/2] weights and [..., n, k/32] e8m0 scales -> tensors of
    the same shapes and bytes in MFMA fragment order (xs_pack_weight_mxfp4_frag)."""
    import torch
    w, s = _u8(w).contiguous(), _u8(s).contiguous()
    n, k = w.shape[-2], w.shape[-1] * 2
    batch = w.numel() // (n * k // 2)
    ow, os_ = torch.empty_like(w), torch.empty_like(s)
    check(lib().xs_pack_weight_mxfp4_frag(_ptr(w), _ptr(s), batch, n, k, _ptr(ow), _ptr(os_), _stream()))
    return ow, os_


def plan(params, tensors):
    """xs_moe_plan: the kernels xs_moe_forward would launch for these params and
    tensors (nothing runs; no GPU needed) as a dict: tile_rows, routed, shared
    (names from GEMM_KINDS; shared None without a shared expert), fused_combine
    (the down GEMM sums each token's rows), shared_combine (the shared expert's
    down launch does)."""
    out = MoePlan()
    check(lib().xs_moe_plan(C.byref(params), C.byref(tensors), C.byref(out)))
    kind = lambda k: None if k < 0 else GEMM_KINDS[k]  # noqa: E731
    return {"tile_rows": out.tile_rows, "routed": kind(out.routed_gemm), "shared": kind(out.shared_gemm),
            "fused_combine": out.fused_combine == 1, "shared_combine": out.fused_combine == 2}


class MoeLayer:
    """Holds weights (device tensors) and calls xs_moe_forward.  frag=True also
    keeps fragment-packed copies of the weights (routed and shared; MXFP4
    layers: routed weights with their scales, and the FP8 shared expert), which
    the GEMMs load straight into registers (same results).  frag="only" keeps
    the packed copies alone (the row-major expert weights are dropped, so the
    layer takes no more memory than before), and every GEMM is a weight-direct
    one.  The weight-direct GEMMs are opt-in (XS_WEIGHT_DIRECT=1 in the
    environment): without it the packed copies go unused, and a frag="only"
    layer's forward raises XsError (unsupported)."""

    def __init__(self, router_w, w13, w13_scale, w2, w2_scale, top_k, router_bias=None,
                 shared=None, routed_format=XS_FP8_E4M3, n_group=1, topk_group=1,
                 renormalize=True, routed_scaling=1.0, router_exact=None, norm_weight=None,
                 norm_eps=1e-6, frag=False, router=None):
        self.router_w, self.router_bias = router_w, router_bias
        self.norm_weight, self.norm_eps = norm_weight, norm_eps
        self.w13, self.w13_scale, self.w2, self.w2_scale = _u8(w13), w13_scale, _u8(w2), w2_scale
        self.shared = None if shared is None else (_u8(shared[0]), shared[1], _u8(shared[2]), shared[3])
        self.top_k, self.routed_format = top_k, routed_format
        self.n_group, self.topk_group = n_group, topk_group
        # router: XS_ROUTER_MFMA / _CERTIFIED / _CHAIN (default certified: the
        # reference's top-k bit for bit).  router_exact=True / False, the older
        # switch, picks the chain router (gemm_cpu logits) / the MFMA router.
        if router is None:
            router = XS_ROUTER_CERTIFIED if router_exact is None else (
                XS_ROUTER_CHAIN if router_exact else XS_ROUTER_MFMA)
        self.renormalize, self.routed_scaling, self.router_exact = renormalize, routed_scaling, int(router)
        self.E, self.H = router_w.shape
        self.I = w2.shape[-1] * (2 if routed_format == XS_FP4_E2M1X2 else 1)
        self._ws = None
        # w13_frag, w2_frag, shared_w13_frag, shared_w2_frag, w13_scale_frag, w2_scale_frag
        self.frag = (None,) * 6
        if frag and routed_format == XS_FP8_E4M3:
            f = [pack_weight_fp8_frag(self.w13), pack_weight_fp8_frag(self.w2), None, None, None, None]
            if self.shared is not None:
                f[2], f[3] = pack_weight_fp8_frag(self.shared[0]), pack_weight_fp8_frag(self.shared[2])
            self.frag = tuple(f)
        elif frag:
            w13p, s13p = pack_weight_mxfp4_frag(self.w13, self.w13_scale)
            w2p, s2p = pack_weight_mxfp4_frag(self.w2, self.w2_scale)
            sh13p = sh2p = None   # the FP8 shared expert
            if self.shared is not None:
                sh13p, sh2p = pack_weight_fp8_frag(self.shared[0]), pack_weight_fp8_frag(self.shared[2])
            self.frag = (w13p, w2p, sh13p, sh2p, s13p, s2p)
        if frag == "only":
            self.w13 = self.w2 = None
            if self.shared is not None:
                self.shared = (None, self.shared[1], None, self.shared[3])

    def params(self, T, x_dtype):
        return MoeParams(T, self.H, self.I, self.E, self.top_k, self.n_group, self.topk_group,
                         int(self.renormalize), float(self.routed_scaling), x_dtype,
                         self.routed_format, int(self.shared is not None), int(self.router_exact),
                         int(self.norm_weight is not None), float(self.norm_eps))

    def workspace(self, T, x_dtype, device):
        import torch
        p = self.params(T, x_dtype)
        nb = lib().xs_moe_workspace_size(C.byref(p))
        if nb == 0:
            check(1)
        if self._ws is None or self._ws.numel() < nb:
            self._ws = torch.empty(nb, dtype=torch.uint8, device=device)
        return self._ws

    def forward(self, x, out=None, debug=None, residual=None):
        """debug: optional dict of preallocated device tensors with keys among
        logits, topk_idx, topk_w, counts, offsets, perm, inv, act_q, act_s, y_rows
        (shapes in include/xs_moe.h).  residual: optional
        [T, H] tensor (dtype of x) added to the output before its rounding; it
        may be `out` itself."""
        import torch
        T = x.shape[0]
        xd = _dtype_code(x)
        if out is None:
            out = torch.empty((T, self.H), dtype=x.dtype, device=x.device)
        ws = self.workspace(T, xd, x.device)
        p = self.params(T, xd)
        sh = self.shared or (None, None, None, None)
        d = debug or {}
        t = MoeTensors(_ptr(x), _ptr(self.router_w), _ptr(self.router_bias), _ptr(self.w13),
                       _ptr(self.w13_scale), _ptr(self.w2), _ptr(self.w2_scale), _ptr(sh[0]),
                       _ptr(sh[1]), _ptr(sh[2]), _ptr(sh[3]), _ptr(out),
                       *[_ptr(d.get(n)) for n in ("logits", "topk_idx", "topk_w", "counts",
                                                 "offsets", "perm", "inv")],
                       _ptr(self.norm_weight), _ptr(residual),
                       *[_ptr(d.get(n)) for n in ("act_q", "act_s", "y_rows")],
                       *[_ptr(f) for f in self.frag])
        check(lib().xs_moe_forward(C.byref(p), C.byref(t), _ptr(ws), ws.numel(), _stream()))
        return out

    def router_stats(self, T, x_dtype=XS_BF16):
        """After forward() on T tokens: (logits the certified router's exact
        pass recomputed, tokens routed after it); (0, 0) for other routers.
        Waits for the stream."""
        out = (C.c_int64 * 2)()
        p = self.params(T, x_dtype)
        check(lib().xs_moe_router_stats(C.byref(p), _ptr(self._ws), out, _stream()))
        return int(out[0]), int(out[1])

    def plan(self, T, x_dtype=XS_BF16):
        """The kernels forward() would launch for T tokens (see plan())."""
        sh = self.shared or (None, None, None, None)
        stand_in = C.c_void_p(256)   # x and out: checked for presence and alignment, never read
        t = MoeTensors(stand_in, _ptr(self.router_w), _ptr(self.router_bias), _ptr(self.w13),
                       _ptr(self.w13_scale), _ptr(self.w2), _ptr(self.w2_scale), _ptr(sh[0]),
                       _ptr(sh[1]), _ptr(sh[2]), _ptr(sh[3]), stand_in, *([None] * 7),
                       _ptr(self.norm_weight), None, None, None, None, *[_ptr(f) for f in self.frag])
        return plan(self.params(T, x_dtype), t)

    def forward_noalloc(self, x, out):
        """The same forward through xs_moe_forward_noalloc: the library's static
        scratch instead of a workspace; `out` is preallocated by the caller."""
        T = x.shape[0]
        p = self.params(T, _dtype_code(x))
        sh = self.shared or (None, None, None, None)
        t = MoeTensors(_ptr(x), _ptr(self.router_w), _ptr(self.router_bias), _ptr(self.w13),
                       _ptr(self.w13_scale), _ptr(self.w2), _ptr(self.w2_scale), _ptr(sh[0]),
                       _ptr(sh[1]), _ptr(sh[2]), _ptr(sh[3]), _ptr(out), *([None] * 7),
                       _ptr(self.norm_weight), None, None, None, None, *[_ptr(f) for f in self.frag])
        check(lib().xs_moe_forward_noalloc(C.byref(p), C.byref(t), _stream()))
        return out
