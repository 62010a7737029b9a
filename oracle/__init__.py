"""CPU oracle for the MoE operator -- TEST INFRASTRUCTURE ONLY.

ctypes wrapper around oracle/_build/liboracle.so (moe_oracle.c).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or as the timed CPU baseline.  The product
(the HIP library, the C++ Tensor ops and the pybind11 module) never loads it.

Reference anchors are given per function in moe_oracle.h / moe_oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libxsref.so")
_lib = None
_ref = None

P = C.c_void_p
I64 = C.c_int64


def build(ref: bool = True) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    targets = ["all"]
    if ref and os.path.isdir("/root/reference/xstar_cpp"):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", _HERE] + targets, check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build(ref=False)
        _lib = C.CDLL(_LIB_PATH)
        L = _lib
        L.xo_bf16_from_f32.restype = C.c_uint16
        L.xo_bf16_from_f32.argtypes = [C.c_float]
        L.xo_e4m3_decode.restype = C.c_float
        L.xo_e4m3_decode.argtypes = [C.c_uint8]
        L.xo_e4m3_encode.restype = C.c_uint8
        L.xo_e4m3_encode.argtypes = [C.c_float]
        L.xo_e2m1_decode.restype = C.c_float
        L.xo_e2m1_decode.argtypes = [C.c_uint8]
        L.xo_e2m1_encode.restype = C.c_uint8
        L.xo_e2m1_encode.argtypes = [C.c_float]
        L.xo_e8m0_decode.restype = C.c_float
        L.xo_e8m0_decode.argtypes = [C.c_uint8]
        for f in ("xo_expf", "xo_sigmoid", "xo_silu"):
            getattr(L, f).restype = C.c_float
            getattr(L, f).argtypes = [C.c_float]
        L.xo_quant_act_fp8.argtypes = [P, I64, I64, P, P]
        L.xo_quant_act_mxfp8.argtypes = [P, I64, I64, P, P]
        L.xo_quant_weight_fp8_block.argtypes = [P, I64, I64, P, P]
        L.xo_quant_weight_mxfp4.argtypes = [P, I64, I64, P, P]
        L.xo_router_logits.argtypes = [P, P, C.c_int, I64, I64, I64, P]
        L.xo_rmsnorm.argtypes = [P, P, C.c_int, I64, I64, C.c_float, P]
        L.xo_route.argtypes = [P, P, I64, I64, I64, I64, I64, C.c_int, C.c_float, P, P]
        L.xo_permute.argtypes = [P, I64, I64, I64, P, P, P, P]
        L.xo_moe_forward.argtypes = [P, P, P]
        L.xo_moe_forward.restype = C.c_int
        L.xo_moe_ref_f32.argtypes = [P] * 7 + [I64] * 5 + [C.c_int, C.c_float, I64, I64, P]
    return _lib


def ref_lib():
    """The reference's own CPU numerics (oracle/_ref), or None if not built."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        _ref = C.CDLL(_REF_PATH)
        _ref.xsref_gemm_f32.argtypes = [P, P, P, I64, I64, I64, C.c_int]
        _ref.xsref_gemm_bf16.argtypes = [P, P, P, I64, I64, I64, C.c_int]
        _ref.xsref_bf16_from_f32.argtypes = [P, P, I64]
        _ref.xsref_sigmoid.argtypes = [P, P, I64]
        _ref.xsref_silu.argtypes = [P, P, I64]
    return _ref


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- vectorised helpers
def e4m3_encode(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([L.xo_e4m3_encode(float(v)) for v in flat], dtype=np.uint8).reshape(np.shape(x))


def e4m3_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e4m3_decode(i) for i in range(256)], dtype=np.float32)


def e2m1_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e2m1_decode(i) for i in range(16)], dtype=np.float32)


def e8m0_table() -> np.ndarray:
    L = lib()
    return np.array([L.xo_e8m0_decode(i) for i in range(256)], dtype=np.float32)


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    # same arithmetic as xo_bf16_from_f32 (vectorised); tests pin one against the other
    return (u >> 16).astype(np.uint16)


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quant_act_fp8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // 128), np.float32)
    lib().xo_quant_act_fp8(_p(x), rows, cols, _p(q), _p(s))
    return q, s


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, bf16: bool = False) -> np.ndarray:
    """RMSNorm over the last axis (xo_rmsnorm; rmsnorm.cpp:27-73).  bf16=True:
    x and w are bf16 bit patterns (uint16) and so is the result; else f32."""
    dt = np.uint16 if bf16 else np.float32
    x = np.ascontiguousarray(x, dtype=dt)
    w = np.ascontiguousarray(w, dtype=dt)
    hidden = x.shape[-1]
    assert w.shape == (hidden,)
    rows = x.size // hidden if hidden else 0
    y = np.empty_like(x)
    if rows:
        lib().xo_rmsnorm(_p(x), _p(w), int(bf16), rows, hidden, float(eps), _p(y))
    return y


def quant_act_mxfp8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // 32), np.uint8)
    lib().xo_quant_act_mxfp8(_p(x), rows, cols, _p(q), _p(s))
    return q, s


def quant_weight_fp8_block(w: np.ndarray):
    """w [..., n, k] f32 -> (q [..., n, k] u8, s [..., n/128, k/128] f32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    q = np.empty(w.shape, np.uint8)
    s = np.empty((*lead, n // 128, k // 128), np.float32)
    nb = int(np.prod(lead)) if lead else 1
    wv, qv, sv = w.reshape(nb, n, k), q.reshape(nb, n, k), s.reshape(nb, n // 128, k // 128)
    for i in range(nb):
        lib().xo_quant_weight_fp8_block(_p(wv[i]), n, k, _p(qv[i]), _p(sv[i]))
    return q, s


def quant_weight_mxfp4(w: np.ndarray):
    """w [..., n, k] f32 -> (q [..., n, k/2] u8 packed, s [..., n, k/32] e8m0)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    q = np.empty((*lead, n, k // 2), np.uint8)
    s = np.empty((*lead, n, k // 32), np.uint8)
    nb = int(np.prod(lead)) if lead else 1
    wv, qv, sv = w.reshape(nb, n, k), q.reshape(nb, n, k // 2), s.reshape(nb, n, k // 32)
    for i in range(nb):
        lib().xo_quant_weight_mxfp4(_p(wv[i]), n, k, _p(qv[i]), _p(sv[i]))
    return q, s


def dequant_weight_fp8_block(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    tab = e4m3_table()
    v = tab[q]
    rep = np.repeat(np.repeat(s, 128, axis=-2), 128, axis=-1)
    return (v * rep).astype(np.float32)


def dequant_weight_mxfp4(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    tab = e2m1_table()
    lo = tab[q & 15]
    hi = tab[q >> 4]
    v = np.stack([lo, hi], axis=-1).reshape(*q.shape[:-1], q.shape[-1] * 2)
    return (v * np.repeat(e8m0_table()[s], 32, axis=-1)).astype(np.float32)


def router_logits(x: np.ndarray, wr: np.ndarray, is_bf16: bool) -> np.ndarray:
    T, H = x.shape
    E = wr.shape[0]
    out = np.empty((T, E), np.float32)
    x = np.ascontiguousarray(x)
    wr = np.ascontiguousarray(wr)
    lib().xo_router_logits(_p(x), _p(wr), int(is_bf16), T, E, H, _p(out))
    return out


def route(logits, bias, k, n_group=1, topk_group=1, renormalize=True, scaling=1.0):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_route(_p(logits), None if b is None else _p(b), T, E, k, n_group, topk_group,
                   int(renormalize), float(scaling), _p(idx), _p(w))
    return idx, w


def permute(idx: np.ndarray, E: int):
    idx = np.ascontiguousarray(idx, np.int32)
    T, k = idx.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    inv = np.empty(T * k, np.int32)
    lib().xo_permute(_p(idx), T, E, k, _p(counts), _p(offsets), _p(perm), _p(inv))
    return counts, offsets, perm, inv


class _Cfg(C.Structure):
    _fields_ = [("T", I64), ("H", I64), ("I", I64), ("E", I64), ("k", I64),
                ("n_group", I64), ("topk_group", I64), ("renormalize", C.c_int),
                ("scaling", C.c_float), ("x_is_bf16", C.c_int), ("routed_fp4", C.c_int),
                ("has_shared", C.c_int), ("nthreads", C.c_int)]


class _In(C.Structure):
    _fields_ = [(n, P) for n in ("x", "router_w", "router_bias", "logits_in", "w13", "s13",
                                 "w2", "s2", "sw13", "ss13", "sw2", "ss2")]


class _Out(C.Structure):
    _fields_ = [(n, P) for n in ("logits", "idx", "w", "counts", "offsets", "perm", "inv",
                                 "out_f32", "out")]


def moe_forward(x, router_w, router_bias, w13, s13, w2, s2, k, shared=None, routed_fp4=False,
                n_group=1, topk_group=1, renormalize=True, scaling=1.0, logits_in=None,
                nthreads=None):
    """Quantized-path oracle.  x/router_w: np.uint16 (bf16 bits) or np.float32.
    shared: (sw13, ss13, sw2, ss2) FP8 tuple or None.  Returns a dict of numpy arrays."""
    is_bf16 = x.dtype == np.uint16
    T, H = x.shape
    E = router_w.shape[0]
    I = w2.shape[-1] * (2 if routed_fp4 else 1)
    cfg = _Cfg(T, H, I, E, k, n_group, topk_group, int(renormalize), float(scaling),
               int(is_bf16), int(routed_fp4), int(shared is not None),
               int(nthreads or min(8, os.cpu_count() or 1)))
    keep = []

    def ptr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    sh = shared or (None, None, None, None)
    inp = _In(ptr(x), ptr(router_w), ptr(router_bias), ptr(logits_in), ptr(w13), ptr(s13),
              ptr(w2), ptr(s2), ptr(sh[0]), ptr(sh[1]), ptr(sh[2]), ptr(sh[3]))
    res = dict(logits=np.empty((T, E), np.float32), idx=np.empty((T, k), np.int32),
               w=np.empty((T, k), np.float32), counts=np.empty(E, np.int32),
               offsets=np.empty(E + 1, np.int32), perm=np.empty(T * k, np.int32),
               inv=np.empty(T * k, np.int32), out_f32=np.empty((T, H), np.float32),
               out=np.empty((T, H), np.uint16 if is_bf16 else np.float32))
    o = _Out(*[res[n].ctypes.data for n in ("logits", "idx", "w", "counts", "offsets", "perm",
                                            "inv", "out_f32", "out")])
    rc = lib().xo_moe_forward(C.byref(cfg), C.byref(inp), C.byref(o))
    if rc != 0:
        raise RuntimeError(f"oracle moe_forward failed ({rc})")
    return res


def moe_ref_f32(x, router_w, router_bias, w13, w2, k, shared=None, renormalize=True,
                scaling=1.0, t0=0, t1=None):
    """Reference-path f32 MoE (the reference's CPU ops composed; single-threaded).
    w13 / w2: arrays [E, ...] or dicts {expert: array} holding only the experts
    the tokens route to."""
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    E = router_w.shape[0]
    t1 = T if t1 is None else t1
    out = np.empty((t1 - t0, H), np.float32)
    keep = []

    def ptr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, np.float32)
        keep.append(a)
        return a.ctypes.data

    def table(w):
        tab = (C.c_void_p * E)()
        for e in range(E):
            a = w.get(e) if isinstance(w, dict) else w[e]
            tab[e] = ptr(a)
        return tab

    any_w2 = next(iter(w2.values())) if isinstance(w2, dict) else w2[0]
    I = any_w2.shape[-1]
    t13, t2 = table(w13), table(w2)
    sw13, sw2 = shared if shared is not None else (None, None)
    lib().xo_moe_ref_f32(ptr(x), ptr(router_w), ptr(router_bias), t13, t2, ptr(sw13),
                         ptr(sw2), T, H, I, E, k, int(renormalize), float(scaling), t0, t1,
                         out.ctypes.data)
    return out
