"""Bit-exact byte bridges between torch tensors and xstar_cpp Tensors (the
parity gate of the reference's tests, tests/bridge.py:10-63 there): bf16
travels as uint16, quantized formats as uint8, f32/int32 as themselves."""
import numpy as np
import torch

import xstar_cpp

_NP_VIEW = {torch.float32: (None, xstar_cpp.DType.Float32), torch.bfloat16: (torch.uint16, xstar_cpp.DType.BFloat16),
            torch.int32: (None, xstar_cpp.DType.Int32)}


def torch_to_cpp(t: torch.Tensor, dtype=None) -> "xstar_cpp.Tensor":
    """Host copy of t's bytes as an xstar Tensor.  dtype overrides the element
    type for raw uint8 tensors (Float8E4M3, Float4E2M1x2, Float8E8M0)."""
    t = t.detach().cpu().contiguous()
    if dtype is not None:
        return xstar_cpp.from_numpy_raw(t.view(torch.uint8).numpy(), list(t.shape), dtype)
    view, d = _NP_VIEW[t.dtype]
    a = t.view(view).numpy() if view is not None else t.numpy()
    return xstar_cpp.from_numpy_raw(a, list(t.shape), d)


def cpp_to_torch(t, ref_shape) -> torch.Tensor:
    """Inverse of torch_to_cpp for Float32 / BFloat16 / Int32 / byte types."""
    raw = xstar_cpp.to_numpy_raw(t)
    d = t.dtype()
    if d == xstar_cpp.DType.Float32:
        return torch.from_numpy(raw.view(np.float32).reshape(ref_shape).copy())
    if d == xstar_cpp.DType.BFloat16:
        return torch.from_numpy(raw.view(np.uint16).reshape(ref_shape).copy()).view(torch.bfloat16)
    if d == xstar_cpp.DType.Int32:
        return torch.from_numpy(raw.view(np.int32).reshape(ref_shape).copy())
    return torch.from_numpy(raw.reshape(ref_shape).copy())
