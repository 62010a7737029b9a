"""safetensors reading (MMapFile, parse_safetensors_header, make_weight_view)
and the MoE layer loader (load_moe_layer), on the CPU.

The parser's error branches follow the reference's own tests
(tests/infra/test_cpp_parse_safetensors_header.py:211-270: file too small,
truncated header, unsupported dtype, __metadata__ skipped, inconsistent
header).  Files written by the safetensors library itself (including
F8_E4M3 / F8_E8M0 / U8 / I32) are read back bit for bit.  The loader's stacking
is checked against torch.cat of the per-expert tensors."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import xstar_cpp
from bridge import cpp_to_torch

D = xstar_cpp.DType


def _raw_file(path, tensors, metadata=None, trailing_comma=False):
    """[u64 header length][JSON][data], built by hand for malformed cases."""
    header, data, off = {}, b"", 0
    for name, (dt, shape, blob) in tensors.items():
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(blob)]}
        data += blob
        off += len(blob)
    if metadata is not None:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    if trailing_comma:
        hb = hb[:-1] + b",}"
    hb += b" " * ((-len(hb)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + data)
    return str(path)


def _view_bytes(mf, meta):
    t = xstar_cpp.make_weight_view(mf, meta.offset, list(meta.shape), meta.dtype)
    return xstar_cpp.to_numpy_raw(t)


# ------------------------------------------------------------ error branches
def test_rejects_file_too_small(tmp_path):
    p = tmp_path / "a"
    p.write_bytes(b"\x01\x02")
    with pytest.raises(RuntimeError, match="file smaller than 8 bytes"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(str(p)))


def test_rejects_truncated_header(tmp_path):
    p = tmp_path / "a"
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(RuntimeError, match="truncated header"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(str(p)))


def test_rejects_unsupported_dtype(tmp_path):
    p = _raw_file(tmp_path / "a", {"y": ("F16", [1], b"\x00\x00")})
    with pytest.raises(RuntimeError, match="dtype not"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(p))


def test_skips_metadata_and_tolerates_trailing_comma(tmp_path):
    p = _raw_file(tmp_path / "a", {"x": ("F32", [1], np.array([1.0], np.float32).tobytes())},
                  metadata={"format": "pt", "nested": {"a": [1, 2, {"b": "c"}]}}, trailing_comma=True)
    meta = xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(p))
    assert "__metadata__" not in meta and list(meta["x"].shape) == [1]


def test_rejects_inconsistent_header(tmp_path):
    p = _raw_file(tmp_path / "a", {"z": ("F32", [2], b"\x00\x00")})
    with pytest.raises(RuntimeError, match="header inconsistent"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(p))


def test_rejects_tensor_past_end_of_file(tmp_path):
    p = _raw_file(tmp_path / "a", {"z": ("F32", [2], b"\x00" * 8)})
    with open(p, "r+b") as f:
        f.truncate(f.seek(0, 2) - 4)
    with pytest.raises(RuntimeError, match="ends past the file"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(p))


def test_rejects_escapes_and_view_bounds(tmp_path):
    p = tmp_path / "a"
    hb = b'{"a\\\\b": {"dtype": "F32", "shape": [0], "data_offsets": [0, 0]}}'
    hb += b" " * ((-len(hb)) % 8)
    p.write_bytes(struct.pack("<Q", len(hb)) + hb)
    with pytest.raises(RuntimeError, match="backslash"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(str(p)))
    q = _raw_file(tmp_path / "b", {"x": ("F32", [2], b"\x00" * 8)})
    mf = xstar_cpp.MMapFile(q)
    with pytest.raises(RuntimeError, match="exceeds mmap region"):
        xstar_cpp.make_weight_view(mf, mf.size() - 4, [2], D.Float32)
    with pytest.raises(RuntimeError, match="not aligned"):
        xstar_cpp.make_weight_view(mf, 2, [1], D.Float32)


# ------------------------------------------------ files written by safetensors
def test_library_written_file_roundtrips_every_dtype(tmp_path):
    g = torch.Generator().manual_seed(0)
    t = {"f32": torch.randn(3, 5, generator=g), "bf16": torch.randn(4, 7, generator=g).to(torch.bfloat16),
         "e4m3": torch.randn(8, 16, generator=g).to(torch.float8_e4m3fn),
         "e8m0": torch.randint(100, 140, (6,), generator=g, dtype=torch.uint8).view(torch.float8_e8m0fnu),
         "u8": torch.randint(0, 255, (2, 9), generator=g, dtype=torch.uint8),
         "i32": torch.randint(-1000, 1000, (5,), generator=g, dtype=torch.int32),
         "empty": torch.zeros(0, 4)}
    p = str(tmp_path / "m.safetensors")
    save_file(t, p, metadata={"format": "pt"})
    mf = xstar_cpp.MMapFile(p)
    meta = xstar_cpp.parse_safetensors_header(mf)
    assert set(meta) == set(t)
    want = {"f32": D.Float32, "bf16": D.BFloat16, "e4m3": D.Float8E4M3, "e8m0": D.Float8E8M0, "u8": D.UInt8,
            "i32": D.Int32, "empty": D.Float32}
    for k, v in t.items():
        assert list(meta[k].shape) == list(v.shape) and meta[k].dtype == want[k]
        assert np.array_equal(_view_bytes(mf, meta[k]), v.contiguous().view(torch.uint8).reshape(-1).numpy()), k


# ---------------------------------------------------------- the layer loader
def _fp8_layer(E=3, H=256, I=128, seed=0, shared=True, bias=True):
    g = torch.Generator().manual_seed(seed)
    t = {"m.gate.weight": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)}
    if bias:
        t["m.gate.e_score_correction_bias"] = torch.randn(E, generator=g)
    names = [f"m.experts.{e}" for e in range(E)] + (["m.shared_experts"] if shared else [])
    for b in names:
        for proj, (n, k) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"{b}.{proj}.weight"] = torch.randn(n, k, generator=g).to(torch.float8_e4m3fn)
            t[f"{b}.{proj}.weight_scale_inv"] = torch.rand(n // 128, k // 128, generator=g) + 0.5
    return t


def _u8(x):
    return x.contiguous().view(torch.uint8) if x.dtype != torch.float32 else x


def _check_stacked(w, t, E, shared=True):
    H, I = w.H, w.I
    assert (w.E, H, I) == (E, 256, 128)
    w13 = cpp_to_torch(w.w13, (E, 2 * I, H))
    s13 = cpp_to_torch(w.w13_scale, (E, 2 * I // 128, H // 128))
    w2 = cpp_to_torch(w.w2, (E, H, I))
    s2 = cpp_to_torch(w.w2_scale, (E, H // 128, I // 128))
    for e in range(E):
        b = f"m.experts.{e}"
        assert torch.equal(w13[e], torch.cat([_u8(t[f"{b}.gate_proj.weight"]), _u8(t[f"{b}.up_proj.weight"])]))
        assert torch.equal(s13[e], torch.cat([t[f"{b}.gate_proj.weight_scale_inv"], t[f"{b}.up_proj.weight_scale_inv"]]))
        assert torch.equal(w2[e], _u8(t[f"{b}.down_proj.weight"]))
        assert torch.equal(s2[e], t[f"{b}.down_proj.weight_scale_inv"])
    rw = cpp_to_torch(w.router_w, (E, H))
    assert torch.equal(rw.view(torch.int16), t["m.gate.weight"].view(torch.int16))
    if shared:
        sw13 = cpp_to_torch(w.shared_w13, (2 * I, H))
        assert torch.equal(sw13, torch.cat([_u8(t["m.shared_experts.gate_proj.weight"]),
                                            _u8(t["m.shared_experts.up_proj.weight"])]))
        assert torch.equal(cpp_to_torch(w.shared_w2_scale, (H // 128, I // 128)),
                           t["m.shared_experts.down_proj.weight_scale_inv"])
    else:
        assert w.shared_w13 is None and w.shared_w2 is None


def test_load_fp8_layer_stacks_gate_up_on_host(tmp_path):
    t = _fp8_layer()
    p = str(tmp_path / "l.safetensors")
    save_file(t, p)
    w = xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CPU)
    _check_stacked(w, t, 3)
    assert torch.equal(cpp_to_torch(w.router_bias, (3,)), t["m.gate.e_score_correction_bias"])
    # packed copies are made on the GPU only
    assert w.w13_frag is None
    with pytest.raises(RuntimeError, match="unsupported device"):
        xstar_cpp.pack_moe_layer_frag(w)
    assert w.w13_frag is None


def test_load_sharded_checkpoint_without_shared_or_bias(tmp_path):
    t = _fp8_layer(E=4, shared=False, bias=False, seed=1)
    keys = sorted(t)
    p1, p2 = str(tmp_path / "a.safetensors"), str(tmp_path / "b.safetensors")
    save_file({k: t[k] for k in keys[::2]}, p1)
    save_file({k: t[k] for k in keys[1::2]}, p2)
    w = xstar_cpp.load_moe_layer([p1, p2], "m", xstar_cpp.Device.CPU)
    _check_stacked(w, t, 4, shared=False)
    assert w.router_bias is None


def test_loader_errors(tmp_path):
    t = _fp8_layer()
    p = str(tmp_path / "l.safetensors")
    bad = dict(t)
    del bad["m.experts.1.up_proj.weight_scale_inv"]
    save_file(bad, p)
    with pytest.raises(RuntimeError, match="missing weight key: m.experts.1.up_proj.weight_scale_inv"):
        xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CPU)
    bad = dict(t)
    bad["m.experts.2.down_proj.weight"] = torch.zeros(256, 256, dtype=torch.float8_e4m3fn)
    save_file(bad, p)
    with pytest.raises(RuntimeError, match="shape mismatch: m.experts.2.down_proj.weight"):
        xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CPU)
    bad = dict(t)
    bad["m.experts.3.gate_proj.weight"] = t["m.experts.0.gate_proj.weight"].clone()
    save_file(bad, p)
    with pytest.raises(RuntimeError, match="more experts than router rows"):
        xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CPU)
    save_file(t, p)
    with pytest.raises(RuntimeError, match="duplicate weight key"):
        xstar_cpp.load_moe_layer([p, p], "m", xstar_cpp.Device.CPU)
    dense = {k: (v.float() if v.dtype == torch.float8_e4m3fn else v) for k, v in t.items() if "scale_inv" not in k}
    save_file(dense, p)
    with pytest.raises(RuntimeError, match="unsupported device"):   # dense weights are quantized on the GPU
        xstar_cpp.load_moe_layer([p], "m", xstar_cpp.Device.CPU)


def test_rejects_byte_count_overflow(tmp_path):
    """shape product fits 64 bits but times the dtype size wraps to 0; a wrapped
    count must not pass the data_offsets check."""
    p = tmp_path / "a"
    hb = json.dumps({"w": {"dtype": "F32", "shape": [2 ** 31, 2 ** 31], "data_offsets": [0, 0]}}).encode()
    hb += b" " * ((-len(hb)) % 8)
    p.write_bytes(struct.pack("<Q", len(hb)) + hb)
    with pytest.raises(RuntimeError, match="element count overflows"):
        xstar_cpp.parse_safetensors_header(xstar_cpp.MMapFile(str(p)))


def test_weight_view_rejects_byte_count_overflow(tmp_path):
    p = _raw_file(tmp_path / "a.safetensors", {"w": ("F32", [2], b"\0" * 8)})
    mf = xstar_cpp.MMapFile(p)
    with pytest.raises(RuntimeError, match="element count overflows"):
        xstar_cpp.make_weight_view(mf, 0, [2 ** 62], D.Float32)
    with pytest.raises(RuntimeError, match="element count overflows"):
        xstar_cpp.make_weight_view(mf, 0, [2 ** 40, 2 ** 40], D.Float32)
