"""Writes the committed golden fixtures under tests/golden/.

Run in the build container (it needs /root/reference only for the _ref vectors):
    python tests/golden/make_golden.py

codecs.npz      -- library answers for the number formats: torch.float8_e4m3fn
                   decode of all 256 codes and RNE encode of 40k sampled f32
                   values (|x| < 464, where torch's cast does not overflow),
                   torch.float8_e8m0fnu decode of all 256 codes, torch's f32 -> bf16
                   cast of 40k sampled values (finite, RNE).
ref_vectors.npz -- outputs of the reference's own CPU code compiled from its
                   sources (oracle/_ref/libxsref.so): gemm_cpu<float> and
                   gemm_cpu<bfloat16> with transB = true (xstar_cpp/include/ops/gemm.h:57-83),
                   bfloat16(float) (xstar_cpp/src/bfloat16.cpp:5-25), sigmoid/silu
                   (xstar_cpp/src/ops/mlp.cpp:10-26), and the reference mlp()
                   composition (mlp.cpp:71-83: linear -> silu*up -> linear, f32)
                   on seeded inputs.
"""
import ctypes as C
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def codecs():
    rng = np.random.default_rng(1234)
    codes = torch.arange(256, dtype=torch.uint8)
    e4m3_tab = codes.view(torch.float8_e4m3fn).float().numpy()
    e8m0_tab = codes.view(torch.float8_e8m0fnu).float().numpy()
    mag = np.exp(rng.uniform(np.log(1e-5), np.log(463.9), 40000)).astype(np.float32)
    sgn = np.where(rng.random(40000) < 0.5, -1.0, 1.0).astype(np.float32)
    e4_in = mag * sgn
    # exact ties between neighbouring codes, where RNE matters most
    grid = e4m3_tab[np.isfinite(e4m3_tab)]
    grid = np.unique(np.abs(grid))
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    e4_in = np.concatenate([e4_in, mids, -mids, grid, -grid]).astype(np.float32)
    e4_out = torch.from_numpy(e4_in).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bf_in = (rng.standard_normal(40000) * np.exp(rng.uniform(-30, 30, 40000))).astype(np.float32)
    bf_out = torch.from_numpy(bf_in).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(os.path.join(HERE, "codecs.npz"), e4m3_table=e4m3_tab,
                        e8m0_table=e8m0_tab, e4m3_enc_in=e4_in, e4m3_enc_out=e4_out,
                        bf16_in=bf_in, bf16_out=bf_out)


def ref_vectors():
    oracle.build(ref=True)
    R = oracle.ref_lib()
    assert R is not None, "oracle/_ref did not build"
    rng = np.random.default_rng(99)
    out = {}
    p = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    # gemm_cpu<float> transB, shapes covering odd sizes and the router shape class
    for name, (m, k, n) in {"g1": (5, 20, 7), "g2": (16, 256, 8), "g3": (2, 4096, 16)}.items():
        A = rng.standard_normal((m, k)).astype(np.float32)
        B = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        Cm = np.empty((m, n), np.float32)
        R.xsref_gemm_f32(p(A), p(B), p(Cm), m, k, n, 1)
        out[f"{name}_A"], out[f"{name}_B"], out[f"{name}_C"] = A, B, Cm
        Ab = oracle.bf16_from_f32(A)
        Bb = oracle.bf16_from_f32(B)
        Cb = np.empty((m, n), np.uint16)
        R.xsref_gemm_bf16(p(Ab), p(Bb), p(Cb), m, k, n, 1)
        out[f"{name}_Ab"], out[f"{name}_Bb"], out[f"{name}_Cb"] = Ab, Bb, Cb
    xs = np.concatenate([np.linspace(-100, 100, 4001, dtype=np.float32),
                         (rng.standard_normal(4000) * 8).astype(np.float32)])
    sg = np.empty_like(xs)
    sl = np.empty_like(xs)
    R.xsref_sigmoid(p(xs), p(sg), xs.size)
    R.xsref_silu(p(xs), p(sl), xs.size)
    out["act_x"], out["sigmoid"], out["silu"] = xs, sg, sl
    bfi = (rng.standard_normal(10000) * np.exp(rng.uniform(-20, 20, 10000))).astype(np.float32)
    bfo = np.empty(bfi.shape, np.uint16)
    R.xsref_bf16_from_f32(p(bfi), p(bfo), bfi.size)
    out["bf16_in"], out["bf16_out"] = bfi, bfo
    # reference mlp() (f32): linear(x, gate_up) -> silu(g)*u -> linear(act, down)
    T, H, I = 16, 256, 128
    x = (rng.standard_normal((T, H)) * 0.02).astype(np.float32)
    w13 = (rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((H, I)) * 0.02).astype(np.float32)
    gu = np.empty((T, 2 * I), np.float32)
    R.xsref_gemm_f32(p(x), p(w13), p(gu), T, H, 2 * I, 1)
    g = np.ascontiguousarray(gu[:, :I])
    s = np.empty_like(g)
    R.xsref_silu(p(g), p(s), g.size)
    act = np.ascontiguousarray((s * gu[:, I:]).astype(np.float32))
    y = np.empty((T, H), np.float32)
    R.xsref_gemm_f32(p(act), p(w2), p(y), T, I, H, 1)
    out.update(mlp_x=x, mlp_w13=w13, mlp_w2=w2, mlp_y=y)
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)


if __name__ == "__main__":
    codecs()
    ref_vectors()
    print("wrote", os.listdir(HERE))
