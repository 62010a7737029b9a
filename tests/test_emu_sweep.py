"""Emulated forwards aimed at kernel instantiations the fixed cases of
tests/test_emu_forward.py do not launch (found by logging, with
EMU_KERNEL_LOG, every instantiation the emulated suites run against the
kernel symbols of the built library):

- the combine for every top-k from 1 to 16, bf16 and f32 outputs;
- the one-block-per-tile GEMMs at 32- and 128-row tiles, FP8 and MXFP4, and
  MXFP4 at 16-row tiles;
- the persistent stream-K MXFP4 GEMMs at 32- and 64-row tiles;
- the approximate MFMA router's prefill (tile) kernel;
- K longer than every LDS ring, so each GEMM family's in-loop refills run;
- the no-allocation forward twice in a row, the second call smaller, on the
  shared scratch (stream-K, fused combine, exact pass, MXFP4);
- the routing kernels at each width (128, 256, 512 and 1024 experts), the
  one-launch decode routing and the prefill routing with its exact pass.

Each case gets the checks of the fixed cases, and the plan (GEMM family and
tile height) is asserted so that a case cannot pass on another kernel."""
from concurrent.futures import ThreadPoolExecutor

import pytest

from test_emu_forward import check_forward, fwd_emu, run_all, run_forward  # noqa: F401  (fwd_emu: fixture)

# args: T H I E k seed fp4 shared router x_f32 zipf norm residual noalloc
TILED = {"XS_MOE_STREAM": "0", "XS_MOE_GEMM": "tiled"}
CASES = [
    # name, env, args, routed GEMM family (0 tiled, 1 stream-K), tile rows
    ("fp8_tiled_bm32", TILED, (64, 256, 256, 8, 4, 201, 0, 1, 1, 0, 0, 0, 0, 0), 0, 32),
    ("fp8_tiled_bm128", TILED, (256, 256, 256, 8, 4, 202, 0, 1, 1, 0, 0, 0, 1, 0), 0, 128),
    ("fp8_tiled_bm128_f32", TILED, (256, 256, 128, 8, 4, 209, 0, 1, 2, 1, 0, 0, 0, 0), 0, 128),
    ("mxfp4_tiled_bm16", {"XS_MOE_STREAM": "0"}, (16, 512, 512, 16, 4, 203, 1, 1, 1, 0, 0, 0, 0, 0), 0, 16),
    ("mxfp4_tiled_bm32", {"XS_MOE_STREAM": "0"}, (64, 512, 512, 8, 4, 204, 1, 1, 1, 0, 0, 0, 0, 0), 0, 32),
    ("mxfp4_tiled_bm128", {"XS_MOE_STREAM": "0"}, (256, 512, 512, 8, 4, 205, 1, 0, 1, 0, 0, 0, 0, 0), 0, 128),
    ("mxfp4_stream_bm32", {"XS_MOE_STREAM": "1"}, (64, 512, 512, 8, 4, 206, 1, 1, 1, 0, 0, 0, 0, 0), 1, 32),
    ("mxfp4_stream_bm64", {"XS_MOE_STREAM": "1"}, (128, 512, 512, 8, 4, 207, 1, 1, 1, 0, 0, 0, 0, 0), 1, 64),
    ("mfma_router_prefill", {}, (300, 256, 256, 8, 2, 208, 0, 1, 0, 0, 0, 0, 0, 0), None, None),
    # K longer than every LDS ring (8 K steps and more), so each kernel's
    # in-loop refills run: tall tiles, stream-K, tiled at 32 and 128 rows,
    # MXFP4 stream-K (256-wide steps), the approximate router's tile kernel
    ("tall_deep_k", {}, (300, 1024, 1024, 4, 2, 220, 0, 1, 1, 0, 1.1, 0, 0, 0), 2, 192),
    ("stream_deep_k", {"XS_MOE_STREAM": "1"}, (64, 1024, 1024, 16, 4, 221, 0, 1, 1, 0, 0, 0, 0, 0), 1, 16),
    ("tiled_deep_k_bm32", TILED, (64, 1024, 1024, 8, 4, 222, 0, 1, 1, 0, 0, 0, 0, 0), 0, 32),
    ("tiled_deep_k_bm128", TILED, (256, 1024, 512, 8, 4, 223, 0, 0, 1, 0, 0, 0, 0, 0), 0, 128),
    ("mxfp4_stream_deep_k", {"XS_MOE_STREAM": "1"}, (64, 2048, 1024, 8, 4, 224, 1, 1, 1, 0, 0, 0, 0, 0), 1, 32),
    ("mfma_router_prefill_deep_k", {}, (300, 1024, 128, 8, 2, 225, 0, 0, 0, 0, 0, 0, 0, 0), None, None),
    # the no-allocation forward at T and then at a smaller T on the shared
    # scratch (which keeps the first call's contents) against the workspace
    # forward: stream-K counters and partial tiles, the fused combine's
    # counters, the certified router's list counters, MXFP4
    ("noalloc_seq_stream", {"EMU_NOALLOC_SEQ": "40", "XS_MOE_GEMM": "tiled", "XS_MOE_STREAM": "1",
                            "XS_STREAM_GROUPED": "0"}, (256, 512, 512, 64, 4, 230, 0, 1, 1, 0, 1.1, 0, 0, 0), 1, None),
    ("noalloc_seq_fused_combine", {"EMU_NOALLOC_SEQ": "300", "XS_MOE_GEMM": "wide", "XS_FUSE_COMBINE": "1"},
     (700, 256, 256, 16, 4, 231, 0, 1, 1, 0, 1.1, 0, 0, 0), 2, None),
    ("noalloc_seq_exact_pass", {"EMU_NOALLOC_SEQ": "20", "XS_ROUTER_MARGIN": "1e30"},
     (200, 512, 256, 32, 6, 232, 0, 1, 1, 0, 1.1, 0, 0, 0), None, None),
    ("noalloc_seq_mxfp4", {"EMU_NOALLOC_SEQ": "48"}, (160, 512, 512, 16, 6, 233, 1, 1, 1, 0, 1.1, 0, 0, 0), None, None),
    # routing widths (64 experts per lane group): the one-launch decode routing
    # at 128, 256 and 512 experts; the prefill routing launches, with every
    # token through the exact pass (margin) so the second routing runs too
    ("route_decode_e128", {}, (32, 256, 128, 128, 6, 210, 0, 1, 1, 0, 0, 0, 0, 0), None, None),
    ("route_decode_e256", {}, (32, 256, 128, 256, 8, 211, 0, 1, 1, 0, 0, 0, 0, 0), None, None),
    ("route_decode_e512", {}, (16, 256, 128, 512, 8, 212, 0, 1, 1, 0, 0, 0, 0, 0), None, None),
    ("route_prefill_e128_exact", {"XS_ROUTER_MARGIN": "1e30"}, (300, 256, 128, 128, 6, 213, 0, 1, 1, 0, 0, 0, 0, 0),
     None, None),
    ("route_prefill_e256_exact", {"XS_ROUTER_MARGIN": "1e30"}, (300, 256, 128, 256, 8, 214, 0, 1, 1, 0, 0, 0, 0, 0),
     None, None),
    ("route_prefill_e512_exact", {"XS_ROUTER_MARGIN": "1e30"}, (300, 256, 128, 512, 8, 215, 0, 1, 1, 0, 0, 0, 0, 0),
     None, None),
    ("route_prefill_e1024_exact", {"XS_ROUTER_MARGIN": "1e30"}, (260, 256, 128, 1024, 16, 216, 0, 0, 1, 0, 0, 0, 0, 0),
     None, None),
    ("route_prefill_e512_mfma", {}, (300, 256, 128, 512, 8, 217, 0, 1, 0, 0, 0, 0, 0, 0), None, None),
]


@pytest.fixture(scope="module")
def sweep_runs(fwd_emu):  # noqa: F811
    return run_all(fwd_emu, CASES)


@pytest.mark.parametrize("name,env,args,routed,rows", CASES, ids=[c[0] for c in CASES])
def test_forward_instantiation(sweep_runs, name, env, args, routed, rows):
    rc, out = sweep_runs[name]
    check_forward(rc, out, env, args, routed, rows)


def test_combine_every_top_k(fwd_emu):  # noqa: F811
    """The combine is compiled per top-k (1..16) and output type: each runs
    once, with a residual on odd k (f32 layers take the chain router)."""
    cases = [(k, xf32) for k in range(1, 17) for xf32 in (0, 1)]

    def one(c):
        k, xf32 = c
        args = (16, 256, 128, 16, k, 100 + k, 0, 1, 2 if xf32 else 1, xf32, 0, 0, k % 2, 0)
        rc, out = run_forward(fwd_emu, {}, args)
        try:
            check_forward(rc, out, {}, args)
            return None
        except AssertionError as e:
            return f"k={k} f32={xf32}: {str(e)[-1500:]}"

    with ThreadPoolExecutor(4) as ex:
        fails = [f for f in ex.map(one, cases) if f]
    assert not fails, "\n\n".join(fails[:3])
