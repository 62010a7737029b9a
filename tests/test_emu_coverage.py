"""Which of the library's kernel instantiations the emulated suites launch
(opt-in: XS_EMU_COVERAGE=<log> names a log written by a run of
tests/test_emu_forward.py, test_emu_stages.py and test_emu_sweep.py with
EMU_KERNEL_LOG=<log> and XS_EMU_FULL=1).  Every instantiation must appear
except the weight-direct GEMMs' step-count variants, which their own
harnesses in tests/test_emu_kernels.py run."""
import os
import sys

import pytest

LOG = os.environ.get("XS_EMU_COVERAGE")
SO = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "xstar-infer_amd", "xstar_cpp_py",
                  "libxs_moe.so")
WEIGHT_DIRECT = ("moe_gemm_wd_kernel", "moe_gemm_wdd_kernel", "moe_gemm_wd4_kernel", "gemm_wd_dense_kernel")


@pytest.mark.skipif(not LOG, reason="set XS_EMU_COVERAGE=<EMU_KERNEL_LOG file of a full emulated run>")
def test_every_kernel_instantiation_is_emulated():
    # tests/emu is CPU test infrastructure that the GPU box does not receive:
    # imported here, not at collection
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "emu"))
    from kernel_coverage import launched, library_kernels
    lib, hit = library_kernels(SO), launched(LOG)
    missing = sorted(k for k in lib - hit if not k.startswith(WEIGHT_DIRECT))
    assert not missing, missing
