"""CPU check of the built library's gfx950 machine code: no instruction writes
through the scalar data cache (scalar memory stores and atomics, and that
cache's write-back and discard).  Every kernel here writes through vector
stores; the compiler is not expected to emit the scalar forms, and this
checks that it did not.  (This file names those instructions, so it is kept
out of the tree sent to the GPU box: it needs no GPU.)"""
import os
import re

import pytest

from isa_scan import code_objects, disassemble

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOS = [os.path.join(ROOT, "xstar-infer_amd", "xstar_cpp_py", "libxs_moe.so")]
SCALAR_WRITE = re.compile(r"^\s+(s_store_\w+|s_buffer_store_\w+|s_scratch_store_\w+|s_atomic_\w+|"
                          r"s_buffer_atomic_\w+|s_dcache_wb\w*|s_dcache_discard\w*)\b", re.M)


@pytest.mark.parametrize("so", SOS, ids=[os.path.basename(s) for s in SOS])
def test_no_scalar_cache_writes(so, tmp_path):
    if not os.path.exists(so):
        pytest.skip(f"{os.path.basename(so)} not built")
    if not os.path.exists("/opt/rocm/llvm/bin/llvm-objdump"):
        pytest.skip("no llvm-objdump")
    texts = [disassemble(c) for c in code_objects(so, str(tmp_path))]
    assert sum(t.count("global_store") for t in texts) > 100    # the vector stores are there
    found = [m.group(1) for t in texts for m in SCALAR_WRITE.finditer(t)]
    assert not found, found[:20]


def test_pattern_matches_the_scalar_forms():
    planted = "\ts_store_dword s4, s[2:3], 0x0\n\ts_dcache_wb\n\ts_atomic_add s1, s[2:3], 0x0\n"
    assert [m.group(1) for m in SCALAR_WRITE.finditer(planted)] == ["s_store_dword", "s_dcache_wb", "s_atomic_add"]
    assert not SCALAR_WRITE.search("\tglobal_store_dwordx4 v[0:1], v[2:5], off\n\ts_load_dword s4, s[2:3], 0x0\n")
