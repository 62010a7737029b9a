"""Turn the tall-tile LDS-ring kernel of moe_gemm_wide.hip into host C++ for
emu.hpp, in namespace xs::wide: the reference of the weight-direct prefill
kernel's bit-identity check (the same per-row arithmetic on 192-row tiles).

usage: gen_wide.py <moe_gemm_wide.hip> <out.inc>"""
import sys

from gen_wd import drop_fn, replace


def main(src_path, out_path):
    src = open(src_path).read()
    i = src.index("namespace xs {\nnamespace {") + len("namespace xs {\nnamespace {")
    j = src.index("template <int BM, bool GATEUP, int NW>\nint launch_wide(", i)
    body = src[i:j]
    for sig in ["__device__ __forceinline__ uint32_t lds_addr(", "__device__ __forceinline__ void dma16(",
                "__device__ __forceinline__ void dma16_nt(", "__device__ __forceinline__ void dma4(",
                "template <int N>\n__device__ __forceinline__ void wait_vm()"]:
        body = drop_fn(body, sig)
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) uint8_t smem[];",
                   "uint8_t *smem = emu_smem();")
    assert "asm volatile" not in body, "an asm statement the emulator has no stand-in for"
    pre = """// generated from moe_gemm_wide.hip by gen_wide.py
#include "xs_moe.h"
namespace xs {
namespace wide {
namespace {
"""
    open(out_path, "w").write(pre + body + "}  // namespace\n}  // namespace wide\n}  // namespace xs\n")


if __name__ == "__main__":
    main(*sys.argv[1:3])
