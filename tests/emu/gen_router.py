"""Turn the device part of moe_router.hip (logits kernels, chain kernel,
route kernel) into host C++ for emu.hpp + router_emu.hpp.

usage: gen_router.py <moe_router.hip> <xs_device.hpp> <moe_internal.hpp> <out.inc>

The kernels are used as written.  Host launchers are dropped, the tile
kernel's asm DMA and wait helpers give way to emu.hpp's stand-ins, the dynamic
LDS arrays become the block's emulated LDS, and the device helpers the kernels
call (the reproducible exp and sigmoid, the wave max, load8 and the FP8 1x128
quantizer) and the device codecs (bf16, software e4m3 and e2m1 encoders) are
taken from their headers.  Every replacement is asserted."""
import sys

from gen_wd import drop_fn, replace


def take_fn(src, sig):
    k = src.index(sig)
    e = src.index("\n}\n", k) + 3
    return src[k:e]


def main(src_path, dev_path, int_path, out_path):
    src = open(src_path).read()
    dev = open(dev_path).read()
    inter = open(int_path).read()
    i = src.index("namespace xs {")
    j = src.index("// ---------------------------------------------------- activation quantizers", i)
    body = src[i:j]
    for sig in ["template <typename T>\nstatic int launch_chain(",
                "__device__ __forceinline__ uint32_t rt_lds(",
                "__device__ __forceinline__ void rt_dma16(",
                "template <int N>\n__device__ __forceinline__ void rt_wait_vm()",
                "int launch_route(", "int router_kind(", "int router_logits_splits(",
                "bool router_quantizes(", "int launch_router_logits(", "int launch_router_fix(",
                "int launch_route_block("]:
        body = drop_fn(body, sig)
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) float prod[];",
                   "float *prod = reinterpret_cast<float *>(emu_smem());")
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) uint8_t smem[];",
                   "uint8_t *smem = emu_smem();")
    body = replace(body, "rt_lds(smem)", "lds_addr(smem)")
    body = replace(body, "rt_dma16(", "dma16x(")
    body = replace(body, "rt_wait_vm<", "wait_vm<")
    body = replace(body, "#pragma clang fp contract(off)\n", "")
    assert "asm volatile" not in body, "an asm statement the emulator has no stand-in for"
    helpers = "".join(take_fn(dev, s) for s in [
        "__device__ __forceinline__ float xs_expf(", "__device__ __forceinline__ float xs_sigmoid(",
        "__device__ __forceinline__ float wave_max(",
        # the device codecs as written (xs::; the emulator's own same-named
        # stand-ins live outside the namespace), for the every-float checks
        "__device__ __forceinline__ uint16_t bf16_from_f32(", "__device__ __forceinline__ uint32_t e4m3_encode_sw(",
        "__device__ __forceinline__ uint32_t e2m1_encode_sw("])
    helpers += "".join(take_fn(inter, s) for s in [
        "__device__ __forceinline__ void load8(const uint16_t *p, float *v)",
        "__device__ __forceinline__ void load4(const uint16_t *p, float *v)",
        "__device__ __forceinline__ void load4(const float *p, float *v)",
        "__device__ __forceinline__ void quant8_fp8("])
    cert = inter[inter.index("struct CertState {"):]
    cert = cert[:cert.index("};") + 2]
    pre = """// generated from moe_router.hip by gen_router.py
#include "xs_moe.h"
namespace xs {
""" + cert + "\n" + helpers + "}  // namespace xs\n"
    open(out_path, "w").write(pre + body + "}  // namespace xs\n")


if __name__ == "__main__":
    main(*sys.argv[1:5])
