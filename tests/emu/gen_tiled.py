"""Turn the tiled expert GEMM kernel of moe_gemm.hip into host C++ for
emu.hpp, in namespace xs::tiled (the weight-direct kernels' generated code
defines GemmArgs and helpers of the same names).

usage: gen_tiled.py <moe_gemm.hip> <out.inc>

Used as the reference of the bit-identity checks: the weight-direct kernels
must hand the MFMAs the same operands, scales and K order."""
import sys

from gen_wd import drop_fn, replace


def main(src_path, out_path):
    src = open(src_path).read()
    i = src.index("namespace xs {") + len("namespace xs {")
    j = src.index("template <int BM, bool GATEUP, bool FP4>\nstatic int launch_one(", i)
    body = src[i:j]
    for sig in ["__device__ __forceinline__ uint32_t lds_off(", "__device__ __forceinline__ void dma16(",
                "__device__ __forceinline__ void dma16_nt(", "__device__ __forceinline__ void dma4(",
                "template <int N>\n__device__ __forceinline__ void wait_vmcnt()"]:
        body = drop_fn(body, sig)
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) uint8_t smem[];",
                   "uint8_t *smem = emu_smem();")
    assert "asm volatile" not in body, "an asm statement the emulator has no stand-in for"
    pre = """// generated from moe_gemm.hip by gen_tiled.py
namespace xs {
namespace tiled {
inline uint32_t lds_off(const void *p) { return lds_addr(p); }
inline void dma16(const void *g, uint32_t lds)
{
    lds = (uint32_t)wave_first(lds, "dma16 lds");
    dma_lane((const uint8_t *)g, lds, 16, "dma16");
}
inline void dma16_nt(const void *g, uint32_t lds) { dma16(g, lds); }
inline void dma4(const void *g, uint32_t lds)
{
    lds = (uint32_t)wave_first(lds, "dma4 lds");
    dma_lane((const uint8_t *)g, lds, 4, "dma4");
}
template <int N>
inline void wait_vmcnt() { emu_wait(N); }
"""
    open(out_path, "w").write(pre + body + "}  // namespace tiled\n}  // namespace xs\n")


if __name__ == "__main__":
    main(*sys.argv[1:3])
