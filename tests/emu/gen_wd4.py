"""Turn the device part of moe_gemm_wd4.hip into host C++ for emu.hpp.

usage: gen_wd4.py <moe_gemm_wd4.hip> <moe_gemm.hpp> <out.inc>

As gen_wd.py: the kernel is used as written, its hardware helpers replaced
by emu.hpp's stand-ins, its register loads counted in the lane's vmcnt queue."""
import sys

from gen_wd import drop_fn, replace


def main(src_path, hdr_path, out_path):
    src = open(src_path).read()
    hdr = open(hdr_path).read()
    i = src.index("namespace xs {")
    j = src.index("template <bool GATEUP, int BM>\nint launch_wd4(", i)
    body = src[i:j] + "}  // namespace\n}  // namespace xs\n"
    for sig in ["__device__ __forceinline__ uint32_t lds_addr(", "__device__ __forceinline__ void dma16(",
                "__device__ __forceinline__ void dma4(",
                "template <int N>\n__device__ __forceinline__ void wait_vm()",
                "__device__ __forceinline__ void barrier_lds()"]:
        body = drop_fn(body, sig)
    body = replace(body, "typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;")
    body = replace(body, "typedef const __attribute__((address_space(1))) uint8_t gu8;", "typedef const uint8_t gu8;")
    body = replace(body, "__builtin_nontemporal_load((gv4i *)(", "wd_gload((")
    body = replace(body, "*(gv4i *)(", "wd_gload(")
    body = replace(body, "*(gu8 *)(", "wd_gload1(")
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) uint8_t smem[];",
                   "uint8_t *smem = emu_smem();")
    assert "asm volatile" not in body, "an asm statement the emulator has no stand-in for"
    ga = hdr[hdr.index("struct GemmArgs"):]
    ga = ga[:ga.index("};") + 2]
    pre = """// generated from moe_gemm_wd4.hip by gen_wd4.py
namespace xs {
""" + ga + """
}
inline void barrier_lds() { __syncthreads(); }
// compiler-visible register loads: read now (the compiler waits for them
// before any use), counted in the lane's vmcnt queue as the hardware counts them
inline v4i wd_gload(const uint8_t *p)
{
    if (!emu_check_global(p, 16)) EMU_ERR("weight load %p outside every buffer", (const void *)p);
    v4i v;
    memcpy(&v, p, 16);
    push(Op{2, nullptr, 0, 0, nullptr, nullptr});
    return v;
}
inline uint8_t wd_gload1(const uint8_t *p)
{
    if (!emu_check_global(p, 1)) EMU_ERR("scale load %p outside every buffer", (const void *)p);
    push(Op{2, nullptr, 0, 0, nullptr, nullptr});
    return *p;
}
"""
    open(out_path, "w").write(pre + body)


if __name__ == "__main__":
    main(*sys.argv[1:4])
