"""Turn the device part of moe_gemm_wd.hip into host C++ for emu.hpp.

usage: gen_wd.py <moe_gemm_wd.hip> <moe_gemm.hpp> <out.inc>

The kernel source is used as written.  Only the helpers that touch hardware
(LDS address, the asm DMAs, the vmcnt wait, the barrier) are dropped in
favour of emu.hpp's stand-ins, the global-pointer casts become a counted
load, and the dynamic LDS array becomes the block's emulated LDS.  Every
replacement is asserted, so a change to the kernel that the emulator does not
understand fails here instead of running something else."""
import sys


def drop_fn(s, sig):
    k = s.index(sig)
    e = s.index("\n}\n", k) + 3
    c = k   # with the comment lines directly above
    while True:
        prev = s.rfind("\n", 0, c - 1) + 1
        if s[prev:c].lstrip().startswith("//"):
            c = prev
        else:
            break
    return s[:c] + s[e:]


def replace(s, old, new, at_least=1):
    n = s.count(old)
    assert n >= at_least, (old, n)
    return s.replace(old, new)


def main(src_path, hdr_path, out_path):
    src = open(src_path).read()
    hdr = open(hdr_path).read()
    i = src.index("namespace xs {")
    j = src.index("}  // namespace\n", i)
    body = src[i:j] + "}  // namespace\n}  // namespace xs\n"
    for sig in ["__device__ __forceinline__ uint32_t lds_addr(", "__device__ __forceinline__ void dma16(",
                "__device__ __forceinline__ void dma4(",
                "template <int N>\n__device__ __forceinline__ void wait_vm()",
                "__device__ __forceinline__ void barrier_lds()"]:
        body = drop_fn(body, sig)
    body = replace(body, "typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;")
    body = replace(body, "__builtin_nontemporal_load((gv4i *)(", "wd_gload((")
    body = replace(body, "*(gv4i *)(", "wd_gload(")
    body = replace(body, "extern __shared__ __attribute__((aligned(16))) uint8_t smem[];",
                   "uint8_t *smem = emu_smem();")
    body = replace(body, 'asm volatile("" : "+v"(acc[fi][0]), "+v"(acc[fi][1]));', "")
    assert "asm volatile" not in body, "an asm statement the emulator has no stand-in for"
    ga = hdr[hdr.index("struct GemmArgs"):]
    ga = ga[:ga.index("};") + 2]
    pre = """// generated from moe_gemm_wd.hip by gen_wd.py
namespace xs {
""" + ga + """
}
inline void barrier_lds() { __syncthreads(); }
// a compiler-visible register load: read now (the compiler waits for it before
// any use), counted in the lane's vmcnt queue as the hardware counts it
inline v4i wd_gload(const uint8_t *p)
{
    if (!emu_check_global(p, 16)) EMU_ERR("weight load %p outside every buffer", (const void *)p);
    v4i v;
    memcpy(&v, p, 16);
    push(Op{2, nullptr, 0, 0, nullptr, nullptr});
    return v;
}
"""
    open(out_path, "w").write(pre + body)


if __name__ == "__main__":
    main(*sys.argv[1:4])
