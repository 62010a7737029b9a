"""Turn the device part of moe_gemm_wdd.hip into host C++ for emu.hpp.

usage: gen_wdd.py <moe_gemm_wdd.hip> <moe_gemm.hpp> <out.inc>

As gen_wd.py: the kernel is used as written.  The global-pointer casts become
a counted load, the static __shared__ arrays come from the block's emulated
LDS, and the empty asm that pins the fold in place is dropped (it only
constrains the compiler)."""
import re
import sys

from gen_wd import replace


def main(src_path, hdr_path, out_path):
    src = open(src_path).read()
    hdr = open(hdr_path).read()
    i = src.index("namespace xs {")
    j = src.index("template <bool GATEUP, int KB>\nint launch_wdd(", i)
    body = src[i:j] + "}  // namespace\n}  // namespace xs\n"
    body = replace(body, "typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;")
    body = replace(body, "__builtin_nontemporal_load((gv4i *)(", "wd_gload((")
    body = replace(body, "*(gv4i *)(", "wd_gload(")
    body, n = re.subn(r"__shared__ (\w+) (\w+)\[([^\]]+)\];", r"\1 *\2 = emu_shared<\1>(\3);", body)
    assert n == 3, n
    body = replace(body, 'asm volatile("" : "+v"(acc[j]));', "")
    assert "asm volatile" not in body and "__shared__" not in body
    ga = hdr[hdr.index("struct GemmArgs"):]
    ga = ga[:ga.index("};") + 2]
    pre = """// generated from moe_gemm_wdd.hip by gen_wdd.py
namespace xs {
""" + ga + """
}
// a compiler-visible register load: read now (the compiler waits for it
// before any use; the kernel has no explicit counter waits to model)
inline v4i wd_gload(const uint8_t *p)
{
    if (!emu_check_global(p, 16)) EMU_ERR("register load %p outside every buffer", (const void *)p);
    v4i v;
    memcpy(&v, p, 16);
    return v;
}
"""
    open(out_path, "w").write(pre + body)


if __name__ == "__main__":
    main(*sys.argv[1:4])
