"""Turn the library's sources into host C++ for the whole-forward emulation
(fwd_main.cpp, hip_emu.hpp): the C ABI, the dispatch and the launchers run as
written, and every kernel launch runs the kernel's source on the CPU.

usage: gen_fwd.py <csrc/hip dir> <out dir>

Per source file the hardware helpers (asm DMAs, vmcnt waits, LDS address
casts) give way to emu.hpp's stand-ins, LDS arrays come from the block's
emulated LDS, and `k<<<grid, block, smem, st>>>(args)` becomes a synchronous
emu_kl launch.  The weight-direct GEMMs' register loads count in
the lane's vmcnt queue (emu.hpp); the single dense GEMM's sc1 partial-tile
accesses become plain bounds-checked ones.  Every replacement is asserted."""
import os
import re
import sys

from gen_wd import replace

PER_LANE_DMA = """inline void {name}(const void *g, uint32_t lds)
{{
    lds = (uint32_t)wave_first(lds, "{name} lds");
    dma_lane((const uint8_t *)g, lds, {n}, "{name}");
}}
"""

HELPERS = {
    "moe_gemm.hip": [
        ("__device__ __forceinline__ uint32_t lds_off(", "inline uint32_t lds_off(const void *p) { return lds_addr(p); }\n"),
        ("__device__ __forceinline__ void dma16(", PER_LANE_DMA.format(name="dma16", n=16)),
        ("__device__ __forceinline__ void dma16_nt(", PER_LANE_DMA.format(name="dma16_nt", n=16)),
        ("__device__ __forceinline__ void dma4(", PER_LANE_DMA.format(name="dma4", n=4)),
        ("template <int N>\n__device__ __forceinline__ void wait_vmcnt()",
         "template <int N>\ninline void wait_vmcnt() { emu_wait(N); }\n"),
    ],
    "moe_gemm_stream.hip": [
        ("__device__ __forceinline__ uint32_t lds_addr(", ""),
        ("__device__ __forceinline__ void dma16_v(", PER_LANE_DMA.format(name="dma16_v", n=16)),
        ("__device__ __forceinline__ void dma16_s(",
         "inline void dma16_s(const uint8_t *sbase, uint32_t voff, uint32_t lds) { dma16(sbase, voff, lds); }\n"),
        ("__device__ __forceinline__ void dma16_s_nt(",
         "inline void dma16_s_nt(const uint8_t *sbase, uint32_t voff, uint32_t lds) { dma16(sbase, voff, lds); }\n"),
        ("__device__ __forceinline__ void dma4_v(", PER_LANE_DMA.format(name="dma4_v", n=4)),
        ("template <int N>\n__device__ __forceinline__ void wait_vm()", ""),
    ],
    "moe_gemm_wide.hip": [
        ("__device__ __forceinline__ uint32_t lds_addr(", ""),
        ("__device__ __forceinline__ void dma16(", ""),
        ("__device__ __forceinline__ void dma16_nt(", ""),
        ("__device__ __forceinline__ void dma4(", ""),
        ("template <int N>\n__device__ __forceinline__ void wait_vm()", ""),
    ],
    "moe_router.hip": [
        ("__device__ __forceinline__ uint32_t rt_lds(", "inline uint32_t rt_lds(const void *p) { return lds_addr(p); }\n"),
        ("__device__ __forceinline__ void rt_dma16(", "inline void rt_dma16(const void *g, uint32_t lds) { dma16x(g, lds); }\n"),
        ("template <int N>\n__device__ __forceinline__ void rt_wait_vm()",
         "template <int N>\ninline void rt_wait_vm() { emu_wait(N); }\n"),
    ],
}

WD_COMMON = [
    ("__device__ __forceinline__ uint32_t lds_addr(", ""),
    ("__device__ __forceinline__ void dma16(", ""),
    ("__device__ __forceinline__ void dma4(", ""),
    ("template <int N>\n__device__ __forceinline__ void wait_vm()", ""),
    ("__device__ __forceinline__ void barrier_lds()", "inline void barrier_lds() { __syncthreads(); }\n"),
]
HELPERS["moe_gemm_wd.hip"] = WD_COMMON
# the single dense GEMM: its sc1 partial-tile store and load are plain
# bounds-checked 16-byte accesses here (x86 orders them before the counter's
# locked atomic, as the sc1 policy and the agent-scope atomic do on the card)
HELPERS["gemm_dense.hip"] = [
    ("__device__ __forceinline__ uint32_t lds_addr(", ""),
    ("__device__ __forceinline__ void dma16(", ""),
    ("__device__ __forceinline__ void dma4(", ""),
    ("template <int N>\n__device__ __forceinline__ void wait_vm()", ""),
    ("__device__ __forceinline__ void store16_coh(",
     "inline void store16_coh(float *p, v4f v)\n{\n"
     "    if (!emu_check_global(p, 16)) { EMU_ERR(\"store16_coh outside every buffer\"); return; }\n"
     "    memcpy(p, &v, 16);\n}\n"),
    ("__device__ __forceinline__ v4f load16_coh(",
     "inline v4f load16_coh(const float *base, uint32_t byte_off)\n{\n"
     "    const uint8_t *p = (const uint8_t *)base + byte_off;\n    v4f v = {0.f, 0.f, 0.f, 0.f};\n"
     "    if (!emu_check_global(p, 16)) { EMU_ERR(\"load16_coh outside every buffer\"); return v; }\n"
     "    memcpy(&v, p, 16);\n    return v;\n}\n"),
]
HELPERS["moe_gemm_wd4.hip"] = WD_COMMON
# compiler-visible register loads of the weight-direct kernels, and the empty
# asm statements that pin their folds in place (compiler constraints only)
TEXT = {
    "moe_gemm_wd.hip": [
        ("typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;"),
        ("__builtin_nontemporal_load((gv4i *)(", "wd_gload(("),
        ("*(gv4i *)(", "wd_gload("),
        ('asm volatile("" : "+v"(acc[fi][0]), "+v"(acc[fi][1]));', ""),
    ],
    # the decode kernel has no explicit counter waits: its loads are not queued
    "moe_gemm_wdd.hip": [
        ("typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;"),
        ("__builtin_nontemporal_load((gv4i *)(", "wd_gload_now(("),
        ("*(gv4i *)(", "wd_gload_now("),
        ('asm volatile("" : "+v"(acc[j]));', ""),
    ],
    "moe_gemm_wd4.hip": [
        ("typedef const __attribute__((address_space(1))) v4i gv4i;", "typedef const v4i gv4i;"),
        ("typedef const __attribute__((address_space(1))) uint8_t gu8;", "typedef const uint8_t gu8;"),
        ("__builtin_nontemporal_load((gv4i *)(", "wd_gload(("),
        ("*(gv4i *)(", "wd_gload("),
        ("*(gu8 *)(", "wd_gload1("),
    ],
}

FILES = ["gemm_dense.hip", "moe_gemm_wd.hip", "moe_gemm_wdd.hip", "moe_gemm_wd4.hip", "moe_forward.hip", "moe_router.hip", "moe_permute.hip", "moe_gemm.hip", "moe_gemm_stream.hip",
         "moe_gemm_wide.hip", "rmsnorm.hip", "xs_runtime.hip"]

STUBS = r"""// generated by gen_fwd.py: nothing to stub (every source is emulated)
"""


def swap_fn(s, sig, new):
    k = s.index(sig)
    e = s.index("\n}\n", k) + 3
    return s[:k] + new + s[e:]


def matching(s, i, open_ch, close_ch):
    """Index just past the bracket matching the one at s[i]."""
    depth = 0
    for j in range(i, len(s)):
        if s[j] == open_ch:
            depth += 1
        elif s[j] == close_ch:
            depth -= 1
            if depth == 0:
                return j + 1
    raise ValueError("unbalanced")


def rewrite_launches(s, src="?"):
    out, pos, n = [], 0, 0
    while True:
        i = s.find("<<<", pos)
        if i < 0:
            break
        # the kernel expression: an identifier with optional balanced template arguments
        j = i
        if s[j - 1] == ">":
            depth, j = 0, j - 1
            while True:
                if s[j] == ">":
                    depth += 1
                elif s[j] == "<":
                    depth -= 1
                    if depth == 0:
                        break
                j -= 1
        if s[j - 1] == "]":   # an indexed array of kernels: fns[i]<<<...>>>
            j = s.rindex("[", 0, j)
        k = j
        while k > 0 and (s[k - 1].isalnum() or s[k - 1] in "_:"):
            k -= 1
        name = s[k:i]
        e = s.index(">>>", i)
        cfg = s[i + 3:e]
        p = e + 3
        assert s[p] == "(", s[i - 40:p + 40]
        q = matching(s, p, "(", ")")
        args = s[p + 1:q - 1]
        out.append(s[pos:k])
        site = f"{src}:{name.split('<')[0]}#{n}"   # launch site, for EMU_KERNEL_LOG
        out.append(f"(emu_note_kernel(\"{site}\"), emu_kl([&] {{ {name}({args}); }}, {cfg}))")
        pos, n = q, n + 1
    out.append(s[pos:])
    return "".join(out), n


def transform(name, s):
    for sig, new in HELPERS.get(name, []):
        s = swap_fn(s, sig, new)
    for old, new in TEXT.get(name, []):
        s = replace(s, old, new)
    s = re.sub(r"extern __shared__ __attribute__\(\(aligned\(16\)\)\) (\w+) (\w+)\[\];",
               r"\1 *\2 = reinterpret_cast<\1 *>(emu_smem());", s)
    s = re.sub(r"__shared__ (\w+) (\w+)\[([^\]]+)\];", r"\1 *\2 = emu_shared<\1>(\3);", s)
    s = re.sub(r"__shared__ (\w+) (\w+);", r"\1 &\2 = *emu_shared<\1>(1);", s)
    assert "__shared__" not in s, name
    s, n = rewrite_launches(s, name)
    # each kernel notes its own instantiation once per launch (EMU_KERNEL_LOG),
    # after a leading #pragma of its body
    out, pos = [], 0
    for m in re.finditer(r"__global__[^;{]*?\)\s*\{", s):
        e = m.end()
        rest = s[e:]
        lead = len(rest) - len(rest.lstrip())
        if rest.lstrip().startswith("#pragma"):
            e += lead + rest.lstrip().index("\n") + 1
        out.append(s[pos:e] + " EMU_NOTE_KERNEL();")
        pos = e
    s = "".join(out) + s[pos:]
    assert "<<<" not in s
    assert "asm volatile" not in s, f"{name}: an asm statement the emulator has no stand-in for"
    return s


def main(src_dir, out_dir):
    os.makedirs(out_dir, exist_ok=True)
    for h in ("xs_device.hpp", "moe_internal.hpp", "moe_gemm.hpp"):
        t = open(os.path.join(src_dir, h)).read()
        if h == "xs_device.hpp":
            t = replace(t, "#include <hip/hip_runtime.h>", '#include "hip_emu.hpp"')
        open(os.path.join(out_dir, h), "w").write(t)
    for f in FILES:
        s = transform(f, open(os.path.join(src_dir, f)).read())
        open(os.path.join(out_dir, f.replace(".hip", ".cpp")), "w").write(
            f"// generated from {f} by gen_fwd.py\n#include \"hip_emu.hpp\"\n" + s)
    open(os.path.join(out_dir, "stubs.cpp"), "w").write('#include "hip_emu.hpp"\n' + STUBS)


if __name__ == "__main__":
    main(*sys.argv[1:3])
