"""Static checks over the gfx950 machine code of the built libxs_moe.so
(run by build.py on every build, and by tests/test_isa_hazards.py).

The GEMM kernels issue their LDS DMAs from inline asm, where the compiler's
hazard recognizer does not look, and the dense kernel loads split-K partials
through inline-asm VMEM loads whose destination registers the compiler
believes are written at issue.  Three faults of that kind are checked on the
disassembly (AMD's own llvm-objdump over code objects built here):

  m0      an LDS DMA (`global_load_lds_*`, `buffer_load_* ... lds`) less than
          one wait state after an SALU write of M0: the DMA would land at the
          previous M0's LDS address;
  sgpr    a VMEM instruction reading an SGPR fewer than five wait states after
          a `v_readfirstlane`/`v_readlane` wrote it;
  vmem    a VGPR read or written while a VMEM load into it is still
          outstanding (no `s_waitcnt vmcnt` has retired it): the load would
          land late, over a register already reused.  A later VMEM load into
          the same register is allowed: loads return in issue order.

Each basic block is scanned in straight-line order; the vmcnt model retires
all but the N most recent VMEM operations at `s_waitcnt vmcnt(N)` (on gfx9
stores and LDS DMAs count in vmcnt too) and starts empty at every branch
target, so a block entered from elsewhere is not checked across the edge.
"""
import os
import re
import subprocess

LLVM = "/opt/rocm/llvm/bin"
_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(so_path, workdir):
    """Extract each translation unit's gfx950 code object from a HIP .so."""
    fat = os.path.join(workdir, "fat.bin")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", so_path, fat], check=True)
    data = open(fat, "rb").read()
    starts = [m.start() for m in re.finditer(re.escape(_BUNDLE_MAGIC), data)]
    out = []
    for n, s in enumerate(starts):
        e = starts[n + 1] if n + 1 < len(starts) else len(data)
        b = os.path.join(workdir, f"b{n}.bin")
        co = os.path.join(workdir, f"c{n}.co")
        with open(b, "wb") as f:
            f.write(data[s:e])
        subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={b}", f"--output={co}"],
                       check=True)
        out.append(co)
    return out


def disassemble(co_path):
    r = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--symbolize-operands", "--mcpu=gfx950", co_path],
                       check=True, capture_output=True, text=True)
    return r.stdout


def _sregs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _blocks(text):
    """Instructions as (line, mnemonic, operand tokens, text); None marks a label."""
    out = []
    for ln, line in enumerate(text.split("\n"), 1):
        s = line.split("//")[0].split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        if s.endswith(":"):
            out.append(None)
            continue
        op = s.split()[0]
        toks = [t.strip().split()[0] if t.strip() else "" for t in s[len(op):].split(",")]
        out.append((ln, op, toks, s))
    return out


def _is_lds_dma(op, text):
    return op.startswith("global_load_lds") or (op.startswith("buffer_load") and re.search(r"\blds\b", text))


def scan(text):
    """Return a list of (kind, line, instruction, detail) findings."""
    insts = _blocks(text)
    found = []
    pending = []        # outstanding VMEM ops in issue order: the VGPRs each will write
    for j, it in enumerate(insts):
        if it is None:
            pending = []
            continue
        ln, op, toks, s = it
        vmem = op.startswith(("global_", "buffer_", "flat_", "scratch_"))
        # wait states before this VMEM op
        if vmem:
            used = set().union(*(_sregs(t) for t in toks)) if toks else set()
            ws, k = 0, j - 1
            while k >= 0 and ws < 5 and insts[k] is not None:
                _, pop, ptoks, _ = insts[k]
                if ws < 1 and _is_lds_dma(op, s) and pop.startswith("s_") and ptoks and ptoks[0] == "m0":
                    found.append(("m0", ln, s, insts[k][3]))
                if pop.startswith(("v_readfirstlane", "v_readlane")) and _sregs(ptoks[0]) & used:
                    found.append(("sgpr", ln, s, f"{insts[k][3]} ({ws} wait states)"))
                ws += (int(ptoks[0], 0) + 1) if pop == "s_nop" else 1
                k -= 1
        # outstanding VMEM destinations
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", s)
            if m:
                n = int(m.group(1))
                pending = pending[len(pending) - n:] if n else []
            continue
        busy = set().union(*pending) if pending else set()
        vm_load = op.startswith(("global_load", "buffer_load", "scratch_load")) and not _is_lds_dma(op, s)
        # a VMEM load may name a register that an earlier load still targets:
        # loads return in issue order, so the later one lands last (its
        # address operands are still checked)
        toks_chk = toks[1:] if vm_load else toks
        touched = set().union(*(_vregs(t) for t in toks_chk)) if toks_chk else set()
        if busy & touched:
            found.append(("vmem", ln, s, f"v{min(busy & touched)} has a load in flight"))
        if vmem:
            returns = ("load" in op and not _is_lds_dma(op, s)) or ("atomic" in op and re.search(r"\bsc0\b", s))
            pending.append(_vregs(toks[0]) if returns else set())
        if op in ("s_endpgm", "s_branch", "s_setpc_b64"):
            pending = []
    return found
