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

The vmcnt model retires all but the N most recent VMEM operations at
`s_waitcnt vmcnt(N)` (on gfx9 stores and LDS DMAs count in vmcnt too).  It is
carried over the control-flow graph of each kernel (fall-through, branch and
loop back-edges): the loads in flight at a block's entry are the merge over
its predecessors, aligned from the most recent one, with the registers of
either path (a fixpoint over the graph), so a load issued before a branch or
in a previous loop iteration is checked where its register is used.  The
wait-state look-back of the m0 and sgpr rules follows the fall-through edge
and every branch into the block.
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


_LABEL = re.compile(r"^[0-9a-fA-F]*\s*<([^>]+)>:$")
_QMAX = 64          # vmcnt is 6 bits: older operations have retired


def _parse(text):
    """Instructions as (line, mnemonic, operand tokens, text) and labels as
    ("label", name), in text order."""
    out = []
    for ln, line in enumerate(text.split("\n"), 1):
        s = line.split("//")[0].split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        if s.endswith(":"):
            m = _LABEL.match(s)
            out.append(("label", m.group(1) if m else s[:-1].strip()))
            continue
        op = s.split()[0]
        toks = [t.strip().split()[0] if t.strip() else "" for t in s[len(op):].split(",")]
        out.append((ln, op, toks, s))
    return out


def _is_lds_dma(op, text):
    return op.startswith("global_load_lds") or (op.startswith("buffer_load") and re.search(r"\blds\b", text))


def _is_branch(op):
    return op == "s_branch" or op.startswith("s_cbranch")


def _ends_flow(op):
    return op in ("s_endpgm", "s_branch", "s_setpc_b64", "s_trap")


def _cfg(items):
    """Basic blocks of the instruction stream: [(first, last)] index ranges
    into items, the successor and predecessor lists, and the block that
    starts at each label."""
    starts = {0}
    for n, it in enumerate(items):
        if it[0] == "label":
            starts.add(n)
        elif _is_branch(it[1]) or _ends_flow(it[1]):
            starts.add(n + 1)
    starts = sorted(x for x in starts if x < len(items))
    blocks = [(a, (starts[i + 1] if i + 1 < len(starts) else len(items)) - 1) for i, a in enumerate(starts)]
    at_label = {}
    for b, (a, z) in enumerate(blocks):
        for n in range(a, z + 1):
            if items[n][0] == "label":
                at_label[items[n][1]] = b
    succ = [[] for _ in blocks]
    for b, (a, z) in enumerate(blocks):
        last = next((items[n] for n in range(z, a - 1, -1) if items[n][0] != "label"), None)
        if last is not None and _is_branch(last[1]):
            tgt = at_label.get(last[2][0])
            if tgt is not None:
                succ[b].append(tgt)
        if (last is None or not _ends_flow(last[1])) and b + 1 < len(blocks):
            # a new function (a non-L label) does not fall through from the last one
            nxt = items[blocks[b + 1][0]]
            if not (nxt[0] == "label" and not re.match(r"L\d+$", nxt[1])):
                succ[b].append(b + 1)
    pred = [[] for _ in blocks]
    for b, ss in enumerate(succ):
        for t in ss:
            pred[t].append(b)
    return blocks, succ, pred


def _merge(qa, qb):
    """Loads in flight on either of two paths, aligned from the most recent
    (register sets as bit masks)."""
    if qa is None:
        return qb
    n = max(len(qa), len(qb))
    pa, pb = (0,) * (n - len(qa)) + qa, (0,) * (n - len(qb)) + qb
    return tuple(x | y for x, y in zip(pa, pb))


def _mask(regs):
    m = 0
    for r in regs:
        m |= 1 << r
    return m


def _decode(it):
    """Per instruction: (vmcnt of an s_waitcnt or None, VGPR mask it touches
    (a load's destination excluded), VGPR mask a VMEM op will write on
    return or None when it is not a VMEM op)."""
    ln, op, toks, s = it
    if op == "s_waitcnt":
        m = re.search(r"vmcnt\((\d+)\)", s)
        return (int(m.group(1)) if m else None, 0, None)
    vmem = op.startswith(("global_", "buffer_", "flat_", "scratch_"))
    vm_load = op.startswith(("global_load", "buffer_load", "scratch_load")) and not _is_lds_dma(op, s)
    # a VMEM load may name a register that an earlier load still targets:
    # loads return in issue order, so the later one lands last (its address
    # operands are still checked)
    toks_chk = toks[1:] if vm_load else toks
    touched = _mask(set().union(*(_vregs(t) for t in toks_chk)) if toks_chk else ())
    dest = None
    if vmem:
        returns = ("load" in op and not _is_lds_dma(op, s)) or ("atomic" in op and re.search(r"\bsc0\b", s))
        dest = _mask(_vregs(toks[0])) if returns else 0
    return (None, touched, dest)


def _step(q, d):
    """The in-flight queue after one decoded instruction, and the mask of
    registers it touches that a load still targets."""
    wait, touched, dest = d
    if wait is not None:
        return (q[len(q) - wait:] if wait else ()), 0
    hit = 0
    if touched and q:
        busy = 0
        for x in q:
            busy |= x
        hit = busy & touched
    if dest is not None:
        q = (q + (dest,))[-_QMAX:]
    return q, hit


def _lookback(items, blocks, pred, b, n, depth=6):
    """Instructions before items[n] (block b) in execution order, newest first,
    over every path into the block, up to `depth` instructions per path."""
    paths = []

    def walk(blk, idx, acc, seen):
        a, _ = blocks[blk]
        k = idx
        while k >= a and len(acc) < depth:
            if items[k][0] != "label":
                acc = acc + [items[k]]
            k -= 1
        if len(acc) >= depth or not pred[blk]:
            paths.append(acc)
            return
        for p in pred[blk]:
            if (p, len(acc)) in seen:
                paths.append(acc)
                continue
            walk(p, blocks[p][1], acc, seen | {(p, len(acc))})

    walk(b, n - 1, [], frozenset())
    return paths


def _cheap_lookback(items, blocks, b, n):
    """The same look-back when the block itself holds five wait states before
    items[n] (the common case): one path, no graph walk; else None."""
    a, _ = blocks[b]
    acc, ws = [], 0
    for k in range(n - 1, a - 1, -1):
        if items[k][0] == "label":
            continue
        acc.append(items[k])
        _, pop, ptoks, _ = items[k]
        ws += (int(ptoks[0], 0) + 1) if pop == "s_nop" else 1
        if ws >= 5:
            return [acc]
    return None


def scan(text):
    """Return a list of (kind, line, instruction, detail) findings."""
    items = _parse(text)
    if not items:
        return []
    blocks, succ, pred = _cfg(items)
    dec = [None if it[0] == "label" else _decode(it) for it in items]
    # fixpoint of the in-flight queue at every block's entry
    entry = [None] * len(blocks)
    entry[0] = ()
    work = [0]
    for b in range(len(blocks)):
        if not pred[b] and entry[b] is None:
            entry[b] = ()
            work.append(b)
    while work:
        b = work.pop()
        q = entry[b]
        a, z = blocks[b]
        for n in range(a, z + 1):
            if dec[n] is not None:
                q, _ = _step(q, dec[n])
        for t in succ[b]:
            m = _merge(entry[t], q)
            if m != entry[t]:
                entry[t] = m
                work.append(t)
    found, seen = [], set()
    for b, (a, z) in enumerate(blocks):
        q = entry[b] if entry[b] is not None else ()
        for n in range(a, z + 1):
            it = items[n]
            if it[0] == "label":
                continue
            ln, op, toks, s = it
            if op.startswith(("global_", "buffer_", "flat_", "scratch_")):
                used = set().union(*(_sregs(t) for t in toks)) if toks else set()
                paths = _cheap_lookback(items, blocks, b, n) or _lookback(items, blocks, pred, b, n)
                for path in paths:
                    ws = 0
                    for prev in path:
                        if ws >= 5:
                            break
                        _, pop, ptoks, ps = prev
                        if ws < 1 and _is_lds_dma(op, s) and pop.startswith("s_") and ptoks and ptoks[0] == "m0":
                            key = ("m0", ln)
                            if key not in seen:
                                seen.add(key)
                                found.append(("m0", ln, s, ps))
                        if pop.startswith(("v_readfirstlane", "v_readlane")) and _sregs(ptoks[0]) & used:
                            key = ("sgpr", ln)
                            if key not in seen:
                                seen.add(key)
                                found.append(("sgpr", ln, s, f"{ps} ({ws} wait states)"))
                        ws += (int(ptoks[0], 0) + 1) if pop == "s_nop" else 1
            q, hit = _step(q, dec[n])
            if hit and ("vmem", ln) not in seen:
                seen.add(("vmem", ln))
                low = (hit & -hit).bit_length() - 1
                found.append(("vmem", ln, s, f"v{low} has a load in flight"))
    return found
