"""Check the LDS-DMA kernels' generated assembly for early uses of LDS reads.

    python check_lds_reads.py [source.hip ...]

The kernels that stage tiles with LDS DMA (gemm_big_kernel, attn_dma_kernel,
attn_prefill_dma_kernel) read LDS with inline-asm ds_read instructions and
wait for them with explicit s_waitcnt lgkmcnt(N): the compiler would otherwise
wait for every DMA in flight before each LDS read it can see. To the compiler
an inline-asm read's destination is ready at issue, so nothing but the kernel's
structure stops it from copying or reading that register before the wait that
covers it, which would use stale data. This script compiles the sources to
gfx950 assembly with the build's flags and scans each DMA kernel in program
order: a vector instruction (an LDS one included: its address or data) touching
the destination of a ds_read that no
lgkmcnt wait has covered yet (LDS operations complete in issue order, so
lgkmcnt(N) covers all but the N newest) is reported. The scan follows the text
and its fall-through edges, not the branches: after an unconditional branch
nothing falls through, so the next block starts with nothing in flight. The
kernels' step loops are unrolled, so every read sits in straight-line code next
to its wait; a read whose destination is copied on a branch edge (the way a
compiler moves registers into place for a join) appears as such a copy on the
fall-through side as well.

The same scan covers inline-asm vector-memory loads into registers (the
decode kernel's query loads, issued ahead of its first DMAs and waited for by
an explicit vmcnt): a vector instruction touching such a load's destination
before a vmcnt wait that covers it is reported. Only loads count towards
vmcnt(N) covering a load (stores may complete out of order with loads; loads,
DMAs included, complete in issue order), so vmcnt(N) covers a load once N or
more loads were issued after it.

A second scan covers every kernel of the sources: an inline-asm instruction
that reads the result of an MFMA. The compiler inserts the wait states an
MFMA result needs before its own instructions read it, but not before an asm
statement, so along every path of the control-flow graph (fall-through and
branch edges) from an MFMA writing a register to an asm instruction reading
it, at least MFMA_WAIT_STATES wait states must pass (one per instruction,
N + 1 per s_nop N): the most any MFMA needs on gfx950 (16-pass shapes), more
than the 8 the compiler itself keeps for a 16x16x32 result.

Exit status 1 if any such use is found.
"""

from __future__ import annotations

import concurrent.futures as cf
import re
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from build import COMMON_FLAGS, CSRC, FILE_FLAGS, hipcc  # noqa: E402

DEFAULT_SOURCES = ["gemm_bf16.hip", "gemm_f16.hip", "attn_bf16.hip", "attn_f16.hip"]
KERNELS = re.compile(r"^(_ZN4fxpr\w*(gemm_big_kernel|attn_dma_kernel|attn_prefill_dma_kernel)\w*):")
ALL_KERNELS = re.compile(r"^(_ZN4fxpr\w+):")
MFMA_WAIT_STATES = 19


def _vregs(tok: str) -> set[int]:
    tok = tok.strip(",|")
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


VMEM_LOAD = re.compile(r"^(global_load|buffer_load|flat_load|global_atomic\w*_rtn|buffer_atomic\w*_rtn)")


def scan_kernel(lines: list[str]) -> list[str]:
    """Early uses of pending ds_read destinations (and of pending inline-asm
    vector-memory load destinations) in one kernel's text."""
    pending: list[set[int]] = []  # LDS operations in flight, oldest first
    vpending: list[set[int]] = []  # vector-memory loads in flight, oldest first (asm destinations only)
    found = []
    in_asm = False
    for text in lines:
        t = text.strip()
        if t == ";;#ASMSTART":
            in_asm = True
            continue
        if t == ";;#ASMEND":
            in_asm = False
            continue
        if not t or t[0] in ";." or t.endswith(":"):
            continue
        op, _, rest = t.partition(" ")
        if op == "s_waitcnt":
            if "lgkmcnt" in t:
                n = int(re.search(r"lgkmcnt\((\d+)\)", t).group(1))
                pending = pending[len(pending) - n:] if 0 < n < len(pending) else ([] if n == 0 else pending)
            if "vmcnt" in t:
                n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
                vpending = vpending[len(vpending) - n:] if 0 < n < len(vpending) else ([] if n == 0 else vpending)
            continue
        if VMEM_LOAD.match(op):
            ops = rest.split()
            used = set()
            for tok in ops[1:]:
                used |= _vregs(tok)
            vlive = set().union(*vpending) if vpending else set()
            if used & vlive:
                found.append(f"{t}  (in flight: v{sorted(used & vlive)})")
            # a DMA (lds) names no destination; the compiler's own loads are
            # waited for by the compiler
            dest = _vregs(ops[0]) if ops and in_asm and "_lds" not in op and not rest.rstrip().endswith(" lds") else set()
            vpending.append(dest)
            continue
        if op.startswith("ds_"):
            ops = rest.split()
            # an LDS instruction's own operands (a read's address, a write's
            # address and data) must not be a pending read's destination
            # either: it may issue after that read has landed
            srcs = ops[1:] if op.startswith("ds_read") else ops
            used = set()
            for tok in srcs:
                used |= _vregs(tok)
            live = set().union(*pending) if pending else set()
            if any(vpending):
                live |= set().union(*vpending)
            if used & live:
                found.append(f"{t}  (in flight: v{sorted(used & live)})")
            pending.append(_vregs(ops[0]) if op.startswith("ds_read") and ops else set())
            continue
        if op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            pending = []  # the next instruction is reached only by a jump
            vpending = []
            continue
        if op.startswith("s_") or not (pending or any(vpending)):
            continue
        used = set()
        for tok in rest.split():
            used |= _vregs(tok)
        live = set().union(*pending) if pending else set()
        if any(vpending):
            live |= set().union(*vpending)
        if used & live:
            found.append(f"{t}  (in flight: v{sorted(used & live)})")
    return found


def _blocks(lines: list[str]) -> tuple[list[list[tuple[str, bool]]], list[list[int]]]:
    """Basic blocks of one kernel's text (instruction, inside inline asm) and
    each block's predecessors."""
    blocks: list[list[tuple[str, bool]]] = [[]]
    names: dict[str, int] = {}
    in_asm = False
    for text in lines:
        t = text.strip()
        if t == ";;#ASMSTART":
            in_asm = True
            continue
        if t == ";;#ASMEND":
            in_asm = False
            continue
        m = re.match(r"^(\.LBB\w+):", t)
        if m:
            if blocks[-1]:
                blocks.append([])
            names[m.group(1)] = len(blocks) - 1
            continue
        if not t or t[0] in ";.":
            continue
        blocks[-1].append((t, in_asm))
        if t.split()[0].startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            blocks.append([])
    preds: list[list[int]] = [[] for _ in blocks]
    for b, ins in enumerate(blocks):
        last = ins[-1][0].split() if ins else [""]
        if last[0].startswith(("s_branch", "s_cbranch")) and last[-1] in names:
            preds[names[last[-1]]].append(b)
        if b + 1 < len(blocks) and not last[0].startswith(("s_branch", "s_endpgm", "s_setpc")):
            preds[b + 1].append(b)
    return blocks, preds


def _wait_states(t: str) -> int:
    op = t.split()
    return int(op[1], 0) + 1 if op[0] == "s_nop" else 1


def scan_mfma_reads(lines: list[str], need: int = MFMA_WAIT_STATES) -> list[str]:
    """Inline-asm instructions naming an MFMA's destination registers fewer
    than `need` wait states after it on some path."""
    blocks, preds = _blocks(lines)
    found = []
    for b, ins in enumerate(blocks):
        for k, (t, in_asm) in enumerate(ins):
            if not in_asm:
                continue
            # every register the instruction names: a read of an MFMA result
            # too early sees the old value, a write (a load's destination)
            # too early can be overwritten by the MFMA's late write-back
            regs0: set[str] = set()
            for part in t.partition(" ")[2].replace(",", " ").split():
                regs0 |= _vregs(part)
            if not regs0:
                continue
            # backward search over (block, registers still traced). A
            # compiler-generated instruction naming a register ends its trace:
            # the compiler kept the MFMA's wait states before it, so the write
            # had landed by then.
            best: dict[tuple[int, frozenset], int] = {}
            work = [(b, k, 0, frozenset(regs0))]
            hit = None
            while work and hit is None:
                blk, pos, dist, regs = work.pop()
                for j in range(pos - 1, -1, -1):
                    u, u_asm = blocks[blk][j]
                    uop, _, urest = u.partition(" ")
                    if uop.startswith("v_mfma") and _vregs(urest.split(",")[0].strip()) & regs:
                        hit = (dist, u)
                        break
                    if not u_asm:
                        named: set[str] = set()
                        for part in urest.replace(",", " ").split():
                            named |= _vregs(part)
                        regs = regs - named
                        if not regs:
                            break
                    dist += _wait_states(u)
                    if dist >= need:
                        break
                else:
                    for p in preds[blk]:
                        if dist < best.get((p, regs), need):
                            best[(p, regs)] = dist
                            work.append((p, len(blocks[p]), dist, regs))
            if hit is not None:
                found.append(f"{t}  ({hit[0]} wait states after {hit[1]})")
    return found


def check_asm(path: Path) -> dict[str, list[str]]:
    src = path.read_text().splitlines()
    out: dict[str, list[str]] = {}
    i = 0
    while i < len(src):
        m = KERNELS.match(src[i])
        if not m:
            i += 1
            continue
        j = i + 1
        # to the function's end: blocks placed after an s_endpgm (an early
        # exit, or code the compiler lays out past the return) are scanned too
        while j < len(src) and not src[j].startswith(".Lfunc_end"):
            j += 1
        out[m.group(1)] = scan_kernel(src[i + 1:j])
        i = j
    return out


def check_mfma_asm(path: Path) -> dict[str, list[str]]:
    src = path.read_text().splitlines()
    out: dict[str, list[str]] = {}
    i = 0
    while i < len(src):
        m = ALL_KERNELS.match(src[i])
        if not m:
            i += 1
            continue
        j = i + 1
        while j < len(src) and not src[j].startswith(".Lfunc_end"):
            j += 1
        out[m.group(1)] = scan_mfma_reads(src[i + 1:j])
        i = j
    return out


def compile_asm(source: Path, out_dir: Path) -> Path:
    out = out_dir / (source.stem + ".s")
    flags = [f for f in COMMON_FLAGS if f != "-fPIC"] + FILE_FLAGS.get(source.name, [])
    res = subprocess.run([hipcc(), *flags, "-S", "--cuda-device-only", str(source), "-o", str(out)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S {source.name} failed:\n{res.stderr[-2000:]}")
    return out


def main(argv: list[str]) -> int:
    sources = [CSRC / s for s in (argv or DEFAULT_SOURCES)]
    bad = bad_mfma = 0
    with tempfile.TemporaryDirectory() as tmp, cf.ThreadPoolExecutor(max_workers=4) as ex:
        for asm in ex.map(lambda s: compile_asm(s, Path(tmp)), sources):
            for kernel, hits in check_asm(asm).items():
                if hits:
                    bad += len(hits)
                    print(f"{asm.stem}: {kernel}")
                    for h in hits[:8]:
                        print("   ", h)
            for kernel, hits in check_mfma_asm(asm).items():
                if hits:
                    bad_mfma += len(hits)
                    print(f"{asm.stem}: {kernel} (MFMA result read by inline asm)")
                    for h in hits[:8]:
                        print("   ", h)
    print("LDS read check:", "ok" if bad == 0 else f"{bad} early uses")
    print("MFMA result check:", "ok" if bad_mfma == 0 else f"{bad_mfma} asm reads too close")
    return 1 if bad or bad_mfma else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
