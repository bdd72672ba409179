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
order: a vector instruction touching the destination of a ds_read that no
lgkmcnt wait has covered yet (LDS operations complete in issue order, so
lgkmcnt(N) covers all but the N newest) is reported. The scan follows the text
and its fall-through edges, not the branches: after an unconditional branch
nothing falls through, so the next block starts with nothing in flight. The
kernels' step loops are unrolled, so every read sits in straight-line code next
to its wait; a read whose destination is copied on a branch edge (the way a
compiler moves registers into place for a join) appears as such a copy on the
fall-through side as well.

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
from build import COMMON_FLAGS, CSRC, hipcc  # noqa: E402

DEFAULT_SOURCES = ["gemm_bf16.hip", "gemm_f16.hip", "attn_bf16.hip", "attn_f16.hip"]
KERNELS = re.compile(r"^(_ZN4fxpr\w*(gemm_big_kernel|attn_dma_kernel|attn_prefill_dma_kernel)\w*):")


def _vregs(tok: str) -> set[int]:
    tok = tok.strip(",|")
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def scan_kernel(lines: list[str]) -> list[str]:
    """Early uses of pending ds_read destinations in one kernel's text."""
    pending: list[set[int]] = []  # LDS operations in flight, oldest first
    found = []
    for text in lines:
        t = text.strip()
        if not t or t[0] in ";." or t.endswith(":"):
            continue
        op, _, rest = t.partition(" ")
        if op == "s_waitcnt" and "lgkmcnt" in t:
            n = int(re.search(r"lgkmcnt\((\d+)\)", t).group(1))
            pending = pending[len(pending) - n:] if 0 < n < len(pending) else ([] if n == 0 else pending)
            continue
        if op.startswith("ds_"):
            ops = rest.split()
            pending.append(_vregs(ops[0]) if op.startswith("ds_read") and ops else set())
            continue
        if op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            pending = []  # the next instruction is reached only by a jump
            continue
        if op.startswith("s_") or not pending:
            continue
        used = set()
        for tok in rest.split():
            used |= _vregs(tok)
        live = set().union(*pending)
        if used & live:
            found.append(f"{t}  (in flight: v{sorted(used & live)})")
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
        while j < len(src) and "s_endpgm" not in src[j]:
            j += 1
        out[m.group(1)] = scan_kernel(src[i + 1:j])
        i = j
    return out


def compile_asm(source: Path, out_dir: Path) -> Path:
    out = out_dir / (source.stem + ".s")
    flags = [f for f in COMMON_FLAGS if f != "-fPIC"]
    res = subprocess.run([hipcc(), *flags, "-S", "--cuda-device-only", str(source), "-o", str(out)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S {source.name} failed:\n{res.stderr[-2000:]}")
    return out


def main(argv: list[str]) -> int:
    sources = [CSRC / s for s in (argv or DEFAULT_SOURCES)]
    bad = 0
    with tempfile.TemporaryDirectory() as tmp, cf.ThreadPoolExecutor(max_workers=4) as ex:
        for asm in ex.map(lambda s: compile_asm(s, Path(tmp)), sources):
            for kernel, hits in check_asm(asm).items():
                if hits:
                    bad += len(hits)
                    print(f"{asm.stem}: {kernel}")
                    for h in hits[:8]:
                        print("   ", h)
    print("LDS read check:", "ok" if bad == 0 else f"{bad} early uses")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
