"""Static check of MFMA-to-VALU register hazards in gfx950 assembly built
here from this repository's kernels.

For every `v_mfma` of a kernel, every control-flow path that follows it is
walked up to `window` wait states (one per issued instruction; `s_nop N`
counts N + 1), and the fewest wait states before a non-MFMA VALU
instruction that

- writes a register the MFMA reads as its accumulator input (SrcC), "WARC";
- writes the MFMA's destination, "WAW";
- reads the MFMA's destination, "RAW"

are recorded.  A path stops following a register once something else has
written it.  The kernels are compiled with the library's own flags
(branchcraft-cuda_amd/build.py) into device-only assembly in a temporary
directory.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "branchcraft-cuda_amd" / "csrc"

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_LABEL = re.compile(r"^([.\w$]+):")


def vregs(text: str) -> frozenset:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            kind, lo, hi = m.group(1), int(m.group(2)), int(m.group(3))
        else:
            kind, lo = m.group(4), int(m.group(5))
            hi = lo
        out.update((kind, r) for r in range(lo, hi + 1))
    return frozenset(out)


def operands(args: str) -> list[str]:
    out, depth, cur = [], 0, ""
    for ch in args:
        depth += ch == "["
        depth -= ch == "]"
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def parse(lines: list[str]):
    """Instructions (op, args) of one function and its label positions."""
    insts, labels = [], {}
    for raw in lines:
        line = raw.split(";")[0].rstrip()
        if not line.strip():
            continue
        m = _LABEL.match(line)
        if m and not line.startswith(("\t", " ")):
            labels[m.group(1)] = len(insts)
            continue
        s = line.strip()
        if s.startswith("."):
            continue
        op = s.split()[0]
        insts.append((op, s[len(op):].strip()))
    return insts, labels


def successors(i, insts, labels):
    op, args = insts[i]
    if op == "s_endpgm":
        return []
    if op == "s_branch":
        return [labels[args.split()[0]]]
    if op.startswith("s_cbranch"):
        return [i + 1, labels[args.split()[0]]]
    return [i + 1]


def scan(insts, labels, window: int = 12) -> dict:
    """Fewest wait states per hazard kind over the function (absent kinds:
    none within `window`)."""
    n = len(insts)
    best: dict[str, int] = {}
    for i, (op, args) in enumerate(insts):
        if not op.startswith("v_mfma"):
            continue
        ops = operands(args)
        dst = vregs(ops[0])
        srcc = vregs(ops[3]) if len(ops) > 3 else frozenset()
        stack = [(s, 0, dst, srcc) for s in successors(i, insts, labels) if s < n]
        seen = set()
        while stack:
            j, ws, d, c = stack.pop()
            if ws > window or not (d or c) or (j, ws, d, c) in seen:
                continue
            seen.add((j, ws, d, c))
            op2, args2 = insts[j]
            if op2.startswith("v_") and not op2.startswith("v_mfma"):
                o2 = operands(args2)
                lane_only = op2.startswith(("v_cmp", "v_readlane", "v_readfirstlane"))
                wr = frozenset() if lane_only or not o2 else vregs(o2[0])
                rd = frozenset().union(*map(vregs, o2 if lane_only else o2[1:])) if o2 else frozenset()
                for kind, hit in (("RAW", rd & d), ("WAW", wr & d), ("WARC", wr & c)):
                    if hit and ws < best.get(kind, 1 << 30):
                        best[kind] = ws
                d, c = d - wr, c - wr
            elif op2.startswith("v_mfma"):
                d = d - vregs(operands(args2)[0])
            elif op2.startswith(("global_load", "buffer_load", "ds_read", "ds_load")):
                wr = vregs(operands(args2)[0])
                d, c = d - wr, c - wr
            cost = int(args2.split()[0], 0) + 1 if op2 == "s_nop" else 1
            stack.extend((s, ws + cost, d, c) for s in successors(j, insts, labels) if s < n)
    return best


def kernels(asm_text: str) -> dict[str, list[str]]:
    """Lines of every kernel function (symbols containing `kernel`)."""
    lines = asm_text.split("\n")
    out, cur, name = {}, None, None
    for line in lines:
        m = re.match(r"^(_Z\S*kernel\S*):", line)
        if m:
            name, cur = m.group(1), []
            continue
        if name is not None:
            if re.match(r"^\.Lfunc_end\d+:", line):
                out[name] = cur
                name, cur = None, None
            else:
                cur.append(line)
    return out


def compile_device_asm(source: Path, out_dir: Path) -> str:
    """gfx950 device assembly of one kernel source, with the library's flags."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    out = out_dir / (source.stem + ".s")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{CSRC}",
           "--cuda-device-only", "-S", str(source), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


def kernarg_rounds(lines: list[str]) -> list[int]:
    """Kernel-argument loads (`s_load*` from the kernarg pointer s[0:1]) issued
    before the kernel's first vector-memory load, grouped by the scalar waits
    between them: [3] is one round of three loads, [1, 2] two serial rounds."""
    groups, cur = [], 0
    for op, args in parse(lines)[0]:
        if op.startswith("s_load") and "s[0:1]" in args:
            cur += 1
        elif op == "s_waitcnt" and "lgkmcnt" in args and cur:
            groups.append(cur)
            cur = 0
        elif op.startswith(("global_load", "buffer_load", "flat_load")):
            break
    if cur:
        groups.append(cur)
    return groups
