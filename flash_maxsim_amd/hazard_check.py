"""Checks compiled gfx950 kernels for MFMA results touched too early.

A VALU, LDS or memory instruction that reads an MFMA's destination registers,
or writes them, must issue a number of wait states after the MFMA (8 for the
16x16x32 f16/bf16 form these kernels use; the compiler pads with s_nop inside
a basic block). Across a branch the compiler has been seen to place such an
instruction 3-7 wait states after the MFMA, which reads a stale register. This
module walks every path of each kernel's assembly (branch targets and loop
back edges included), counts wait states per path (one per instruction, N+1
per s_nop N) and reports every read or write of a pending MFMA result that
comes sooner than the limit.

Usage: ``python -m flash_maxsim_amd.hazard_check`` compiles every csrc/*.hip
to device assembly with the library's flags and prints the findings (exit
status 1 if there are any).
"""

from __future__ import annotations

import concurrent.futures
import re
import subprocess
import sys
import tempfile
from dataclasses import dataclass
from pathlib import Path

MFMA_WAIT_STATES = 8

_RANGE = re.compile(r"v\[(\d+):(\d+)\]$")
_SINGLE = re.compile(r"v(\d+)$")
_LABEL = re.compile(r"^(\.LBB\w+):")
_FUNC = re.compile(r"^([A-Za-z_]\w*):")
_WRITES_FIRST = ("buffer_load", "global_load", "flat_load", "ds_read", "scratch_load")


@dataclass(frozen=True)
class Finding:
    kernel: str
    mfma_line: int
    line: int
    wait_states: int
    kind: str  # "RAW" (read of the result) or "WAW" (overwrite of it)
    mfma: str
    instr: str


def _vregs(tok: str) -> frozenset:
    tok = tok.split()[0] if tok else ""
    m = _RANGE.match(tok)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _SINGLE.match(tok)
    return frozenset({int(m.group(1))}) if m else frozenset()


def _age(pending: dict, n: int, need: int) -> dict:
    return {k: w + n for k, w in pending.items() if w + n < need}


def _merge(a: dict, b: dict) -> dict:
    out = dict(a)
    for k, w in b.items():
        out[k] = min(out.get(k, w), w)
    return out


def check_asm(text: str, need: int = MFMA_WAIT_STATES) -> list[Finding]:
    """Findings for every kernel in an amdgcn assembly listing."""
    lines = text.split("\n")
    funcs: list[tuple[str, list[tuple[int, str]]]] = []
    for i, raw in enumerate(lines):
        s = raw.strip()
        m = _FUNC.match(s)
        if m and not s.startswith("."):
            funcs.append((m.group(1), []))
        elif funcs:
            funcs[-1][1].append((i, s))
    found: set[Finding] = set()
    for name, body in funcs:
        at_label: dict[str, dict] = {}
        # Three sweeps carry pending MFMAs along loop back edges.
        for _ in range(3):
            pending: dict = {}  # (regs, mfma line) -> wait states since the MFMA
            live = True
            for i, s in body:
                lab = _LABEL.match(s)
                if lab:
                    pending = _merge(pending if live else {}, at_label.get(lab.group(1), {}))
                    live = True
                    continue
                s = s.split(";")[0].strip()
                if not s or s.startswith("."):
                    continue
                op = s.split()[0]
                ops = [t.strip() for t in s[len(op):].split(",")]
                if op == "s_endpgm":
                    pending, live = {}, False
                    continue
                if op == "s_nop":
                    pending = _age(pending, int(ops[0], 0) + 1, need)
                    continue
                if not op.startswith("v_mfma"):
                    writes_first = (op.startswith("v_") and not op.startswith("v_cmp")) or op.startswith(
                        _WRITES_FIRST)
                    wr = _vregs(ops[0]) if writes_first and ops else frozenset()
                    rd = set()
                    for t in ops[1:] if writes_first else ops:
                        rd |= _vregs(t)
                    for (regs, ml), w in pending.items():
                        for kind, hit in (("RAW", rd & regs), ("WAW", wr & regs)):
                            if hit:
                                found.add(Finding(name, ml + 1, i + 1, w, kind, lines[ml].strip(), lines[i].strip()))
                    if wr:
                        pending = {(r - wr, ml): w for (r, ml), w in pending.items() if r - wr}
                pending = _age(pending, 1, need)
                if op.startswith("v_mfma"):
                    pending[(_vregs(ops[0]), i)] = 0
                if op.startswith("s_cbranch") or op == "s_branch":
                    tgt = ops[0].split()[0]
                    at_label[tgt] = _merge(at_label.get(tgt, {}), pending)
                    if op == "s_branch":
                        live = False
    return sorted(found, key=lambda f: (f.kernel, f.line))


def device_asm(src: Path, out_dir: Path) -> Path:
    """Compiles one HIP source to gfx950 assembly with the library's flags."""
    from flash_maxsim_amd.build import HIP_FLAGS, _hipcc

    include = Path(__file__).resolve().parents[1] / "include"
    out = out_dir / (src.stem + ".s")
    flags = [f for f in HIP_FLAGS if f not in ("-fPIC", "-Wall")]
    cmd = [_hipcc(), *flags, f"-I{include}", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{res.stderr}")
    return out


def check_sources(sources: list[Path] | None = None) -> list[Finding]:
    from flash_maxsim_amd.build import CSRC

    sources = sources or sorted(CSRC.glob("*.hip"))
    with tempfile.TemporaryDirectory() as tmp:
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(sources)) as pool:
            outs = list(pool.map(lambda s: device_asm(s, Path(tmp)), sources))
        findings: list[Finding] = []
        for o in outs:
            findings += check_asm(o.read_text())
    return findings


if __name__ == "__main__":
    res = check_sources()
    for f in res:
        print(f"{f.kernel}\n  {f.mfma_line}: {f.mfma}\n  {f.line} (+{f.wait_states}, {f.kind}): {f.instr}")
    print(f"{len(res)} finding(s)")
    sys.exit(1 if res else 0)
