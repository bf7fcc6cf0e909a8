"""Build-time check of the MFMA result hazard in the gfx950 code built here.

An MFMA writes its destination registers many cycles after it issues, and the
hardware does not interlock every later read of them: the instruction stream
must leave enough wait states (independent instructions, or ``s_nop``) between
the MFMA and the first instruction that reads its result.  The compiler
inserts them, but a branch between the MFMA and the read once let a read on
the branch-taken path follow after two instructions (a nondeterministic wrong
result in the last result register of the fused block tail's products).  This
module disassembles the
device code of every object the build produced and walks each MFMA's
successors along every control-flow path, counting wait states, and reports
each read of the MFMA's destination that comes too early.

Counting rules: every instruction is one wait state, ``s_nop n`` is n + 1; a
path ends at ``s_endpgm``, at a write of every destination register, or once
the count reaches the requirement.  A following MFMA that accumulates into
exactly the same registers (its C operand) is the supported back-to-back
chain and is not a read; a read through its A/B operands is.  The requirement
(``REQUIRED_WAIT_STATES``) is the smallest distance the compiler leaves on
straight-line code in these kernels, so the check catches paths that lose
wait states, not the compiler's own choice.

The same walk over the disassembly also lists every packed FP32 VALU
instruction (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32).  Every device compile
disables them (-packed-fp32-ops); hipcc's host pass warns that it does not know
the feature and the build filters that line, so this check is what shows the
device pass honoured it.

Only code compiled in this repository is read (the AMD assembly of our own
objects, extracted with the ROCm LLVM tools).
"""

from __future__ import annotations

import re
import subprocess
import tempfile
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Set, Tuple

LLVM_BIN = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
REQUIRED_WAIT_STATES = 8
_SEARCH_LIMIT = 64  # wait states after which no path is followed further

_LINE = re.compile(r"^\s+(?P<text>[a-z_0-9]+[^/]*?)\s*//\s*(?P<addr>[0-9A-Fa-f]+):(?P<rest>.*)$")
_FUNC = re.compile(r"^(?P<addr>[0-9a-f]+) <(?P<name>[^>]+)>:$")
_TARGET = re.compile(r"<(?P<name>[^>+]+)\+0x(?P<off>[0-9a-f]+)>")
_REG_RANGE = re.compile(r"\b([va])\[(\d+):(\d+)\]")
_REG_ONE = re.compile(r"\b([va])(\d+)\b")
_STORE_PREFIXES = ("global_store", "buffer_store", "ds_write", "ds_store", "flat_store", "scratch_store",
                   "global_load_lds", "buffer_load_lds", "global_atomic", "buffer_atomic", "ds_add", "ds_max",
                   "ds_min")


@dataclass
class Insn:
    addr: int
    mnemonic: str
    operands: List[str]
    text: str
    target: Optional[int] = None  # branch target address


@dataclass
class Finding:
    function: str
    mfma: str
    mfma_addr: int
    read: str
    read_addr: int
    wait_states: int

    def __str__(self) -> str:
        return (f"{self.function}: '{self.read}' at 0x{self.read_addr:x} reads the result of "
                f"'{self.mfma}' at 0x{self.mfma_addr:x} after {self.wait_states} wait states "
                f"(needs {REQUIRED_WAIT_STATES})")


@dataclass
class Report:
    functions: int = 0
    mfmas: int = 0
    findings: List[Finding] = field(default_factory=list)
    min_straight_line: Optional[int] = None  # smallest distance seen on any path
    packed_fp32: List[str] = field(default_factory=list)  # "function: instruction"


def _regs(operand: str) -> Set[Tuple[str, int]]:
    out: Set[Tuple[str, int]] = set()
    for kind, lo, hi in _REG_RANGE.findall(operand):
        out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    stripped = _REG_RANGE.sub(" ", operand)
    for kind, r in _REG_ONE.findall(stripped):
        out.add((kind, int(r)))
    return out


def _split_operands(text: str) -> Tuple[str, List[str]]:
    parts = text.strip().split(None, 1)
    mnemonic = parts[0]
    if len(parts) == 1:
        return mnemonic, []
    return mnemonic, [p.strip() for p in parts[1].split(",")]


def _defs_uses(insn: Insn) -> Tuple[Set[Tuple[str, int]], Set[Tuple[str, int]]]:
    m = insn.mnemonic
    if m.startswith("s_"):
        return set(), set()
    if not insn.operands:
        return set(), set()
    if m.startswith(_STORE_PREFIXES):
        uses: Set[Tuple[str, int]] = set()
        for op in insn.operands:
            uses |= _regs(op)
        return set(), uses
    defs = _regs(insn.operands[0])
    uses = set()
    for op in insn.operands[1:]:
        uses |= _regs(op)
    return defs, uses


def parse_disassembly(text: str) -> Dict[str, List[Insn]]:
    functions: Dict[str, List[Insn]] = {}
    current: Optional[List[Insn]] = None
    starts: Dict[str, int] = {}
    pending: List[Tuple[Insn, str, int]] = []
    for line in text.splitlines():
        fm = _FUNC.match(line)
        if fm:
            current = functions.setdefault(fm.group("name"), [])
            starts[fm.group("name")] = int(fm.group("addr"), 16)
            continue
        lm = _LINE.match(line)
        if not lm or current is None:
            continue
        mnemonic, operands = _split_operands(lm.group("text"))
        insn = Insn(int(lm.group("addr"), 16), mnemonic, operands, lm.group("text").strip())
        tm = _TARGET.search(lm.group("rest"))
        if tm and (mnemonic.startswith("s_cbranch") or mnemonic == "s_branch"):
            pending.append((insn, tm.group("name"), int(tm.group("off"), 16)))
        current.append(insn)
    for insn, name, off in pending:
        if name in starts:
            insn.target = starts[name] + off
    return functions


def _wait_states(insn: Insn) -> int:
    if insn.mnemonic == "s_nop" and insn.operands:
        try:
            return int(insn.operands[0], 0) + 1
        except ValueError:
            return 1
    return 1


def check_function(name: str, insns: List[Insn], report: Report) -> None:
    index = {insn.addr: i for i, insn in enumerate(insns)}
    for i, insn in enumerate(insns):
        if not insn.mnemonic.startswith("v_mfma"):
            continue
        report.mfmas += 1
        dst = _regs(insn.operands[0])
        # (position, wait states so far, destination registers still holding the result)
        stack = [(i + 1, 0, frozenset(dst))]
        seen: Dict[Tuple[int, frozenset], int] = {}
        while stack:
            pos, waits, live = stack.pop()
            while 0 <= pos < len(insns) and waits < _SEARCH_LIMIT and live:
                key = (pos, live)
                if seen.get(key, _SEARCH_LIMIT + 1) <= waits:
                    break
                seen[key] = waits
                cur = insns[pos]
                defs, uses = _defs_uses(cur)
                if cur.mnemonic.startswith("v_mfma") and len(cur.operands) >= 4:
                    # back-to-back accumulation into the same registers is supported
                    c_regs = _regs(cur.operands[3])
                    ab_regs = _regs(cur.operands[1]) | _regs(cur.operands[2])
                    chained = c_regs == set(live) or c_regs == dst
                    uses = ab_regs if chained else (ab_regs | c_regs)
                hit = uses & live
                if hit:
                    if report.min_straight_line is None or waits < report.min_straight_line:
                        report.min_straight_line = waits
                    if waits < REQUIRED_WAIT_STATES:
                        report.findings.append(Finding(name, insn.text, insn.addr, cur.text, cur.addr, waits))
                    live = live - hit  # each register's first read is the one that counts
                live = live - defs
                if cur.mnemonic == "s_endpgm" or cur.mnemonic.startswith("s_setpc"):
                    break
                if cur.target is not None and cur.target in index:
                    stack.append((index[cur.target], waits + _wait_states(cur), live))
                    if cur.mnemonic == "s_branch":
                        break
                waits += _wait_states(cur)
                pos += 1


def disassemble_object(obj: Path, workdir: Path) -> str:
    """AMD assembly of the gfx950 code object embedded in a hipcc object file."""
    objcopy = LLVM_BIN / "llvm-objcopy"
    bundler = LLVM_BIN / "clang-offload-bundler"
    objdump = LLVM_BIN / "llvm-objdump"
    fatbin = workdir / (obj.stem + ".fatbin")
    code = workdir / (obj.stem + ".co")
    subprocess.run([str(objcopy), f"--dump-section=.hip_fatbin={fatbin}", str(obj), str(workdir / "scratch.o")],
                   check=True, capture_output=True)
    subprocess.run([str(bundler), "--unbundle", "--type=o", f"--targets={TARGET}", f"--input={fatbin}",
                    f"--output={code}"], check=True, capture_output=True)
    out = subprocess.run([str(objdump), "-d", "--mcpu=gfx950", str(code)], check=True, capture_output=True,
                         text=True)
    return out.stdout


def tools_available() -> bool:
    return all((LLVM_BIN / t).exists() for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


_PACKED_FP32 = ("v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32")


def check_text(text: str) -> Report:
    report = Report()
    for name, insns in parse_disassembly(text).items():
        report.functions += 1
        check_function(name, insns, report)
        report.packed_fp32 += [f"{name}: {i.text}" for i in insns if i.mnemonic.startswith(_PACKED_FP32)]
    return report


def _check_one(obj: str) -> Report:
    with tempfile.TemporaryDirectory() as tmp:
        return check_text(disassemble_object(Path(obj), Path(tmp)))


def check_objects(objects: Iterable[Path], jobs: int = 8) -> Report:
    """Disassemble and check every object (in parallel processes)."""
    from concurrent.futures import ProcessPoolExecutor

    paths = [str(p) for p in objects]
    total = Report()
    with ProcessPoolExecutor(max_workers=max(1, min(jobs, len(paths)))) as pool:
        for part in pool.map(_check_one, paths):
            total.functions += part.functions
            total.mfmas += part.mfmas
            total.findings += part.findings
            total.packed_fp32 += part.packed_fp32
            if part.min_straight_line is not None and (
                total.min_straight_line is None or part.min_straight_line < total.min_straight_line
            ):
                total.min_straight_line = part.min_straight_line
    return total


if __name__ == "__main__":
    import sys

    rep = check_objects(Path(p) for p in sys.argv[1:])
    print(f"{rep.functions} functions, {rep.mfmas} MFMAs, smallest MFMA-to-read distance "
          f"{rep.min_straight_line}, {len(rep.findings)} finding(s), "
          f"{len(rep.packed_fp32)} packed FP32 instruction(s)")
    for f in rep.findings[:20]:
        print(f)
    for f in rep.packed_fp32[:20]:
        print(f)
    sys.exit(1 if rep.findings or rep.packed_fp32 else 0)
