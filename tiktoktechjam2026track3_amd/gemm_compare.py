"""The wide GEMM against torch.nn.functional.linear (hipBLASLt) on one product
shape, as rocprofv3 sees them: per-dispatch time, shader cycles and clock,
MFMA and memory-instruction counts, and the stalls of the load path.

``run M N K`` computes bias-only products y = x W^T + b three ways, checks that
they are bitwise equal, then issues ``REPS`` products of each back to back:
F.linear (the reference's nn.Linear), the library's wide GEMM on the
tile-packed weight, and on the plain weight.  Warm-up calls come first (the
plugin measures torch's reduction order for the shape with products of its
own), so the last ``REPS`` dispatches of each kernel family are the timed
ones.  Run it under rocprofv3, one counter set per run:

    rocprofv3 --kernel-trace --output-format csv -d OUT/trace -o run -- \\
        python3 -m tiktoktechjam2026track3_amd.gemm_compare run 32768 1024 4096
    rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VMEM_RD \\
        SQ_INSTS_LDS SQ_VMEM_TA_ADDR_FIFO_FULL --output-format csv -d OUT/p1 -o run -- python3 -m ...
    rocprofv3 --pmc TCP_TCC_READ_REQ_sum TA_ADDR_STALLED_BY_TC_CYCLES_sum \\
        TA_BUFFER_READ_LDS_WAVEFRONTS_sum --output-format csv -d OUT/p2 -o run -- python3 -m ...
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/p3 -o run -- python3 -m ...

``summarize OUT/trace OUT/p1 OUT/p2 OUT/p3 --out FILE`` then writes the
markdown table.  Like the rest of the rocprofv3 tooling, ``summarize`` only
reads profiler output.
"""

from __future__ import annotations

import argparse
import sys
from typing import Dict, List, Optional, Sequence

from .profiling import Dispatch, read_dispatches

REPS = 3
SIMDS = 1024  # MI355X: 256 CUs x 4 SIMDs
XCDS = 8

# (column title, substring of the kernel name)
FAMILIES = (
    ("hipBLASLt (F.linear)", "Cijk_"),
    ("packed W, 256x256x32, 4 stages", "gemm_big_kernel<256, 256, 32, 4, 0,"),
    ("plain W, 256x256x64, 2 stages", "gemm_big_kernel<256, 256, 64, 2, 0,"),
)

# (row title, counter) in table order
COUNTER_ROWS = (
    ("SQ_INSTS_MFMA", "SQ_INSTS_MFMA"),
    ("SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_RD"),
    ("SQ_INSTS_LDS", "SQ_INSTS_LDS"),
    ("TA_BUFFER_READ_LDS_WAVEFRONTS (direct-to-LDS loads)", "TA_BUFFER_READ_LDS_WAVEFRONTS_sum"),
    ("TCP_TCC_READ_REQ (L1 to L2 requests)", "TCP_TCC_READ_REQ_sum"),
    ("TA_ADDR_STALLED_BY_TC_CYCLES", "TA_ADDR_STALLED_BY_TC_CYCLES_sum"),
    ("SQ_VMEM_TA_ADDR_FIFO_FULL", "SQ_VMEM_TA_ADDR_FIFO_FULL"),
    ("FETCH_SIZE (KiB, uncalibrated)", "FETCH_SIZE"),
)


def run(m: int, n: int, k: int) -> int:
    import torch
    import torch.nn.functional as F

    from . import native

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(m + n + k)
    a = torch.randn(m, k, generator=g, device=dev).bfloat16()
    w = ((torch.rand(n, k, generator=g, device=dev) * 2 - 1) / k**0.5).bfloat16()
    b = ((torch.rand(n, generator=g, device=dev) * 2 - 1) / 32).bfloat16()
    wp = native.prepack_weight(w)
    plain = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    packed = torch.empty_like(plain)
    native.linear(a, w, b, native.ENC_EPI_BIAS, out=plain)
    native.linear(a, w, b, native.ENC_EPI_BIAS, out=packed, packed_weight=wp)
    ref = F.linear(a, w, b)
    torch.cuda.synchronize()
    if not (torch.equal(ref, plain) and torch.equal(ref, packed)):
        print("the products differ from F.linear", file=sys.stderr)
        return 1
    for _ in range(REPS):
        F.linear(a, w, b)
    for _ in range(REPS):
        native.linear(a, w, b, native.ENC_EPI_BIAS, out=packed, packed_weight=wp)
    for _ in range(REPS):
        native.linear(a, w, b, native.ENC_EPI_BIAS, out=plain)
    torch.cuda.synchronize()
    print(f"done {m}x{n}x{k}: {REPS} products each, bitwise equal", flush=True)
    return 0


def _family(dispatches: Sequence[Dispatch], pattern: str) -> List[Dispatch]:
    return [d for d in dispatches if pattern in d.name][-REPS:]


def summarize(dirs: Sequence[str]) -> str:
    """Markdown table over the families, from one kernel-trace directory and
    any number of counter directories."""
    durations: Dict[str, float] = {}
    counters: Dict[str, Dict[str, float]] = {title: {} for title, _ in FAMILIES}
    for directory in dirs:
        dispatches = read_dispatches(directory)
        for title, pattern in FAMILIES:
            picked = _family(dispatches, pattern)
            if not picked:
                continue
            if picked[0].counters is None:
                durations[title] = sum(d.duration_ns for d in picked) / len(picked)
            else:
                for name in picked[0].counters:
                    counters[title][name] = sum(d.counters.get(name, 0.0) for d in picked) / len(picked)
    titles = [title for title, _ in FAMILIES]
    lines = ["| per dispatch | " + " | ".join(titles) + " |", "|---|" + "---:|" * len(titles)]

    def row(label: str, values: List[Optional[float]], fmt: str) -> None:
        cells = ["—" if v is None else format(v, fmt) for v in values]
        lines.append(f"| {label} | " + " | ".join(cells) + " |")

    row("time (µs, kernel trace)", [durations[t] / 1e3 if t in durations else None for t in titles], ".1f")
    cycles = [counters[t].get("GRBM_GUI_ACTIVE") for t in titles]
    row("shader cycles (GRBM_GUI_ACTIVE / 8 XCDs)", [c / XCDS if c is not None else None for c in cycles], ".4g")
    clocks: List[Optional[float]] = []
    for t, c in zip(titles, cycles):
        clocks.append(c / XCDS / durations[t] if c is not None and t in durations else None)
    row("shader clock (GHz, cycles over the trace time)", clocks, ".2f")
    busy = []
    for t, c in zip(titles, cycles):
        mfma = counters[t].get("SQ_VALU_MFMA_BUSY_CYCLES")
        busy.append(100.0 * mfma / (SIMDS * c / XCDS) if mfma is not None and c else None)
    row("MFMA busy (%)", busy, ".1f")
    for label, name in COUNTER_ROWS:
        row(label, [counters[t].get(name) for t in titles], ".4g")
    return "\n".join(lines) + "\n"


def main(argv: Optional[Sequence[str]] = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = parser.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("m", type=int)
    r.add_argument("n", type=int)
    r.add_argument("k", type=int)
    s = sub.add_parser("summarize")
    s.add_argument("dirs", nargs="+")
    s.add_argument("--out", required=True)
    s.add_argument("--title", default="Wide GEMM against hipBLASLt")
    s.add_argument("--command", action="append", default=[])
    args = parser.parse_args(argv)
    if args.cmd == "run":
        return run(args.m, args.n, args.k)
    text = f"# {args.title}\n\n"
    if args.command:
        text += ("Produced by (from the repository root on one MI355X, `cd /tmp && export TMPDIR=/tmp` "
                 "first):\n\n" + "".join(f"    {c}\n" for c in args.command) + "\n")
    text += (f"Each value is the mean over the last {REPS} dispatches of the family; counter runs "
             "serialise the dispatches, so each ran alone on the device.\n\n" + summarize(args.dirs))
    with open(args.out, "w") as fh:
        fh.write(text)
    print(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
