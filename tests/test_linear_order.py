"""The stream-K order measurement (linear_order.py), pinned on the CPU.

The GPU measures which output tiles hipBLASLt accumulates in two partial sums
by reading which outputs of a probe product survive.  These tests check the
principle and the reader without a GPU:

  * the rounding rule the probe rests on, with real fp32 accumulation in both
    orders (one pass, and P1 + P2 split at s): the 2^-4 term survives exactly
    when its block lies at or after s;
  * the table reader on survivor patterns produced by that arithmetic for
    random split tables, including the stream-K structure measured on the
    MI355X (two-tile tails, 16-row groups, per-workgroup K ranges);
  * planted mistakes: tiles narrower or shorter than 256, a second split
    point, are rejected rather than misread.
"""

import math
import random

import numpy as np
import pytest
import torch

from tiktoktechjam2026track3_amd import linear_order as lo

BIG = np.float32(2.0 ** 20)
SMALL = np.float32(2.0 ** -4)


def probe_output(k: int, split: int, block: int) -> np.float32:
    """Output of one probe element, A = 1: K blocks of 32 in sequence, the
    tile's partial sums split at ``split`` (0: one pass), added in fp32."""
    terms = np.zeros(k, dtype=np.float32)
    terms[0] = BIG
    terms[k - 32] = -BIG
    terms[32 * block] = SMALL

    def seq(lo_k, hi_k):
        acc = np.float32(0)
        for t in terms[lo_k:hi_k]:
            acc = np.float32(acc + t)
        return acc

    if split == 0:
        return seq(0, k)
    return np.float32(seq(0, split) + seq(split, k))


@pytest.mark.parametrize("k", [96, 256, 1024])
def test_probe_survives_exactly_when_its_block_is_in_the_second_partial(k):
    nb = k // 32
    for split in [0] + list(range(32, k, 32)):
        for block in range(1, nb - 1):
            survived = probe_output(k, split, block) != 0
            assert survived == (split > 0 and 32 * block >= split), (k, split, block)


def survivors_for(table, tile_rows, n, k, phase, rows_in_last=256):
    """Survivor pattern [rows, n] that probes of a 256 x 256 split table give."""
    period = k // 32 - 2
    blocks = 1 + (np.arange(n) + phase) % period
    rows = (tile_rows - 1) * 256 + rows_in_last
    out = np.zeros((rows, n), dtype=bool)
    for tr in range(tile_rows):
        for tc in range(n // 256):
            s = table[tr * (n // 256) + tc]
            if s:
                out[tr * 256:(tr + 1) * 256, tc * 256:(tc + 1) * 256] = (32 * blocks[tc * 256:(tc + 1) * 256] >= s)
    return torch.from_numpy(out), torch.from_numpy(blocks)


def test_rule_table_matches_fp32_arithmetic_per_element():
    # the vectorised pattern above is the fp32 arithmetic's, element by element
    k = 256
    rng = random.Random(3)
    table = [rng.choice([0, 64, 128, 192]) for _ in range(4)]
    surv, blocks = survivors_for(table, 1, 1024, k, 0)
    for n in range(0, 1024, 7):
        got = probe_output(k, table[n // 256], int(blocks[n])) != 0
        assert got == bool(surv[0, n])


def stream_k_table(m, n, k, g, du=64, wgm=16):
    """Split table (from the first split tile row) of a two-tile, data-parallel
    first stream-K schedule: the structure measured on the MI355X."""
    tm, tn = math.ceil(m / 256), n // 256
    tiles, ipt = tm * tn, k // du
    order = []
    for g0 in range(0, tm, wgm):
        for c in range(tn):
            for r in range(min(wgm, tm - g0)):
                order.append((g0 + r, c))
    if tiles % g == 0:
        return None
    sk = g + tiles % g
    per, extra = divmod(sk * ipt, g)
    splits = {}
    for w in range(1, g):
        t, off = divmod(w * per + min(w, extra), ipt)
        if off:
            splits[order[tiles - sk + t]] = off * du
    if not splits:
        return None
    first = min(r for r, _ in splits)
    rows = tm - first
    return first, rows, [splits.get((first + r, c), 0) for r in range(rows) for c in range(tn)]


@pytest.mark.parametrize("m,n,k,g", [(100000, 1024, 1024, 256), (3200000, 1024, 1024, 255),
                                     (400000, 1024, 1024, 250), (100000, 4096, 1024, 250),
                                     (100000, 1024, 4096, 256)])
def test_reader_recovers_stream_k_tables(m, n, k, g):
    first, rows, table = stream_k_table(m, n, k, g)
    last = m - (m - 1) // 256 * 256
    for phase in (0, (k // 32 - 2) // 2):
        surv, blocks = survivors_for(table, rows, n, k, phase, rows_in_last=last)
        assert lo._table_from(surv, blocks, m, n) == (rows, table)


def test_builtin_tables_follow_the_stream_k_structure():
    # the two tables measured on the MI355X and committed in csrc/streamk_tail.h
    import re
    from pathlib import Path

    text = (Path(lo.__file__).parent / "csrc" / "streamk_tail.h").read_text()
    tables = {int(mm.group(1)): [int(v) for v in mm.group(2).replace("\n", " ").split(",") if v.strip()]
              for mm in re.finditer(r"kTailSplit_(\d+)_1024_1024\[\d+\] = \{([^}]*)\}", text)}
    entries = {int(mm.group(1)): (int(mm.group(2)), int(mm.group(3)))
               for mm in re.finditer(r"\{(\d+), 1024, 1024, (\d+), (\d+), 4, kTailSplit", text)}
    for m, g in ((100000, 256), (3200000, 255)):
        first, rows, table = stream_k_table(m, 1024, 1024, g)
        assert entries[m] == (first, rows)
        assert tables[m] == table


def test_reader_rejects_other_tile_shapes():
    n, k = 1024, 1024
    table = [0, 512, 0, 0]
    surv, blocks = survivors_for(table, 1, n, k, 0)
    # a 128-column half tile with another split point
    bad = surv.clone()
    bad[:, 384:512] = torch.from_numpy(32 * blocks[384:512].numpy() >= 256)
    with pytest.raises(lo.UnrepresentableOrderError, match="more than one split"):
        lo._table_from(bad, blocks, 256, n)
    # a 128-row half tile that splits differently
    bad = surv.clone()
    bad[128:, 256:512] = False
    with pytest.raises(lo.UnrepresentableOrderError, match="256-row tile"):
        lo._table_from(bad, blocks, 256, n)


def test_small_and_narrow_shapes_are_not_probed():
    assert lo.measure(256, 1024, 1024, torch.device("cpu")).kind == "unprobed"
    assert lo.measure(4096, 1024, 64, torch.device("cpu")).kind == "unprobed"
