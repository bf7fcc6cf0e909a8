"""The reduction order of the reference's nn.Linear, measured per product shape.

Every projection of the reference is an ``nn.Linear`` (transformer_benchmark/
models.py:30-33, 724-725), which on ROCm is a hipBLASLt product.  For bf16
products with more than a few hundred rows hipBLASLt runs "stream-K" kernels:
a persistent grid of g workgroups takes the output tiles in rounds, and the
last g + (tiles mod g) tiles are dealt out by K iterations, so a tile whose
iterations straddle two workgroups is accumulated as two partial sums that
are then added, ``bf16((P1 + P2) + bias)`` with P1 over K < s and P2 over
K >= s.  The native GEMM reproduces that order (gemm_tail_split_kernel) when
it knows which tiles split and where.  That depends on the tile shape and the
grid the library picks for each shape (an internal cost model: 28 672 rows
of [*, 1024] x [1024, 1024] run on 224 workgroups, 3.2 M rows on 255, 1 M
rows on 256), so it is measured here, once per (device, M, N, K), from two
probe products through ``torch.nn.functional.linear`` itself, and handed to
the library (``enc_linear_order_register``).  The probes' outputs are never
used as results: they only reveal the order.

Probe: A is all ones; weight row n holds +2^20 in the first 32-wide K block,
-2^20 in the last, and 2^-4 in one block b(n) in between.  Summed in one pass
the 2^-4 is rounded away next to 2^20 (half an fp32 ulp, ties to even); it
survives only when block b(n) lies in a partial sum that starts after the
+2^20 and ends with the -2^20, i.e. when the tile is split at s <= 32 b(n).
So an output is nonzero exactly when its tile splits at or before its
column's block.  Every 256-column tile holds every block value (b(n) cycles
with period K/32 - 2 <= 254), so the smallest surviving block of a tile is its
split.  The measurement is accepted only if the whole survivor pattern is what
a table of 256 x 256 tiles predicts, in both probes (the second shifts b(n) by
half a period), which rules out tiles of other shapes; otherwise the shape is
reported as one the native GEMM cannot reproduce.

Shapes with at most 256 rows are not measured: there the library splits K
across workgroups in other ways, which ``gemm_split_plan`` (csrc/gemm.hip)
reproduces for the shapes it lists.  Neither are products with K < 96 (no
middle block for the probe); those accumulate K sequentially in every case
that the test suite checks.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

BLOCK = 32      # K granularity of the probe (the native tail kernel splits at 32-deep K blocks)
TILE = 256      # edge of the library's tail tiles that the native GEMM reproduces
MAX_ENTRIES = 1024  # table entries the library takes (enc_linear_order_register)
MIN_ROWS = 257  # below this the split-K rules of gemm_split_plan apply
ROW_CHUNK = 65536


class UnrepresentableOrderError(RuntimeError):
    """hipBLASLt reduces this product in an order the native GEMM does not reproduce."""


@dataclass
class LinearOrder:
    """How the reference's nn.Linear accumulates one [M, K] x [N, K]^T shape."""

    m: int
    n: int
    k: int
    kind: str  # "sequential", "tail", "unprobed" or "unrepresentable"
    first_tile_row: int = 0
    tile_rows: int = 0
    tile_cols: int = 0
    split: List[int] = field(default_factory=list)
    reason: str = ""

    @property
    def representable(self) -> bool:
        return self.kind != "unrepresentable"

    def split_tiles(self) -> int:
        return sum(1 for s in self.split if s)


_lock = threading.Lock()
_orders: Dict[Tuple[int, int, int, int], LinearOrder] = {}


def _probe(a: torch.Tensor, m: int, n: int, k: int, phase: int) -> Tuple[int, Optional[torch.Tensor], torch.Tensor]:
    """One probe: (first tile row with a surviving output, the survivor
    pattern of the rows from there to M as bool on the host, or None when no
    output survived; the block of each column)."""
    import torch.nn.functional as F

    device = a.device
    nb = k // BLOCK
    period = nb - 2
    cols = torch.arange(n, device=device)
    blocks = 1 + (cols + phase) % period
    w = torch.zeros(n, k, device=device, dtype=torch.float32)
    w[:, 0] = 2.0 ** 20
    w[:, k - BLOCK] = -(2.0 ** 20)
    w[cols, BLOCK * blocks] = 2.0 ** -4
    w = w.bfloat16()
    bias = torch.zeros(n, device=device, dtype=torch.bfloat16)
    out = F.linear(a, w, bias)
    del w
    first = None
    for r in range(0, m, ROW_CHUNK):
        idx = torch.nonzero((out[r:r + ROW_CHUNK] != 0).any(dim=1))
        if idx.numel():
            first = r + int(idx[0])
            break
    if first is None:
        return 0, None, blocks.cpu()
    first_tile_row = first // TILE
    tail_tiles = (m - first_tile_row * TILE + TILE - 1) // TILE * max(1, n // TILE)
    if tail_tiles > MAX_ENTRIES:
        raise UnrepresentableOrderError(f"split tiles spread over {tail_tiles} tiles, past the table limit")
    survivors = (out[first_tile_row * TILE:] != 0).cpu()
    del out
    return first_tile_row, survivors, blocks.cpu()


def _table_from(survivors: torch.Tensor, blocks: torch.Tensor, m: int, n: int) -> Tuple[int, List[int]]:
    """(tile_rows, split table) read off one probe's survivors, or raise
    UnrepresentableOrderError when no 256 x 256 table explains them."""
    rows = survivors.shape[0]
    tile_rows = (rows + TILE - 1) // TILE
    tile_cols = n // TILE
    split: List[int] = []
    for tr in range(tile_rows):
        band = survivors[tr * TILE: min(rows, (tr + 1) * TILE)]
        rep = band[0]
        if not bool((band == rep).all()):
            raise UnrepresentableOrderError("rows of one 256-row tile are split differently")
        for tc in range(tile_cols):
            got = rep[tc * TILE:(tc + 1) * TILE]
            b = blocks[tc * TILE:(tc + 1) * TILE]
            if not bool(got.any()):
                split.append(0)
                continue
            threshold = int(b[got].min())
            if not torch.equal(got, b >= threshold):
                raise UnrepresentableOrderError("a 256-column tile holds more than one split point")
            split.append(BLOCK * threshold)
    return tile_rows, split


def measure(m: int, n: int, k: int, device: torch.device) -> LinearOrder:
    """Probe torch.nn.functional.linear for one bf16 shape on ``device``."""
    if m < MIN_ROWS or k < 3 * BLOCK or k % BLOCK:
        return LinearOrder(m, n, k, "unprobed")
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"the reduction order of [{m}, {k}] x [{n}, {k}]^T is not known yet and cannot be measured "
            "during graph capture; run the product once eagerly (or call linear_order.ensure) first")
    a = torch.ones(m, k, device=device, dtype=torch.bfloat16)
    period = k // BLOCK - 2
    tables = []
    try:
        for phase in (0, period // 2):
            first_tile_row, survivors, blocks = _probe(a, m, n, k, phase)
            if survivors is None:
                tables.append(None)
                continue
            if n % TILE:
                raise UnrepresentableOrderError(f"split tiles in a product with N = {n}, not a multiple of 256")
            if period > TILE:
                raise UnrepresentableOrderError(f"split tiles with K = {k}: a 256-column tile cannot show every block")
            tables.append((first_tile_row,) + _table_from(survivors, blocks, m, n))
    except UnrepresentableOrderError as error:
        return LinearOrder(m, n, k, "unrepresentable", reason=str(error))
    finally:
        del a
    if tables[0] is None and tables[1] is None:
        return LinearOrder(m, n, k, "sequential")
    if tables[0] is None or tables[1] is None or tables[0] != tables[1]:
        return LinearOrder(m, n, k, "unrepresentable", reason="the two probes read different split points")
    first_tile_row, tile_rows, split = tables[0]
    return LinearOrder(m, n, k, "tail", first_tile_row=first_tile_row, tile_rows=tile_rows,
                       tile_cols=n // TILE, split=split)


def register(order: LinearOrder, device: torch.device) -> None:
    """Hand a measured order to the native library for ``device``."""
    import ctypes

    from . import native

    lib = native.load_library()
    index = device.index if device.index is not None else torch.cuda.current_device()
    if order.kind == "tail":
        table = (ctypes.c_uint16 * len(order.split))(*order.split)
        status = lib.enc_linear_order_register(index, order.m, order.n, order.k, order.first_tile_row,
                                               order.tile_rows, order.tile_cols, ctypes.cast(table, ctypes.c_void_p))
    elif order.kind == "sequential":
        status = lib.enc_linear_order_register(index, order.m, order.n, order.k, 0, 0, 0, None)
    else:
        return
    native._check("enc_linear_order_register", status)


def ensure(m: int, n: int, k: int, device: torch.device) -> LinearOrder:
    """The order of [m, k] x [n, k]^T on ``device``: measured and registered on
    first use, cached for the process."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, m, n, k)
    order = _orders.get(key)
    if order is not None:
        return order
    with _lock:
        order = _orders.get(key)
        if order is None:
            with torch.cuda.device(index):
                order = measure(m, n, k, torch.device("cuda", index))
                register(order, torch.device("cuda", index))
            _orders[key] = order
    return order


def ensure_encoder(tokens: int, d_model: int, ffn_dim: int, device: torch.device) -> List[LinearOrder]:
    """Orders of the encoder's three product shapes: q/k/v/out_proj
    [T, D] x [D, D]^T, ffn_in [T, D] x [F, D]^T and ffn_out [T, F] x [D, F]^T."""
    shapes = {(tokens, d_model, d_model), (tokens, ffn_dim, d_model), (tokens, d_model, ffn_dim)}
    return [ensure(m, n, k, device) for m, n, k in sorted(shapes)]


def known_encoder_orders(tokens: int, d_model: int, ffn_dim: int, device: torch.device) -> List[LinearOrder]:
    """The encoder's three orders without measuring anything (for callers that
    must not allocate); raises if one that needs a measurement is missing."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    result = []
    for m, n, k in sorted({(tokens, d_model, d_model), (tokens, ffn_dim, d_model), (tokens, d_model, ffn_dim)}):
        order = _orders.get((index, m, n, k))
        if order is None:
            if m >= MIN_ROWS and k >= 3 * BLOCK and k % BLOCK == 0:
                raise RuntimeError(
                    f"the reduction order of [{m}, {k}] x [{n}, {k}]^T has not been measured on cuda:{index}; "
                    "call linear_order.ensure_encoder (which allocates) before the no-allocation forward")
            order = LinearOrder(m, n, k, "unprobed")
        result.append(order)
    return result


def require(order: LinearOrder) -> None:
    if not order.representable:
        raise UnrepresentableOrderError(
            f"torch.nn.functional.linear reduces [{order.m}, {order.k}] x [{order.n}, {order.k}]^T in an order "
            f"the native GEMM does not reproduce: {order.reason}")


def known_orders() -> Dict[Tuple[int, int, int, int], LinearOrder]:
    return dict(_orders)


def forget() -> None:
    """Drop every measured order, here and in the library."""
    from . import native

    with _lock:
        _orders.clear()
        if native.library_loaded():
            native._check("enc_linear_order_clear", native.load_library().enc_linear_order_clear())
