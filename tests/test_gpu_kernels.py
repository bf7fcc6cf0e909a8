"""Kernel-level parity of libmi355x_encoder.so on the GPU.

Each HIP kernel is called through the C ABI (via the ctypes binding) and checked
against a plain PyTorch fp32 computation of the same op with the reference's
bf16 rounding points, or against the oracle's attention restatement.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.encoder_oracle import attention_rows
from tiktoktechjam2026track3_amd import native

pytestmark = pytest.mark.gpu

RTOL = 1.6e-2  # the build's bf16 gate
ATOL = 1e-2


def within_ulps(ref: torch.Tensor, out: torch.Tensor, ulps: float = 1.0) -> bool:
    """|out - ref| <= ulps * bf16 spacing at |ref|, plus a floor of 2^-12 of the
    tensor's rms for values near zero, where fp32 accumulation order alone moves
    a cancelled result by many of its own (tiny) ulps."""
    ref = ref.float()
    out = out.float()
    _, exponent = torch.frexp(ref)
    spacing = torch.ldexp(torch.ones_like(ref), exponent - 8)  # bf16: 8 significant bits
    floor = 2.0**-12 * ref.pow(2).mean().sqrt()
    return bool(((out - ref).abs() <= ulps * spacing + floor).all())


def within_composite(ref: torch.Tensor, out: torch.Tensor, inner: torch.Tensor, slope: float) -> bool:
    """For out = f(bf16(y)) with f of |slope| <= slope: a one-ulp difference of
    the bf16 linear output y (fp32 accumulation order) moves out by at most
    slope * spacing(y), on top of out's own rounding."""
    ref, out, inner = ref.float(), out.float(), inner.float()
    _, e_out = torch.frexp(ref)
    _, e_in = torch.frexp(inner)
    tol = torch.ldexp(torch.ones_like(ref), e_out - 8) + slope * torch.ldexp(torch.ones_like(inner), e_in - 8)
    floor = 2.0**-12 * ref.pow(2).mean().sqrt()
    return bool(((out - ref).abs() <= tol + floor).all())


def bitwise_fraction(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.contiguous().view(torch.int16) == b.contiguous().view(torch.int16)).float().mean())


def strict_gate(ref: torch.Tensor, out: torch.Tensor, rtol=RTOL, atol=ATOL) -> int:
    ref = ref.float()
    out = out.float()
    err = (out - ref).abs()
    ok = torch.isfinite(ref) & torch.isfinite(out) & ((err < atol) | (err < rtol * ref.abs()))
    return int((~ok).sum().item())


@pytest.fixture(autouse=True)
def _no_tf32():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev


def test_library_loads_and_reports_version():
    lib = native.load_library()
    assert lib.enc_version() >> 16 == 1


@pytest.mark.parametrize("width", [32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("rows", [1, 7, 4099])
def test_layernorm_matches_torch(device, rows, width):
    g = torch.Generator(device=device).manual_seed(rows * 7 + width)
    x = (torch.randn(rows, width, generator=g, device=device) * 3 + 0.5).bfloat16()
    w = (torch.randn(width, generator=g, device=device) * 0.5 + 1).bfloat16()
    b = (torch.randn(width, generator=g, device=device) * 0.1).bfloat16()
    ref = F.layer_norm(x.float(), (width,), w.float(), b.float(), 1e-5).bfloat16()
    out = native.layernorm(x, w, b, 1e-5)
    assert within_ulps(ref, out, 1)
    # torch's own bf16 LayerNorm on the device (the reference's op): the
    # statistics follow its operation order, so the outputs are identical
    torch_bf16 = F.layer_norm(x, (width,), w, b, 1e-5)
    assert torch.equal(torch_bf16, out)


@pytest.mark.parametrize("width", [32, 128, 256, 512, 1024, 4096])
def test_layernorm_merge_order_rows(device, width):
    """Rows holding one large value and two values just under half an ulp of
    it: whether the two small ones survive depends on which partial
    statistics meet first and on the reciprocals used, so every row checks
    the reduction order against torch's."""
    rows = 2048
    g = torch.Generator(device="cpu").manual_seed(width)
    pos = torch.stack([torch.randperm(width, generator=g)[:3] for _ in range(rows)]).to(device)
    x = torch.zeros(rows, width, device=device)
    r = torch.arange(rows, device=device)
    x[r, pos[:, 0]] = 1.0
    x[r, pos[:, 1]] = 1.5 * 2.0**-25
    x[r, pos[:, 2]] = 1.5 * 2.0**-25
    x = x.bfloat16()
    w = torch.ones(width, device=device, dtype=torch.bfloat16)
    b = torch.zeros(width, device=device, dtype=torch.bfloat16)
    ref = F.layer_norm(x, (width,), w, b, 1e-5)
    out = native.layernorm(x, w, b, 1e-5)
    assert torch.equal(ref, out)


@pytest.mark.parametrize("width", [32, 128, 512])
def test_layernorm_row_mask_zeroes_rows(device, width):
    x = torch.randn(67, width, device=device).bfloat16()
    w = torch.ones(width, device=device).bfloat16()
    b = torch.full((width,), 0.25, device=device).bfloat16()
    mask = torch.rand(67, device=device) > 0.5
    out = native.layernorm(x, w, b, 1e-5, row_mask=mask)
    assert torch.all(out[~mask] == 0)
    assert torch.equal(out[mask], F.layer_norm(x, (width,), w, b, 1e-5)[mask])


def _linear_case(device, m, n, k, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    a = torch.randn(m, k, generator=g, device=device).bfloat16()
    w = (torch.rand(n, k, generator=g, device=device) * 2 - 1).mul(1 / math.sqrt(k)).bfloat16()
    bias = (torch.rand(n, generator=g, device=device) * 2 - 1).mul(1 / math.sqrt(k)).bfloat16()
    res = torch.randn(m, n, generator=g, device=device).bfloat16()
    y = F.linear(a.float(), w.float(), bias.float())  # fp32 reference
    return a, w, bias, res, y


SHAPES = [
    (1, 512, 512),
    (100, 1536, 512),
    (128, 2048, 512),
    (128, 512, 2048),
    (1000, 1024, 1024),
    (8192, 3072, 1024),
    (8192, 1024, 4096),
    (4096, 4096, 1024),
]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear_bias(device, m, n, k):
    a, w, bias, _, y = _linear_case(device, m, n, k, m + n + k)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS)
    assert within_ulps(y, out, 1)
    # torch's bf16 nn.Linear (the reference op) accumulates in the same MFMA
    # K order: the outputs agree bit for bit except where it splits K
    assert bitwise_fraction(F.linear(a, w, bias), out) > 0.999


@pytest.mark.parametrize("m,n,k", SHAPES[:6])
def test_linear_gelu(device, m, n, k):
    a, w, bias, _, y = _linear_case(device, m, n, k, 3 * m + n)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU)
    ref = F.gelu(y.bfloat16().float(), approximate="none").bfloat16()
    assert strict_gate(ref, out) == 0
    assert within_composite(ref, out, y, 1.13)  # max |gelu'| = 1.129
    assert bitwise_fraction(F.gelu(F.linear(a, w, bias), approximate="none"), out) > 0.999


@pytest.mark.parametrize("packed", [False, True], ids=["plain", "packed"])
def test_gelu_epilogue_every_bf16_input(device, packed):
    """The wide kernel's GELU epilogue looks its result up in a table of
    bf16(gelu_erf(x)) over all 65536 bf16 patterns x, filled on the device by
    the same erf code.  With zero weights the nn.Linear output is the bias
    (+0 for a -0 bias, NaN for a NaN one), so a bias row holding every bf16
    pattern sends each table entry through the epilogue: bit for bit torch's
    GELU of torch's product, NaN for NaN, on every row."""
    m, n, k = 1024, 65536, 64
    a = torch.randn(m, k, device=device).bfloat16()
    w = torch.zeros(n, k, device=device, dtype=torch.bfloat16)
    bias = torch.arange(n, device=device, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    wp = native.prepack_weight(w) if packed else None
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU, packed_weight=wp)
    ref = F.gelu(F.linear(a, w, bias), approximate="none")
    nan_out, nan_ref = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_out, nan_ref)
    same = out.view(torch.int16) == ref.view(torch.int16)
    assert bool((same | nan_ref).all()), int((~(same | nan_ref)).sum())


def test_gelu_epilogue_table_and_erf_paths(device):
    """Both paths of the wide kernel's GELU epilogue, told apart: with one
    table entry overwritten (x = 1.0), the table path returns the planted
    value for exactly that input; with the ready flag cleared, every input
    goes through the erf and all 65536 outputs are torch's again.  Both paths
    are checked over every bf16 input."""
    m, n, k = 1024, 65536, 64
    a = torch.randn(m, k, device=device).bfloat16()
    w = torch.zeros(n, k, device=device, dtype=torch.bfloat16)
    bias = torch.arange(n, device=device, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    ref = F.gelu(F.linear(a, w, bias), approximate="none")
    nan_ref = torch.isnan(ref)

    def mismatches(out):
        same = out.view(torch.int16) == ref.view(torch.int16)
        return ~(same | (nan_ref & torch.isnan(out)))

    one, planted = 0x3F80, 0x1234
    try:
        native.debug_gelu_table(device, entry=one, value=planted)
        out = native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU)
        bad = mismatches(out)
        assert bool(bad[:, one].all()) and bool((out[:, one].view(torch.int16) == planted).all())
        assert int(bad.sum()) == m, "only the planted entry differs: the table path ran"
        native.debug_gelu_table(device, ready=0)
        out = native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU)
        assert int(mismatches(out).sum()) == 0, "the erf path ignores the table"
    finally:
        native.debug_gelu_table(device, ready=1, entry=one, value=-1)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU)
    assert int(mismatches(out).sum()) == 0


@pytest.mark.parametrize("epi", [native.ENC_EPI_BIAS_RESIDUAL_KEEP, native.ENC_EPI_BIAS_RESIDUAL_ZERO])
@pytest.mark.parametrize("m,n,k", [(100, 512, 512), (8192, 1024, 1024), (1000, 1024, 4096)])
def test_linear_residual(device, m, n, k, epi):
    a, w, bias, res, y = _linear_case(device, m, n, k, 5 * m + k)
    mask = torch.rand(m, device=device) > 0.3
    out = native.linear(a, w, bias, epi, residual=res, row_mask=mask)
    ref = (res.float() + y.bfloat16().float()).bfloat16()
    assert strict_gate(ref[mask], out[mask]) == 0
    assert within_composite(ref[mask], out[mask], y[mask], 1.0)
    torch_ref = res + F.linear(a, w, bias)
    assert bitwise_fraction(torch_ref[mask], out[mask]) > 0.999
    if epi == native.ENC_EPI_BIAS_RESIDUAL_KEEP:
        assert torch.equal(out[~mask], res[~mask])
    else:
        assert torch.all(out[~mask] == 0)
    # no mask: every row takes the residual sum
    out2 = native.linear(a, w, bias, epi, residual=res)
    assert within_composite(ref, out2, y, 1.0)


@pytest.mark.parametrize(
    "m,n,k",
    [(8192, 96, 32), (8192, 32, 32), (37, 96, 32), (1, 32, 32), (300, 64, 96), (8192, 384, 128), (8192, 128, 128),
     (128, 384, 128), (37, 128, 128), (256, 128, 384), (1, 384, 128)],
)
def test_linear_narrow_and_d128_shapes_bitwise(device, m, n, k):
    """The official matrix's projection shapes: d_model 32 (N or K not a
    multiple of 64: the one-block-per-wavefront kernel) and d_model 128 (with
    up to 256 rows: the skinny kernel's 128-wide K stages); every epilogue
    equals torch's bf16 ops bit for bit."""
    a, w, bias, res, _ = _linear_case(device, m, n, k, 29 * m + n + k)
    ref = F.linear(a, w, bias)
    assert torch.equal(native.linear(a, w, bias, native.ENC_EPI_BIAS), ref)
    assert torch.equal(native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU), F.gelu(ref, approximate="none"))
    mask = torch.rand(m, device=device) > 0.3
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS_RESIDUAL_ZERO, residual=res, row_mask=mask)
    assert torch.equal(out[mask], (res + ref)[mask]) and torch.all(out[~mask] == 0)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS_RESIDUAL_KEEP, residual=res, row_mask=mask)
    assert torch.equal(out[mask], (res + ref)[mask]) and torch.equal(out[~mask], res[~mask])


@pytest.mark.parametrize("m,n,k", [(128, 512, 2048), (64, 512, 2048), (256, 512, 2048), (16, 1536, 512), (1, 512, 512), (16, 1024, 4096), (128, 1024, 4096)])
def test_linear_split_k_order_bitwise(device, m, n, k):
    """Shapes where torch's bf16 nn.Linear splits K: the kernel's partial sums
    follow the same chunking, so the outputs are equal bit for bit."""
    a, w, bias, res, _ = _linear_case(device, m, n, k, 17 * m + n + k)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS)
    assert torch.equal(out, F.linear(a, w, bias))
    out_res = native.linear(a, w, bias, native.ENC_EPI_BIAS_RESIDUAL_ZERO, residual=res)
    assert torch.equal(out_res, res + F.linear(a, w, bias))


@pytest.mark.parametrize("m,n,k", [
    (3200000, 1024, 1024), (100000, 1024, 1024),  # c5 and one c5 sequence
    (1600000, 1024, 1024), (1000000, 1024, 1024), (400000, 1024, 1024), (50000, 1024, 1024),
    (100000, 4096, 1024), (100000, 1024, 4096),  # an F = 4096 FFN at one c5 sequence
])
def test_linear_streamk_tail_bitwise(device, m, n, k):
    """[M, K] x [N, K]^T in the library's stream-K regime: the reduction order
    of torch's nn.Linear is measured on this device for the shape
    (linear_order.py) and the kernel follows it, so every output, tail rows
    included, is equal bit for bit, at row counts whose tails differ (and at
    50 000 rows, where the library's grid divides the tiles and nothing
    splits).  At c5's M the packed QKV projection matches the three separate
    products the reference runs."""
    from tiktoktechjam2026track3_amd import linear_order

    g = torch.Generator(device=device).manual_seed(m % 9973 + n + k)
    a = torch.randn(m, k, generator=g, device=device).bfloat16()
    w = ((torch.rand(n, k, generator=g, device=device) * 2 - 1) / math.sqrt(k)).bfloat16()
    bias = ((torch.rand(n, generator=g, device=device) * 2 - 1) / 32).bfloat16()
    ref = F.linear(a, w, bias)
    out = native.linear(a, w, bias, native.ENC_EPI_BIAS)
    order = linear_order.ensure(m, n, k, device)
    mismatches = int((ref.view(torch.int16) != out.view(torch.int16)).sum())
    print(f"[streamk] {m}x{n}x{k}: order {order.kind}, {order.split_tiles()} split tiles, "
          f"{mismatches} mismatching outputs", flush=True)
    assert order.kind in ("sequential", "tail")
    assert mismatches == 0
    del out
    assert torch.equal(native.linear(a, w, bias, native.ENC_EPI_BIAS_GELU), F.gelu(ref, approximate="none"))
    if m == 3200000:
        w3 = ((torch.rand(3072, 1024, generator=g, device=device) * 2 - 1) / 32).bfloat16()
        b3 = ((torch.rand(3072, generator=g, device=device) * 2 - 1) / 32).bfloat16()
        q, k_, v_t = native.qkv_proj(a.view(32, 100000, 1024), w3, b3, 16)
        for i, got in enumerate((q, k_)):
            part = F.linear(a, w3[1024 * i:1024 * (i + 1)], b3[1024 * i:1024 * (i + 1)])
            assert torch.equal(part.view(32, 100000, 16, 64).transpose(1, 2), got)


def test_measured_orders_match_the_committed_tables(device):
    """The runtime measurement reads the same split tables off the library
    that the maintainer probe committed (csrc/streamk_tail.h, measured with
    torch 2.10.0+rocm7.0 on a 256-CU MI355X).  A different build or device may
    legitimately differ: the test then names the versions instead of failing
    on bits."""
    import re
    from pathlib import Path

    from tiktoktechjam2026track3_amd import linear_order

    text = (Path(native.__file__).parent / "csrc" / "streamk_tail.h").read_text()
    props = torch.cuda.get_device_properties(device)
    if torch.__version__ != "2.10.0+rocm7.0" or props.multi_processor_count != 256:
        pytest.skip(f"tables were measured with torch 2.10.0+rocm7.0 on 256 CUs; this is torch "
                    f"{torch.__version__} (HIP {torch.version.hip}) on {props.multi_processor_count} CUs")
    for mm in re.finditer(r"\{(\d+), 1024, 1024, (\d+), (\d+), 4, (kTailSplit_\w+)\}", text):
        m, first, rows, name = int(mm.group(1)), int(mm.group(2)), int(mm.group(3)), mm.group(4)
        body = re.search(name + r"\[\d+\] = \{([^}]*)\}", text).group(1)
        table = [int(v) for v in body.replace("\n", " ").split(",") if v.strip()]
        order = linear_order.ensure(m, 1024, 1024, device)
        assert (order.kind, order.first_tile_row, order.tile_rows, order.split) == ("tail", first, rows, table), m


@pytest.mark.parametrize("n,k", [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096), (1536, 512), (384, 256),
                                 (128, 32)])
def test_prepack_weight_layout(device, n, k):
    """The packed copy is W[N, K] regrouped as [N / P][K / 32][P][32] (P = 256
    when N % 256 == 0, else 128): a pure permutation, checked against the same
    regrouping done with torch views."""
    g = torch.Generator(device=device).manual_seed(n + k)
    w = torch.randn(n, k, generator=g, device=device).bfloat16()
    p = native.prepack_rows(n, k)
    assert p == (256 if n % 256 == 0 else 128)
    ref = w.view(n // p, p, k // 32, 32).permute(0, 2, 1, 3).reshape(-1)
    assert torch.equal(native.prepack_weight(w), ref)


@pytest.mark.parametrize(
    "m,n,k,epi",
    [
        (8192, 3072, 1024, native.ENC_EPI_BIAS),               # 256x128x64 tiles (c3 qkv rows)
        (32768, 3072, 1024, native.ENC_EPI_BIAS),              # 256x256x32 (c4 qkv)
        (32768, 4096, 1024, native.ENC_EPI_BIAS_GELU),         # 256x128x32, two per CU (ffn_in)
        (32768, 1024, 4096, native.ENC_EPI_BIAS_RESIDUAL_ZERO),
        (32768, 1024, 1024, native.ENC_EPI_BIAS_RESIDUAL_KEEP),
        (5000, 384, 256, native.ENC_EPI_BIAS),                 # P = 128, ragged last tile row
        (1100, 128, 1024, native.ENC_EPI_BIAS),                # 128x128x64 tiles
        (100000, 1024, 1024, native.ENC_EPI_BIAS),             # stream-K tail rows read the plain weight
        (200, 1024, 1024, native.ENC_EPI_BIAS),                # few rows: the packed copy goes unread
        # 256x256 tiles: one and two 64-deep blocks in the two-stage ring
        # (plain weight), two to 130 32-deep blocks in the four-stage ring
        # (packed), K % 128 == 64, each with a ragged last tile row
        (8292, 1024, 64, native.ENC_EPI_BIAS_RESIDUAL_ZERO),
        (8292, 1024, 128, native.ENC_EPI_BIAS_RESIDUAL_KEEP),
        (4100, 2048, 320, native.ENC_EPI_BIAS_RESIDUAL_ZERO),
        (8292, 1024, 4160, native.ENC_EPI_BIAS_RESIDUAL_KEEP),
        # c4's out_proj and ffn_out shapes with a row mask (the residual
        # epilogue's prefetched mask bytes)
        (32768, 1024, 1024, native.ENC_EPI_BIAS_RESIDUAL_KEEP),
        (32768, 1024, 4096, native.ENC_EPI_BIAS_RESIDUAL_ZERO),
    ],
)
def test_linear_prepacked_is_bitwise_the_plain_product(device, m, n, k, epi):
    g = torch.Generator(device=device).manual_seed(m + n + k)
    a = torch.randn(m, k, generator=g, device=device).bfloat16()
    w = ((torch.rand(n, k, generator=g, device=device) * 2 - 1) / math.sqrt(k)).bfloat16()
    bias = ((torch.rand(n, generator=g, device=device) * 2 - 1) / 32).bfloat16()
    residual = mask = None
    if epi in (native.ENC_EPI_BIAS_RESIDUAL_KEEP, native.ENC_EPI_BIAS_RESIDUAL_ZERO):
        residual = torch.randn(m, n, generator=g, device=device).bfloat16()
        mask = torch.rand(m, generator=g, device=device) > 0.3
    plain = native.linear(a, w, bias, epi, residual=residual, row_mask=mask)
    packed = native.linear(a, w, bias, epi, residual=residual, row_mask=mask, packed_weight=native.prepack_weight(w))
    mismatches = int((plain.view(torch.int16) != packed.view(torch.int16)).sum())
    print(f"[prepack] {m}x{n}x{k} epi {epi}: {mismatches} mismatches", flush=True)
    assert mismatches == 0
    if epi == native.ENC_EPI_BIAS:
        assert torch.equal(packed, F.linear(a, w, bias))
    elif residual is not None:
        # masked rows: the residual (keep) or zero, the others torch's sum
        ref = residual + F.linear(a, w, bias)
        assert bitwise_fraction(ref[mask], packed[mask]) > 0.999
        if epi == native.ENC_EPI_BIAS_RESIDUAL_KEEP:
            assert torch.equal(packed[~mask], residual[~mask])
        else:
            assert torch.all(packed[~mask] == 0)


def test_linear_prepacked_rejects_unpackable_shapes(device):
    a = torch.zeros(2048, 1024, device=device, dtype=torch.bfloat16)
    w = torch.zeros(96, 1024, device=device, dtype=torch.bfloat16)
    bias = torch.zeros(96, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no packed form"):
        native.prepack_weight(w)
    with pytest.raises(native.EncoderKernelError, match="out_features % 128") as info:
        native.linear(a, w, bias, packed_weight=torch.zeros(96 * 1024, device=device, dtype=torch.bfloat16))
    assert info.value.code == native.ENC_ERR_UNSUPPORTED


@pytest.mark.parametrize("rows,d,f", [(128, 512, 2048), (8192, 1024, 4096), (100000, 1024, 1024), (4096, 128, 128),
                                     (300, 256, 1024)])
def test_ffn_fused_is_the_reference_ffn(device, rows, d, f):
    """enc_ffn_fused_bf16 = residual + ffn_out(gelu(ffn_in(h))) with the
    block's masked rows zeroed, bit for bit as torch computes the reference
    block's FFN (models.py:724-725, 734-737)."""
    g = torch.Generator(device=device).manual_seed(rows + d + f)
    h = torch.randn(rows, d, generator=g, device=device).bfloat16()
    res = torch.randn(rows, d, generator=g, device=device).bfloat16()
    w1 = ((torch.rand(f, d, generator=g, device=device) * 2 - 1) / math.sqrt(d)).bfloat16()
    b1 = ((torch.rand(f, generator=g, device=device) * 2 - 1) / math.sqrt(d)).bfloat16()
    w2 = ((torch.rand(d, f, generator=g, device=device) * 2 - 1) / math.sqrt(f)).bfloat16()
    b2 = ((torch.rand(d, generator=g, device=device) * 2 - 1) / math.sqrt(f)).bfloat16()
    mask = torch.rand(rows, generator=g, device=device) > 0.2
    out = native.ffn(h, w1, b1, w2, b2, res, row_mask=mask)
    ref = res + F.linear(F.gelu(F.linear(h, w1, b1), approximate="none"), w2, b2)
    ref = ref.masked_fill(~mask[:, None], 0)
    mismatches = int((ref.view(torch.int16) != out.view(torch.int16)).sum())
    print(f"[ffn] {rows}x{d}x{f}: {mismatches} mismatches against torch", flush=True)
    assert mismatches == 0
    # the same two products through enc_linear_bf16
    two = native.linear(native.linear(h, w1, b1, native.ENC_EPI_BIAS_GELU), w2, b2,
                        native.ENC_EPI_BIAS_RESIDUAL_ZERO, residual=res, row_mask=mask)
    assert torch.equal(two, out)
    # out may alias the residual
    inplace = res.clone()
    native.ffn(h, w1, b1, w2, b2, inplace, row_mask=mask, out=inplace)
    assert torch.equal(inplace, out)


@pytest.mark.parametrize(
    "b,s,d,h",
    [(1, 128, 512, 8), (2, 100, 512, 8), (8, 1024, 1024, 16), (3, 37, 1024, 16), (64, 128, 32, 4), (3, 37, 128, 16),
     (2, 100, 1024, 4), (4, 300, 128, 32), (4, 1024, 128, 32), (40, 40, 1024, 16), (3, 1000, 1024, 8), (2, 4100, 1024, 16)],
)
def test_qkv_head_major(device, b, s, d, h):
    """Head-major Q, K and padded V^T against torch's linear.  The shapes
    reach every kernel family: the 16-row tiles (few rows or K <= 256), the
    large tiles with full and partial tile rows, sequences shorter than a
    tile's row stride (40 x 40) and not a multiple of 8 (4100), and a
    head_dim of 4 at a shape the large tiles would otherwise take."""
    g = torch.Generator(device=device).manual_seed(b * s + d)
    x = torch.randn(b, s, d, generator=g, device=device).bfloat16()
    w = (torch.randn(3 * d, d, generator=g, device=device) / math.sqrt(d)).bfloat16()
    bias = (torch.randn(3 * d, generator=g, device=device) * 0.05).bfloat16()
    q, k, v_t = native.qkv_proj(x, w, bias, h)
    y = F.linear(x.float(), w.float(), bias.float()).bfloat16()
    hd = d // h
    ref = y.view(b, s, 3, h, hd).permute(2, 0, 3, 1, 4)  # [3, B, H, S, hd]
    assert within_ulps(ref[0], q, 1) and within_ulps(ref[1], k, 1)
    assert within_ulps(ref[2].transpose(-1, -2), v_t[..., :s], 1)
    packed = F.linear(x, w, bias).view(b, s, 3, h, hd).permute(2, 0, 3, 1, 4)
    assert bitwise_fraction(packed[0], q) > 0.999 and bitwise_fraction(packed[1], k) > 0.999
    assert bitwise_fraction(packed[2].transpose(-1, -2), v_t[..., :s]) > 0.999


def test_softmax_exp_matches_device_expf_exhaustively(device):
    """The exact attention's inlined exp equals the device library's expf on
    every float in [-104, -0] (below -103.28 both return 0) and at -inf."""
    assert native.selfcheck_expf(0x80000000, 0xC2D00000, device) == 0
    assert native.selfcheck_expf(0xFF800000, 0xFF800000, device) == 0  # -inf
    assert native.selfcheck_expf(0x00000000, 0x00000000, device) == 0  # +0


def _attention_inputs(device, b, h, s, seed, hd=64):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(b, h, s, hd, generator=g, device=device).bfloat16()
    k = torch.randn(b, h, s, hd, generator=g, device=device).bfloat16()
    v = torch.randn(b, h, s, hd, generator=g, device=device).bfloat16()
    ld = native.vt_stride(s)
    v_t = torch.full((b, h, hd, ld), float("nan"), device=device, dtype=torch.bfloat16)
    v_t[..., :s] = v.transpose(-1, -2)
    return q, k, v, v_t


def _oracle_context(q, k, v, causal, mask):
    b, h, s, hd = q.shape
    ctx = attention_rows(q, k, v, hd**-0.5, causal, mask, torch.arange(s, device=q.device))
    return ctx.transpose(1, 2).reshape(b, s, h * hd)


def _context_error(ref: torch.Tensor, out: torch.Tensor) -> float:
    return float((ref.float() - out.float()).abs().max())


def within_weight_rounding(ref, out, q, k, v, causal, mask=None) -> bool:
    """|out - ref| <= 2^-7 * sum_j p_j |v_j| + one bf16 spacing of ref.

    The reference and the online kernel each round every softmax weight once
    to bf16 (relative error <= 2^-9), at different points; the context error is
    bounded by that weight error times the magnitudes of the values it weighs,
    which the oracle gives as the attention context of |v|."""
    scale_terms = _oracle_context(q, k, v.abs(), causal, mask).float()
    ref, out = ref.float(), out.float()
    _, exponent = torch.frexp(ref)
    spacing = torch.ldexp(torch.ones_like(ref), exponent - 8)
    return bool(((out - ref).abs() <= 2.0**-7 * scale_terms + spacing).all())


@pytest.mark.parametrize("online", [False, True], ids=["exact", "online"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h,s", [(1, 1, 1), (1, 2, 63), (2, 3, 64), (1, 2, 100), (2, 8, 128), (1, 4, 1000), (2, 16, 1024), (1, 2, 4100)])
def test_attention_unmasked(device, b, h, s, causal, online):
    # v_t's padding columns hold NaN: a kernel that multiplies them (even by 0) fails
    q, k, v, v_t = _attention_inputs(device, b, h, s, 11 * s + b)
    out = native.attention(q, k, v_t, 0.125, causal, online=online)
    ref = _oracle_context(q, k, v, causal, None)
    assert strict_gate(ref, out) == 0, f"max abs {_context_error(ref, out)}"
    if not online:
        # exact three-sweep softmax: the same bf16 probabilities as the
        # reference up to rare last-bit differences of exp/sum order
        assert bitwise_fraction(ref, out) > 0.99
    else:
        # one-pass online softmax: the weights are rounded before (not after)
        # normalisation; the difference is bounded by that rounding
        assert within_weight_rounding(ref, out, q, k, v, causal)
    if causal:
        # row 0 attends only to key 0: its context is v[:, :, 0] exactly
        assert torch.equal(out[:, 0, :].view(b, h, 64), v[:, :, 0, :])


@pytest.mark.parametrize("online", [False, True], ids=["exact", "online"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h,s", [(4, 2, 256), (3, 4, 1000), (2, 2, 8192)])
def test_attention_prefix_padding(device, b, h, s, causal, online):
    q, k, v, v_t = _attention_inputs(device, b, h, s, 13 * s + b)
    g = torch.Generator(device=device).manual_seed(s)
    lengths = torch.randint(max(1, s // 2), s + 1, (b,), generator=g, device=device)
    lengths[0] = 1 if b > 1 else lengths[0]
    mask = torch.arange(s, device=device)[None, :] < lengths[:, None]
    kv_len = native.mask_lengths(mask)
    assert torch.equal(kv_len.long(), lengths)
    out = native.attention(q, k, v_t, 0.125, causal, kv_len=kv_len, online=online)
    ref = _oracle_context(q, k, v, causal, mask)
    valid = mask[..., None].expand_as(out)
    assert strict_gate(ref[valid], out[valid]) == 0
    assert torch.all(out[~valid] == 0)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_online_long_rows_match_exact(device, causal):
    """Long rows (block-softmax regime of the reference): the online kernel
    stays within the weight-rounding bound of the bit-exact kernel."""
    q, k, v, v_t = _attention_inputs(device, 1, 4, 12288, 77)
    online = native.attention(q, k, v_t, 0.125, causal, online=True)
    exact = native.attention(q, k, v_t, 0.125, causal)
    assert strict_gate(exact, online) == 0
    assert within_weight_rounding(exact, online, q, k, v, causal)


def test_attention_online_large_scores(device):
    """Scores spanning hundreds of units (growing maxima along the row force
    the lazy rescale) still give the reference's context."""
    b, h, s = 1, 2, 2048
    q, k, v, v_t = _attention_inputs(device, b, h, s, 5)
    ramp = torch.linspace(0, 6, s, device=device)[None, None, :, None]
    k = (k.float() * (1 + ramp)).bfloat16()
    q = (q.float() * 4).bfloat16()
    for causal in (False, True):
        out = native.attention(q, k, v_t, 0.125, causal, online=True)
        ref = _oracle_context(q, k, v, causal, None)
        assert strict_gate(ref, out) == 0, f"max abs {_context_error(ref, out)}"


@pytest.mark.parametrize(
    "b,h,s,causal,prefix",
    [(1, 8, 128, False, False), (8, 16, 1024, True, False), (4, 16, 8192, True, True), (4, 16, 4096, False, False)],
)
def test_attention_config_shapes_bitwise(device, b, h, s, causal, prefix):
    """At the benchmark configurations' shapes the reference's batched matmuls
    accumulate K in the kernel's order and the softmax follows torch's
    regime (warp softmax up to 2048 keys, block softmax with the hardware exp
    beyond), so the context equals the oracle's bit for bit."""
    q, k, v, v_t = _attention_inputs(device, b, h, s, 3 * s + h)
    kv_len = mask = None
    if prefix:
        g = torch.Generator(device=device).manual_seed(s + 1)
        lengths = torch.randint(s // 2, s + 1, (b,), generator=g, device=device)
        mask = torch.arange(s, device=device)[None, :] < lengths[:, None]
        kv_len = lengths.int()
    out = native.attention(q, k, v_t, 0.125, causal, kv_len=kv_len)
    ref = _oracle_context(q, k, v, causal, mask)
    if mask is not None:
        valid = mask[..., None].expand_as(out)
        assert torch.equal(ref[valid], out[valid])
        assert torch.all(out[~valid] == 0)
    else:
        assert torch.equal(ref, out)


@pytest.mark.parametrize(
    "b,h,s,causal,prefix,q_gain,scale",
    [(16, 16, 300, True, False, 1.0, 0.125), (8, 16, 777, True, False, 1.0, 0.125),
     (8, 16, 1024, True, False, 12.0, 0.125), (4, 16, 2048, True, False, 1.0, 0.125),
     (8, 16, 1000, False, False, 1.0, 0.125), (8, 16, 1024, False, True, 1.0, 0.125),
     (8, 16, 1024, True, False, 1.0, 0.1), (8, 16, 1000, False, True, 4.0, 0.1)],
)
def test_attention_half_tile_rows_bitwise(device, b, h, s, causal, prefix, q_gain, scale):
    """Head-dim-64 rows of 257-2048 keys with enough rows to fill the chip
    (causal without key masks; non-causal past 512 keys, with or without a
    prefix mask) take the three-wavefront kernel that runs sweeps B and C one
    32-key half tile at a time.  A ragged last tile (300, 777, 1000), padded
    keys, scores large enough for weights below 2^-100 (q_gain 12: the IEEE
    division path) and a scale that is not a power of two (0.1: the scores
    rounded twice, bf16(bf16(q.k) * scale)) must still give the oracle's
    bits."""
    q, k, v, v_t = _attention_inputs(device, b, h, s, 5 * s + b)
    q = (q.float() * q_gain).bfloat16()
    kv_len = mask = None
    if prefix:
        g = torch.Generator(device=device).manual_seed(s + 7)
        lengths = torch.randint(s // 2, s + 1, (b,), generator=g, device=device)
        mask = torch.arange(s, device=device)[None, :] < lengths[:, None]
        kv_len = lengths.int()
    out = native.attention(q, k, v_t, scale, causal, kv_len=kv_len)
    ctx = attention_rows(q, k, v, scale, causal, mask, torch.arange(s, device=device))
    ref = ctx.transpose(1, 2).reshape(b, s, h * 64)
    if mask is not None:
        valid = mask[..., None].expand_as(out)
        assert torch.equal(ref[valid], out[valid]), f"max abs {_context_error(ref[valid], out[valid])}"
        assert torch.all(out[~valid] == 0)
    else:
        assert torch.equal(ref, out), f"max abs {_context_error(ref, out)}"


@pytest.mark.parametrize(
    "hd,b,h,s,causal,prefix,exact",
    [
        (32, 64, 4, 128, True, True, True),  # official cases 1-6 (d_model 128, 4 heads)
        (32, 1, 4, 128, False, False, True),
        (32, 64, 4, 32, True, True, True),  # official case 12
        (32, 8, 4, 1024, True, True, True),  # official case 13's rows
        (32, 2, 3, 300, False, True, True),
        (32, 1, 2, 4100, True, False, False),  # block-softmax regime
        (128, 64, 1, 128, True, True, True),  # official case 9 (1 head of 128)
        (128, 2, 2, 200, False, False, True),
        (128, 1, 2, 1000, True, True, True),
        (128, 1, 1, 4100, False, False, True),
        (64, 64, 2, 128, True, True, True),  # official case 10 (2 heads of 64)
        (8, 64, 16, 128, True, True, True),  # official case 11 (16 heads of 8)
        (8, 64, 4, 128, True, True, True),  # official case 7's attention (d_model 32)
        (8, 2, 3, 300, False, True, False),
        (8, 1, 2, 4100, True, False, False),
        (256, 64, 4, 128, True, True, True),  # official case 8 (4 heads of 256)
        (256, 2, 2, 200, False, False, True),
        (256, 1, 2, 1000, True, True, True),
        (256, 1, 1, 4100, False, False, True),
    ],
)
def test_attention_head_dims_bitwise(device, hd, b, h, s, causal, prefix, exact):
    """Head dims 8, 32, 128 and 256 at the official matrix's shapes (and the row
    regimes either side of 2048 keys): with the scale hd^-0.5 (a power of two
    only for 256), the context equals the oracle's bit for bit.

    Measured exceptions (exact=False), none at an official shape: for head
    dims 8 and 32 the reference's P.V product (N = 8 or 32) reduces K in
    another order at some lengths (300 keys at head dim 8; 2560 and 4100 keys,
    not 4096, at head dim 32), and a few context values per 10^4 then differ
    by one bf16 ulp.  Those cases are held to the strict gate and a 99.9%
    bitwise share."""
    q, k, v, v_t = _attention_inputs(device, b, h, s, 5 * s + hd + b, hd=hd)
    kv_len = mask = None
    if prefix:
        g = torch.Generator(device=device).manual_seed(s + hd)
        lengths = torch.randint(max(1, s // 2), s + 1, (b,), generator=g, device=device)
        mask = torch.arange(s, device=device)[None, :] < lengths[:, None]
        kv_len = lengths.int()
    out = native.attention(q, k, v_t, hd**-0.5, causal, kv_len=kv_len)
    ref = _oracle_context(q, k, v, causal, mask)
    valid = torch.ones_like(out, dtype=torch.bool) if mask is None else mask[..., None].expand_as(out)
    print(f"[attention hd {hd}] bitwise share {bitwise_fraction(ref[valid], out[valid]):.6f}", flush=True)
    if exact:
        assert torch.equal(ref[valid], out[valid]), f"max abs {_context_error(ref[valid], out[valid])}"
    else:
        assert strict_gate(ref[valid], out[valid]) == 0
        assert bitwise_fraction(ref[valid], out[valid]) > 0.999
    assert torch.all(out[~valid] == 0)
    if causal:
        assert torch.equal(out[:, 0, :].view(b, h, hd), v[:, :, 0, :])


def test_attention_online_rejects_other_head_dims(device):
    q, k, v, v_t = _attention_inputs(device, 1, 1, 64, 3, hd=32)
    with pytest.raises(native.EncoderKernelError, match="head_dim must be 64"):
        native.attention(q, k, v_t, 32**-0.5, False, online=True)


@pytest.mark.parametrize("online", [False, True], ids=["exact", "online"])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_general_mask(device, causal, online):
    b, h, s = 2, 4, 300
    q, k, v, v_t = _attention_inputs(device, b, h, s, 99)
    g = torch.Generator(device=device).manual_seed(5)
    mask = torch.rand(b, s, generator=g, device=device) > 0.4
    mask[:, 0] = True
    out = native.attention(q, k, v_t, 0.125, causal, key_mask=mask, online=online)
    ref = _oracle_context(q, k, v, causal, mask)
    rows = mask[..., None].expand_as(out)  # valid query rows always see >= 1 key
    assert strict_gate(ref[rows], out[rows]) == 0


@pytest.mark.parametrize("online", [False, True], ids=["exact", "online"])
def test_attention_non_power_of_two_scale(device, online):
    q, k, v, v_t = _attention_inputs(device, 1, 2, 200, 7)
    scale = 0.1
    out = native.attention(q, k, v_t, scale, False, online=online)
    ctx = attention_rows(q, k, v, scale, False, None, torch.arange(200, device=device))
    ref = ctx.transpose(1, 2).reshape(1, 200, 128)
    assert strict_gate(ref, out) == 0
