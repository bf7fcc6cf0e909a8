"""Pin the oracle (CPU).

Every oracle function is checked against golden vectors that the reference
itself produced (tests/golden/make_golden.py) and, where mathematics fixes the
answer, against independent fp64 forms (oracle/numerics.py).  A final group of
tests plants plausible mistakes in copies of the oracle and shows the checks
catch them.
"""

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.encoder_oracle as eo
from oracle import numerics

GOLDEN = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLDEN / "reference_vectors.json").read_text())
ARR = np.load(GOLDEN / "reference_vectors.npz", allow_pickle=False)
CPU = torch.device("cpu")


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().float().numpy().tobytes()).hexdigest()


# ------------------------------------------------------------- weights ----

@pytest.mark.parametrize("name", sorted(META["weights"]))
def test_init_state_dict_matches_reference(name):
    entry = META["weights"][name]
    b, s, d, h, f, layers, causal = entry["config"]
    sd = eo.init_state_dict(d, h, f, layers, seed=entry["seed"])
    assert list(sd) == list(entry["params"]), "parameter names/order differ"
    for key, ref in entry["params"].items():
        value = sd[key]
        assert list(value.shape) == ref["shape"], key
        assert sha(value) == ref["sha256_fp32"], key
        if f"w/{name}/{key}" in ARR:
            assert np.array_equal(ARR[f"w/{name}/{key}"], value.numpy())


def test_linear_init_bounds_follow_fan_in():
    sd = eo.init_state_dict(256, 4, 1024, 1, seed=0)
    for key, fan_in in (("layers.0.attention.q_proj.weight", 256), ("layers.0.ffn_out.weight", 1024)):
        bound = 1 / math.sqrt(fan_in)
        assert float(sd[key].abs().max()) <= bound * (1 + 1e-6)
        assert float(sd[key].abs().max()) > 0.95 * bound  # uniform fills the interval


# -------------------------------------------------------------- inputs ----

@pytest.mark.parametrize("name", sorted(META["inputs"]))
def test_generate_case_matches_reference(name):
    entry = META["inputs"][name]
    b, s, d = entry["config"][:3]
    x, mask = eo.generate_case(b, s, d, CPU, torch.float32, entry["seed"], entry["padding_ratio"], entry["input_scale"])
    assert sha(x) == entry["x"]["sha256_fp32"]
    assert mask.sum(1).tolist() == entry["lengths"]
    if f"in/{name}/mask" in ARR:
        assert np.array_equal(ARR[f"in/{name}/mask"], mask.numpy())
    # prefix shape and padded rows zeroed
    for row, length in enumerate(entry["lengths"]):
        assert bool(mask[row, :length].all()) and not bool(mask[row, length:].any())
        assert float(x[row, length:].abs().sum()) == 0.0


def test_c4_lengths_range():
    lengths = META["inputs"]["c4_cpu"]["lengths"]
    assert all(4096 <= n <= 8192 for n in lengths)


# ------------------------------------------------------------- forward ----

def _forward_case(name):
    entry = META["forward"][name]
    b, s, d, h, f, layers, causal = entry["config"]
    dtype = torch.float32 if entry["dtype"] == "torch.float32" else torch.bfloat16
    sd = eo.init_state_dict(d, h, f, layers, seed=entry["weight_seed"])
    sd = {k: v.to(dtype) for k, v in sd.items()}
    x, mask = eo.generate_case(b, s, d, CPU, dtype, entry["input_seed"], entry["padding_ratio"])
    with torch.inference_mode():
        y = eo.encoder_forward(sd, x, mask, causal, h, layers)
    return entry, sd, x, mask, y


@pytest.mark.parametrize("name", [n for n in META["forward"] if n != "c1"])
def test_forward_matches_reference_tiny(name):
    entry, _, _, _, y = _forward_case(name)
    ref = torch.from_numpy(ARR[f"fwd/{name}/y"])
    if entry["dtype"] == "torch.float32":
        assert torch.allclose(y, ref, rtol=1e-5, atol=1e-5)
    else:
        assert torch.equal(y.float(), ref), float((y.float() - ref).abs().max())


def test_forward_matches_reference_c1():
    entry, _, _, _, y = _forward_case("c1")
    rows = entry["sample_rows"]
    ref = torch.from_numpy(ARR["fwd/c1/y_rows"])
    assert torch.allclose(y[:, rows, :], ref, rtol=1e-5, atol=1e-5)
    assert abs(float(y.double().sum()) - entry["y"]["sum"]) < 1e-3
    assert abs(float((y.double() ** 2).sum()) - entry["y"]["sumsq"]) < 1e-2


@pytest.mark.parametrize("name", ["tiny_causal_pad_fp32", "tiny_noncausal_fp32"])
def test_forward_matches_fp64_definition(name):
    entry, sd, x, mask, y = _forward_case(name)
    b, s, d, h, f, layers, causal = entry["config"]
    npsd = {k: v.double().numpy() for k, v in sd.items()}
    ref = numerics.encoder_forward(npsd, x.double().numpy(), mask.numpy(), causal, h, layers)
    assert np.allclose(y.double().numpy(), ref, rtol=1e-4, atol=2e-5)


def test_bf16_forward_matches_fp64_definition_with_bf16_rounding():
    entry, sd, x, mask, y = _forward_case("tiny_hd64_pad_bf16")
    b, s, d, h, f, layers, causal = entry["config"]
    npsd = {k: v.double().numpy() for k, v in sd.items()}
    ref = numerics.encoder_forward(npsd, x.double().numpy(), mask.numpy(), causal, h, layers, bf16=True)
    diff = np.abs(y.double().numpy() - ref)
    ok = (diff < 1e-2) | (diff < 1.6e-2 * np.abs(ref))
    assert ok.all(), diff.max()


# ------------------------------------------------- closed forms / invariants ----

def test_layer_norm_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 256, generator=g, dtype=torch.float64) * 4 + 1
    w = torch.rand(256, generator=g, dtype=torch.float64)
    b = torch.randn(256, generator=g, dtype=torch.float64)
    ref = numerics.layer_norm(x.numpy(), w.numpy(), b.numpy())
    assert np.allclose(F.layer_norm(x, (256,), w, b, 1e-5).numpy(), ref, atol=1e-12)
    y = numerics.layer_norm(x.numpy(), np.ones(256), np.zeros(256))
    assert np.allclose(y.mean(-1), 0, atol=1e-12) and np.allclose(y.var(-1), 1 / (1 + 1e-5 / x.numpy().var(-1)), atol=1e-9)


def test_gelu_closed_form():
    xs = np.array([-6.0, -1.0, -0.5, 0.0, 0.5, 1.0, 3.0])
    expected = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs])
    assert np.allclose(numerics.gelu(xs), expected, atol=1e-15)
    t = torch.tensor(xs)
    assert np.allclose(F.gelu(t, approximate="none").numpy(), expected, atol=1e-12)


def test_attention_rows_brute_force_and_invariants():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, 3, 9, 8, generator=g, dtype=torch.float64) for _ in range(3))
    mask = torch.ones(2, 9, dtype=torch.bool)
    mask[1, 6:] = False
    for causal in (False, True):
        ctx = eo.attention_rows(q, k, v, 8**-0.5, causal, mask, torch.arange(9))
        ref = numerics.attention(q.numpy(), k.numpy(), v.numpy(), 8**-0.5, causal, mask.numpy())
        # the oracle's softmax runs in fp32 as the reference's does (scores.float()),
        # so fp64 inputs agree with the fp64 definition to fp32 precision
        assert np.allclose(ctx.numpy(), ref, atol=2e-6)
        if causal:
            assert torch.allclose(ctx[:, :, 0], v[:, :, 0])  # row 0 sees key 0 only
    # rows of probabilities sum to one: the context of constant values is that constant
    ones = torch.ones_like(v) * 0.75
    ctx = eo.attention_rows(q, k, ones, 0.3, True, mask, torch.arange(9))
    assert torch.allclose(ctx, torch.full_like(ctx, 0.75))


def test_row_subset_layer_equals_full_layer():
    sd = eo.init_state_dict(64, 1, 128, 1, seed=7)
    x, mask = eo.generate_case(2, 40, 64, CPU, torch.float32, 3, 0.3)
    full = eo.encoder_layer(sd, 0, x, mask, True, 1)
    rows = torch.tensor([0, 5, 17, 39])
    sub = eo.encoder_layer(sd, 0, x, mask, True, 1, rows=rows)
    assert torch.allclose(full[:, rows], sub, atol=1e-6)
    blocked = eo.encoder_layer(sd, 0, x, mask, True, 1, block_rows=7)
    assert torch.allclose(full, blocked, atol=1e-6)


def test_pack_qkv_order():
    sd = eo.init_state_dict(32, 4, 64, 1, seed=1)
    packed = eo.pack_qkv(sd)
    w = packed["layers.0.attention.qkv_proj.weight"]
    assert torch.equal(w[:32], sd["layers.0.attention.q_proj.weight"])
    assert torch.equal(w[32:64], sd["layers.0.attention.k_proj.weight"])
    assert torch.equal(w[64:], sd["layers.0.attention.v_proj.weight"])
    assert "layers.0.attention.q_proj.weight" not in packed


def test_compare_rule_matches_reference_verdicts():
    for case in META["compare"]:
        res = eo.compare(torch.tensor(case["ref"]), torch.tensor(case["opt"]), case["rtol"], case["atol"])
        assert res["passed"] == case["passed"]
        assert res["failed"] == case["failed_elements"]


# ------------------------------------------------------ planted mistakes ----

def _planted_forward(monkeypatch, name, patch):
    patch(monkeypatch)
    _, _, _, _, y = _forward_case(name)
    return y


@pytest.mark.parametrize(
    "mistake",
    ["drop_scale", "no_causal", "transposed_ffn_order", "gelu_tanh"],
)
def test_planted_mistakes_are_caught(monkeypatch, mistake):
    name = "tiny_causal_pad_fp32"
    ref = torch.from_numpy(ARR[f"fwd/{name}/y"])
    original_rows = eo.attention_rows
    original_layer = eo.encoder_layer

    if mistake == "drop_scale":
        monkeypatch.setattr(eo, "attention_rows", lambda q, k, v, scale, *a: original_rows(q, k, v, 1.0, *a))
    elif mistake == "no_causal":
        monkeypatch.setattr(eo, "attention_rows", lambda q, k, v, scale, causal, *a: original_rows(q, k, v, scale, False, *a))
    elif mistake == "transposed_ffn_order":
        def layer(sd, i, *a, **kw):
            sd = dict(sd)
            p = f"layers.{i}."
            sd[p + "ffn_in.bias"] = sd[p + "ffn_in.bias"].flip(0)
            return original_layer(sd, i, *a, **kw)
        monkeypatch.setattr(eo, "encoder_layer", layer)
    elif mistake == "gelu_tanh":
        original_gelu = F.gelu
        monkeypatch.setattr(eo.F, "gelu", lambda t, approximate="none": original_gelu(t, approximate="tanh"))
    _, _, _, _, y = _forward_case(name)
    assert not torch.allclose(y, ref, rtol=1e-5, atol=1e-5), mistake


def test_final_mask_is_what_zeroes_padded_rows():
    """With the default init (final_norm.bias = 0) padded rows reach the final
    LayerNorm as zero rows and leave it as zeros even without the final
    masked_fill; a non-zero bias shows that the mask, not the init, zeroes
    them (models.py:917-918)."""
    sd = eo.init_state_dict(32, 2, 64, 1, seed=3)
    sd["final_norm.bias"] = torch.full_like(sd["final_norm.bias"], 0.25)
    x, mask = eo.generate_case(2, 12, 32, CPU, torch.float32, 5, 0.5)
    assert not bool(mask.all())
    with torch.inference_mode():
        y = eo.encoder_forward(sd, x, mask, True, 2, 1)
        h = eo.encoder_layer(sd, 0, x, mask, True, 2)
        unmasked = eo.final_norm(sd, h, None)
    assert torch.all(y[~mask] == 0) and bool((y[mask] != 0).any())
    assert torch.allclose(unmasked[~mask], torch.full_like(unmasked[~mask], 0.25))  # the planted mistake shows
    assert torch.equal(unmasked[mask], y[mask])


def test_sequence_subset_forward_equals_full_forward():
    """encoder_forward_sequences (whole-batch Linear layers, attention for the
    listed sequences only) gives the full forward's values on those sequences."""
    b, s_len, d, h, f, layers = 3, 16, 32, 4, 64, 2
    sd = eo.init_state_dict(d, h, f, layers, seed=5)
    x, _ = eo.generate_case(b, s_len, d, CPU, torch.float32, 6, 0.0)
    full = eo.encoder_forward(sd, x, None, False, h, layers, block_rows=4)
    sub = eo.encoder_forward_sequences(sd, x, (0, 2), False, h, layers, block_rows=4)
    torch.testing.assert_close(sub, full[[0, 2]], rtol=1e-5, atol=1e-6)
