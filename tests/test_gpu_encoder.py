"""End-to-end parity of the HIP encoder forward against the oracle on the GPU.

Weights come from the seeded default init of the package's BaselineTransformer
(the reference's construction order); inputs from generate_random_case.  The
oracle (oracle/encoder_oracle.py) runs the reference math with torch-ROCm ops on
the same device, and the candidate runs the C-ABI path.  The gate is the build's
bf16 tolerance: strict |d| < 1e-2 OR |d| < 1.6e-2 |ref| for every element.
"""

import time

import pytest
import torch

from oracle.encoder_oracle import compare, encoder_forward, encoder_forward_sequences
from tiktoktechjam2026track3_amd import native
from tiktoktechjam2026track3_amd.cases import (
    ENCODER_CONFIGS,
    OFFICIAL_TEST_CASES,
    TransformerConfig,
    generate_random_case,
)
from tiktoktechjam2026track3_amd.models import BaselineTransformer, UserOptimizedTransformer, copy_model_weights

pytestmark = pytest.mark.gpu

RTOL = 1.6e-2
ATOL = 1e-2


def build_models(config: TransformerConfig, seed: int, device):
    torch.manual_seed(seed)
    baseline = BaselineTransformer(config)
    candidate = UserOptimizedTransformer(config)
    copy_model_weights(baseline, candidate)
    sd = {k: v.to(device=device, dtype=torch.bfloat16) for k, v in baseline.state_dict().items()}
    candidate = candidate.to(device=device, dtype=torch.bfloat16).eval()
    return sd, candidate


def run_parity(name: str, device, trial: int = 0):
    spec = ENCODER_CONFIGS[name]
    cfg = spec.config
    sd, candidate = build_models(cfg, spec.seed, device)
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, spec.seed + trial, spec.padding_ratio, 1.0)
        out = candidate(x, mask)
        ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
        torch.cuda.synchronize()
    result = compare(ref, out, RTOL, ATOL)
    print(f"[parity] {name} trial {trial}: {result}", flush=True)
    return result, out, mask


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_encoder_parity(device, name):
    result, out, mask = run_parity(name, device)
    assert result["passed"], result
    if not bool(mask.all()):
        assert torch.all(out[~mask] == 0)


# Official cases: d_model 128 at head dims 32 (1-6, 12, 13), 128 (9), 64 (10)
# and 8 (11); d_model 32 at head dim 8 (7); d_model 1024 at head dim 256 (8).
# Case 14 is c5's shape (the slow test below).
OFFICIAL_COVERED = (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13)


@pytest.mark.parametrize("case_id", OFFICIAL_COVERED)
def test_encoder_parity_official_cases(device, case_id):
    """Four causal layers at the case's shape against the oracle, on the
    reference runner's default input (seed 1234, no padding) and on a padded
    variant; the bitwise share is printed for the record."""
    cfg = OFFICIAL_TEST_CASES[case_id - 1]
    sd, candidate = build_models(cfg, 1234, device)
    for padding in (0.0, 0.25):
        with torch.inference_mode():
            x, mask = generate_random_case(cfg, device, torch.bfloat16, 1234, padding, 1.0)
            out = candidate(x, mask)
            ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
            torch.cuda.synchronize()
        result = compare(ref, out, RTOL, ATOL)
        bitwise = float((ref.view(torch.int16) == out.view(torch.int16)).float().mean())
        print(f"[parity] official case {case_id} padding {padding}: {result} bitwise={bitwise:.6f}", flush=True)
        assert result["passed"], result
        if padding > 0:
            assert torch.all(out[~mask] == 0)


@pytest.mark.parametrize(
    "cfg",
    [TransformerConfig(3, 37, 128, 4, 64, 2, True), TransformerConfig(2, 45, 64, 2, 128, 2, False),
     TransformerConfig(2, 48, 64, 2, 128, 1, False), TransformerConfig(5, 19, 32, 1, 32, 3, True)],
    ids=["d128-f64-causal", "d64-f128", "d64-f128-whole-slabs", "d32-f32-causal"],
)
def test_encoder_parity_narrow_ragged(device, cfg):
    """Narrow models run the fused block tail (out_proj .. ffn_out in one
    kernel): token counts that leave a partial 16-row slab, d_model != ffn_dim,
    with and without padding, against the oracle bit for bit, on the capturing
    call and on two graph replays (a result read before its MFMA landed once
    showed up only on some calls)."""
    sd, candidate = build_models(cfg, 77, device)
    for padding in (0.0, 0.3):
        with torch.inference_mode():
            x, mask = generate_random_case(cfg, device, torch.bfloat16, 5, padding, 1.0)
            outs = [candidate(x, mask) for _ in range(3)]
            ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
            torch.cuda.synchronize()
        result = compare(ref, outs[0], RTOL, ATOL)
        assert result["passed"], result
        for out in outs:
            assert torch.equal(ref, out)


@pytest.mark.parametrize(
    "cfg",
    [TransformerConfig(1, 100, 256, 4, 512, 3, True), TransformerConfig(2, 64, 512, 8, 1024, 2, False),
     TransformerConfig(1, 256, 1024, 16, 1024, 2, True), TransformerConfig(3, 50, 2048, 16, 512, 2, False)],
    ids=["d256-ragged-causal", "d512", "d1024-256rows-causal", "d2048"],
)
def test_encoder_parity_few_row_models(device, cfg):
    """Up to 256 tokens with d_model 256-2048 every projection takes the
    few-row (16-row tile) kernels, split-K where the library splits: bit for
    bit the oracle, with and without padding (a partial last row block at 100
    and 150 tokens), on the capturing call and on two graph replays."""
    sd, candidate = build_models(cfg, 91, device)
    for padding in (0.0, 0.3):
        with torch.inference_mode():
            x, mask = generate_random_case(cfg, device, torch.bfloat16, 7, padding, 1.0)
            outs = [candidate(x, mask) for _ in range(3)]
            ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
            torch.cuda.synchronize()
        result = compare(ref, outs[0], RTOL, ATOL)
        print(f"[parity] few-row model {cfg} padding {padding}: {result}", flush=True)
        assert result["passed"], result
        for out in outs:
            assert torch.equal(ref, out)


def test_encoder_parity_second_trial_c4(device):
    result, _, _ = run_parity("c4", device, trial=1)
    assert result["passed"], result


# Every c5 sequence is checked: among them those whose element offsets pass
# 2^31 (activations and head-major Q/K beyond sequence 20), and the last, whose
# final ~18K rows are the library's stream-K tail tiles.
C5_SEQUENCES = tuple(range(32))


def _c5_sampled(device, causal: bool):
    spec = ENCODER_CONFIGS["c5"]
    cfg = spec.config
    sd, candidate = build_models(cfg, spec.seed, device)
    candidate.config = TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                                         cfg.num_layers, causal)
    name = "case 14 (causal c5)" if causal else "c5"
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, spec.seed, spec.padding_ratio, 1.0)
        t0 = time.perf_counter()
        picked = candidate(x, mask)[list(C5_SEQUENCES)]
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        print(f"[{name}] candidate forward done in {t1 - t0:.1f} s, finite={bool(torch.isfinite(picked).all())}",
              flush=True)
        candidate._hip.workspace = None  # room for the oracle's full-batch activations
        torch.cuda.empty_cache()
        ref = encoder_forward_sequences(sd, x, C5_SEQUENCES, causal, cfg.num_heads, cfg.num_layers)
        torch.cuda.synchronize()
        print(f"[{name}] oracle done in {time.perf_counter() - t1:.1f} s", flush=True)
    results = []
    for i, b in enumerate(C5_SEQUENCES):
        result = compare(ref[i], picked[i], RTOL, ATOL)
        bitwise = float((ref[i].view(torch.int16) == picked[i].view(torch.int16)).float().mean())
        results.append((b, result, bitwise))
    for b, result, bitwise in results:  # one verdict line per sequence, at the end
        print(f"[parity] {name} sequence {b}: passed={result['passed']} failed={result['failed']}/"
              f"{result['total']} max_abs_error={result['max_abs_error']} bitwise={bitwise:.6f}", flush=True)
    return results


def _summary(capsys, name, results):
    """One line past pytest's output capture: the driver's log tail shows it."""
    passed = sum(bool(r["passed"]) for _, r, _ in results)
    worst = max(r["max_abs_error"] for _, r, _ in results)
    bitwise = min(bw for _, _, bw in results)
    with capsys.disabled():
        print(f"\n[parity] {name}: {passed}/{len(results)} sequences pass the strict gate, "
              f"max_abs_error {worst}, bitwise share >= {bitwise:.6f}", flush=True)


@pytest.mark.slow
def test_encoder_parity_c5_sampled_sequences(device, capsys):
    """c5 (B=32, S=100000): the whole batch runs through the HIP forward; the
    oracle recomputes the sampled sequences over all layers, with its Linear
    layers on the whole [3.2M, 1024] batch as the reference runs them and its
    attention walking equal 1000-row query blocks (scores are never
    materialised for more rows than that).  All 32 sequences are held to the
    strict gate."""
    results = _c5_sampled(device, causal=False)
    _summary(capsys, "c5", results)
    for b, result, _ in results:
        assert result["passed"], (b, result)


@pytest.mark.slow
def test_encoder_parity_case14_causal_c5_sampled_sequences(device, capsys):
    """The reference's official case 14 (cases.py:56): c5's shape with a causal
    mask, which ran out of memory on the reference's GPU.  All 32 sequences,
    strict gate, as for c5."""
    results = _c5_sampled(device, causal=True)
    _summary(capsys, "case 14 (causal c5)", results)
    for b, result, _ in results:
        assert result["passed"], (b, result)


def test_graph_replay_matches_eager(device):
    spec = ENCODER_CONFIGS["c2"]
    cfg = spec.config
    sd, candidate = build_models(cfg, spec.seed, device)
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, 7, 0.0, 1.0)
        first = candidate(x, mask)  # capture
        assert candidate._cuda_graph is not None
        eager = candidate._forward_native(x, mask, "all_true")
        outs = []
        for i in range(4):
            outs.append(candidate(x, mask))
            torch.cuda.synchronize()
            _ = candidate._forward_native(x, mask, "all_true")  # eager work between replays
        for o in [first] + outs:
            assert torch.equal(o, eager)
        assert outs[0].data_ptr() != outs[1].data_ptr()  # independent clones
        # new input values through the same static buffer
        x.copy_(torch.randn_like(x))
        replayed = candidate(x, mask)
        eager2 = candidate._forward_native(x, mask, "all_true")
        assert torch.equal(replayed, eager2)
        ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
        assert compare(ref, replayed, RTOL, ATOL)["passed"]


def test_graph_survives_eager_call_at_another_shape(device):
    """A call at another sequence length runs eagerly and replaces the eager
    workspace; the captured graph must keep writing its own buffers, so the
    next replay at the captured shape still equals the eager forward."""
    spec = ENCODER_CONFIGS["c2"]
    cfg = spec.config
    _, candidate = build_models(cfg, spec.seed, device)
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, 11, 0.0, 1.0)
        candidate(x, mask)  # capture
        graph = candidate._cuda_graph
        assert graph is not None
        x_other = torch.randn(cfg.batch_size, cfg.seq_len + 64, cfg.d_model, device=device).bfloat16()
        other = candidate(x_other)  # eager, new workspace size
        torch.cuda.synchronize()
        assert candidate._cuda_graph is graph  # no recapture for the other shape
        filler = torch.full((64 * 1024 * 1024,), 7, dtype=torch.uint8, device=device)  # reuse freed memory
        replayed = candidate(x, mask)
        torch.cuda.synchronize()
        assert candidate._cuda_graph is graph
        eager = candidate._forward_native(x, mask, "all_true")
        assert torch.equal(replayed, eager)
        assert torch.equal(candidate._forward_native(x_other, None, "all_true"), other)
        del filler


def _unpacked_forward(candidate, x, mask=None):
    """The native forward from the plain weights only (no packed copies)."""
    cfg = candidate.config
    table, eps, packed = candidate._native_weights(x.device, 0)
    assert not packed
    b, s, d = x.shape
    workspace = torch.empty(native.encoder_workspace_bytes(b, s, d, cfg.num_heads, cfg.ffn_dim),
                            device=x.device, dtype=torch.uint8)
    out = torch.empty_like(x)
    kv_len = row_mask = None
    if mask is not None and not bool(mask.all()):
        kv_len = native.mask_lengths(mask)
        row_mask = mask.contiguous().view(torch.uint8)
    native.encoder_forward(x, out, workspace, table, cfg.num_heads, cfg.ffn_dim, cfg.num_layers, eps,
                           cfg.causal, kv_len, None, row_mask)
    return out


def test_encoder_packed_weights_bitwise_unpacked(device):
    """c4 (prefix padding, causal): the forward over the tile-packed weight
    copies equals the forward over the plain weights bit for bit."""
    spec = ENCODER_CONFIGS["c4"]
    cfg = spec.config
    _, candidate = build_models(cfg, spec.seed, device)
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, spec.seed + 5, spec.padding_ratio, 1.0)
        packed = candidate(x, mask)
        assert candidate._hip.packed is not None and len(candidate._hip.packed_views) == 4 * cfg.num_layers
        plain = _unpacked_forward(candidate, x, mask)
        torch.cuda.synchronize()
    mismatches = int((packed.view(torch.int16) != plain.view(torch.int16)).sum())
    print(f"[packed] c4: {mismatches} mismatches against the plain-weight forward", flush=True)
    assert mismatches == 0


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_packed_copies_follow_in_place_weight_updates(device, graph):
    """An in-place weight update after a forward is seen by the next forward:
    the packed copies are remade (eager), and the graph, whose kernels read
    them, is captured again."""
    cfg = TransformerConfig(1, 2048, 256, 4, 1024, 2, True)  # 2048 rows: packed, graph-eligible
    _, candidate = build_models(cfg, 13, device)
    seq = cfg.seq_len if graph else 1536  # another length runs eagerly
    g = torch.Generator(device=device).manual_seed(3)
    with torch.inference_mode():
        x = torch.randn(1, seq, cfg.d_model, generator=g, device=device).bfloat16()
        before = candidate(x)
        assert (candidate._cuda_graph is not None) == graph
        captures = candidate._cuda_graph_capture_count
        candidate.layers[1].ffn_in.weight.mul_(0.5)
        candidate.layers[0].attention.qkv_proj.weight.add_(0.01)
        after = candidate(x)
        torch.cuda.synchronize()
        plain = _unpacked_forward(candidate, x)
        torch.cuda.synchronize()
        if graph:
            assert candidate._cuda_graph_capture_count == captures + 1
            assert torch.equal(candidate(x), plain)  # replay of the new capture
    assert not torch.equal(before, after)
    assert torch.equal(after, plain)


def test_online_attention_encoder_stays_close(device):
    """The opt-in one-pass attention: its bf16 weight-rounding noise compounds
    over the layers, so it is held to a looser bound than the reference's gate
    (the exact default is what meets the gate)."""
    spec = ENCODER_CONFIGS["c3"]
    cfg = spec.config
    sd, candidate = build_models(cfg, spec.seed, device)
    candidate.online_attention = True
    with torch.inference_mode():
        x, mask = generate_random_case(cfg, device, torch.bfloat16, spec.seed, spec.padding_ratio, 1.0)
        out = candidate(x, mask)
        ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
    result = compare(ref, out, RTOL, ATOL)
    print(f"[parity] c3 online attention: {result}", flush=True)
    assert result["max_abs_error"] < 0.25
    assert result["failed"] < 0.01 * result["total"]


def test_native_only_rejects_a_float32_input(device):
    cfg = TransformerConfig(1, 16, 512, 8, 1024, 1, False)
    model = UserOptimizedTransformer(cfg).to(device).eval()
    model.native_only = True
    with torch.inference_mode(), pytest.raises(NotImplementedError, match="bfloat16"):
        model(torch.randn(1, 16, 512, device=device))
    assert model.native_calls == 0


def test_float32_on_the_gpu_takes_the_logged_torch_fallback(device):
    # the reference's native fallback for non-BF16 inputs (TECHNICAL_REPORT.md:542-548)
    cfg = TransformerConfig(2, 24, 512, 8, 1024, 2, True)
    torch.manual_seed(7)
    baseline = BaselineTransformer(cfg)
    candidate = UserOptimizedTransformer(cfg)
    copy_model_weights(baseline, candidate)
    baseline = baseline.to(device).eval()
    candidate = candidate.to(device).eval()
    candidate.native_only = False
    x, mask = generate_random_case(cfg, device, torch.float32, 5, 0.5, 1.0)
    with torch.inference_mode():
        ref = baseline(x, mask)
        out = candidate(x, mask)
    assert candidate.native_calls == 0 and sum(candidate.fallback_calls.values()) == 1
    assert "bfloat16" in next(iter(candidate.fallback_calls))
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5), float((out - ref).abs().max())


def test_grad_enabled_call_records_autograd_history(device):
    # the kernels record no history: a training call runs the torch ops and
    # its gradients are the baseline's
    cfg = TransformerConfig(1, 16, 128, 4, 256, 1, False)
    torch.manual_seed(3)
    baseline = BaselineTransformer(cfg)
    candidate = UserOptimizedTransformer(cfg)
    copy_model_weights(baseline, candidate)
    baseline = baseline.to(device=device, dtype=torch.float32)
    candidate = candidate.to(device=device, dtype=torch.float32)
    candidate.native_only = False
    x = torch.randn(1, 16, 128, device=device)
    out = candidate(x)
    ref = baseline(x)
    assert out.requires_grad and out.grad_fn is not None
    out.float().square().sum().backward()
    ref.float().square().sum().backward()
    assert "autograd" in next(iter(candidate.fallback_calls))
    g_ref = baseline.layers[0].ffn_in.weight.grad
    g_out = candidate.layers[0].ffn_in.weight.grad
    assert torch.allclose(g_out, g_ref, rtol=1e-4, atol=1e-5)
    # the same module under inference mode takes the native forward again
    candidate = candidate.to(dtype=torch.bfloat16).eval()
    with torch.inference_mode():
        candidate(x.bfloat16())
    assert candidate.native_calls == 1


def test_general_mask_parity(device):
    cfg = TransformerConfig(2, 200, 512, 8, 1024, 2, True)
    sd, candidate = build_models(cfg, 3, device)
    g = torch.Generator(device=device).manual_seed(1)
    with torch.inference_mode():
        x = torch.randn(2, 200, 512, generator=g, device=device).bfloat16()
        mask = torch.rand(2, 200, generator=g, device=device) > 0.3
        mask[:, 0] = True
        x = x.masked_fill(~mask[..., None], 0)
        assert candidate._mask_kind(mask) == "general"
        out = candidate(x, mask)
        ref = encoder_forward(sd, x, mask, cfg.causal, cfg.num_heads, cfg.num_layers)
    result = compare(ref, out, RTOL, ATOL)
    assert result["passed"], result
    assert torch.all(out[~mask] == 0)
