"""Pin the product's harness against the reference's own values (CPU).

tests/test_oracle.py pins the oracle's copies of these functions; the tests
here hold the package that the CLI, the bench and every GPU test actually run
to the same fixtures (tests/golden/reference_vectors.*, written by running the
reference's Python in this container):

  * ``models.BaselineTransformer`` seeded default init, per parameter sha256,
    for the tiny shapes and all five measurement configurations (pins the
    module construction order, models.py:20-33, 719-725, 896-907);
  * ``cases.generate_random_case`` on CPU (the RNG call order, cases.py:60-98);
  * the baseline and the candidate's CPU forwards (models.py:909-919);
  * ``correctness.compare_outputs`` verdicts (correctness.py:40-109) and
    ``timing.percentile`` values (timing.py:17-30);
  * the facade's export list (torch_transformer_benchmark.py:64-123).
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import torch_transformer_benchmark as facade
from tiktoktechjam2026track3_amd import cases, correctness, models, timing
from tiktoktechjam2026track3_amd.cases import TransformerConfig

GOLDEN = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLDEN / "reference_vectors.json").read_text())
ARR = np.load(GOLDEN / "reference_vectors.npz", allow_pickle=False)
CPU = torch.device("cpu")


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().float().numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("name", sorted(META["weights"]))
def test_baseline_init_matches_reference(name):
    entry = META["weights"][name]
    torch.manual_seed(entry["seed"])
    model = models.BaselineTransformer(TransformerConfig(*entry["config"]))
    sd = model.state_dict()
    assert list(sd) == list(entry["params"]), "parameter names or order differ"
    for key, ref in entry["params"].items():
        assert list(sd[key].shape) == ref["shape"], key
        assert sha(sd[key]) == ref["sha256_fp32"], key


def test_candidate_receives_the_baseline_weights():
    # runner order: seed, baseline, candidate, strict copy (runner.py:304-326)
    entry = META["weights"]["c2"]
    config = TransformerConfig(*entry["config"])
    torch.manual_seed(entry["seed"])
    baseline = models.BaselineTransformer(config)
    candidate = models.UserOptimizedTransformer(config)
    models.copy_model_weights(baseline, candidate)
    for i in range(config.num_layers):
        packed = candidate.layers[i].attention.qkv_proj.weight
        for j, part in enumerate(("q", "k", "v")):
            key = f"layers.{i}.attention.{part}_proj.weight"
            d = config.d_model
            assert sha(packed[j * d:(j + 1) * d]) == entry["params"][key]["sha256_fp32"], key
        key = f"layers.{i}.ffn_out.weight"
        assert sha(candidate.layers[i].ffn_out.weight) == entry["params"][key]["sha256_fp32"], key


@pytest.mark.parametrize("name", sorted(META["inputs"]))
def test_generate_random_case_matches_reference(name):
    entry = META["inputs"][name]
    config = TransformerConfig(*entry["config"])
    x, mask = cases.generate_random_case(
        config, CPU, torch.float32, entry["seed"], entry["padding_ratio"], entry["input_scale"])
    assert sha(x) == entry["x"]["sha256_fp32"]
    assert mask.sum(1).tolist() == entry["lengths"]
    if f"in/{name}/x" in ARR:
        assert np.array_equal(ARR[f"in/{name}/x"], x.numpy())
        assert np.array_equal(ARR[f"in/{name}/mask"], mask.numpy())
    else:
        assert np.array_equal(ARR[f"in/{name}/x_row0"], x[0, :4].numpy())


def _forward(name, candidate: bool):
    entry = META["forward"][name]
    config = TransformerConfig(*entry["config"])
    dtype = torch.float32 if entry["dtype"] == "torch.float32" else torch.bfloat16
    torch.manual_seed(entry["weight_seed"])
    model = models.BaselineTransformer(config)
    if candidate:
        other = models.UserOptimizedTransformer(config)
        models.copy_model_weights(model, other)
        model = other
    model = model.to(dtype=dtype).eval()
    x, mask = cases.generate_random_case(config, CPU, dtype, entry["input_seed"], entry["padding_ratio"], 1.0)
    with torch.inference_mode():
        return entry, model(x, mask)


@pytest.mark.parametrize("candidate", [False, True], ids=["baseline", "candidate"])
@pytest.mark.parametrize("name", [n for n in META["forward"] if n != "c1"])
def test_forward_matches_reference_tiny(name, candidate):
    entry, y = _forward(name, candidate)
    ref = torch.from_numpy(ARR[f"fwd/{name}/y"])
    if entry["dtype"] == "torch.float32":
        assert torch.allclose(y, ref, rtol=1e-5, atol=1e-5)
    else:
        assert torch.equal(y.float(), ref), float((y.float() - ref).abs().max())


@pytest.mark.parametrize("candidate", [False, True], ids=["baseline", "candidate"])
def test_forward_matches_reference_c1(candidate):
    entry, y = _forward("c1", candidate)
    rows = entry["sample_rows"]
    assert torch.allclose(y[:, rows, :], torch.from_numpy(ARR["fwd/c1/y_rows"]), rtol=1e-5, atol=1e-5)
    assert abs(float(y.double().sum()) - entry["y"]["sum"]) < 1e-3


@pytest.mark.parametrize("index", range(len(META["compare"])))
def test_compare_outputs_matches_reference(index):
    case = META["compare"][index]
    ref = torch.tensor(case["ref"])
    opt = torch.tensor(case["opt"])
    result = correctness.compare_outputs(ref, opt, rtol=case["rtol"], atol=case["atol"])
    assert result.passed == case["passed"]
    assert result.failed_elements == case["failed_elements"]
    assert result.failed_feature_dims == case["failed_feature_dims"]


@pytest.mark.parametrize("index", range(len(META["percentile"])))
def test_percentile_matches_reference(index):
    case = META["percentile"][index]
    assert timing.percentile(case["values"], case["q"]) == case["result"]


# the reference facade's __all__ (torch_transformer_benchmark.py:80-123): the
# names a caller may import from it
REFERENCE_FACADE_NAMES = [
    "AccuracyResult", "AccuracySummary", "BaselineSelfAttention", "BaselineTransformer",
    "BaselineTransformerBlock", "OFFICIAL_TEST_CASES", "PROFILE_CANDIDATE_REPLAYS", "PROFILE_MAX_CASES",
    "PROFILE_MAX_EVENTS", "PROFILE_WARMUP_REPLAYS", "TimingResult", "TransformerConfig",
    "UserOptimizedTransformer", "benchmark_models", "benchmark_once", "compare_outputs", "config_from_args",
    "configure_runtime", "copy_model_weights", "environment_metadata", "execution_failed_result",
    "generate_random_case", "is_out_of_memory_error", "main", "maybe_compile", "official_case_result",
    "parse_args", "percentile", "profile_candidate", "release_case_memory", "resolve_device", "resolve_dtype",
    "run_accuracy_tests", "run_benchmark_case", "run_official_matrix", "run_single_case", "settings_metadata",
    "summarize_profile_events", "validate_args", "warmup_model", "write_json_document", "write_json_result",
    "write_matrix_result",
]


def test_facade_exports_every_reference_name():
    assert len(REFERENCE_FACADE_NAMES) == 43
    missing = [n for n in REFERENCE_FACADE_NAMES if n not in facade.__all__ or not hasattr(facade, n)]
    assert not missing, missing
    assert facade.TimingResult is timing.TimingResult
    assert callable(facade.profile_candidate) and callable(facade.summarize_profile_events)
