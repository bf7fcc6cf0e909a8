"""CLI drop-in: flags, JSON schemas, failure classification and exit codes.

The result documents must pass the structural checks the reference's unchanged
benchmarkctl applies before it accepts a job (orchestrator/crates/benchmarkctl/
src/main.rs:1155-1240), restated in ``benchmarkctl_summary`` below.  Everything
runs on the CPU with tiny shapes.
"""

import json
import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from tiktoktechjam2026track3_amd import runner
from tiktoktechjam2026track3_amd.cases import ENCODER_CONFIGS, TransformerConfig
from tiktoktechjam2026track3_amd.models import UnsupportedShapeError

ROOT = Path(__file__).resolve().parent.parent
CPU = torch.device("cpu")
TINY = ["--device", "cpu", "--dtype", "float32", "--accuracy-trials", "1", "--warmup", "0",
        "--repeats", "2", "--benchmark-rounds", "1"]


def benchmarkctl_summary(doc):
    """The acceptance checks of benchmarkctl's read_result_summary."""
    assert isinstance(doc.get("schema_version"), int)
    if doc["schema_version"] == 1:
        for field in ("config", "environment", "settings", "accuracy"):
            assert isinstance(doc.get(field), dict), field
        assert doc.get("performance") is None or isinstance(doc["performance"], dict)
        assert isinstance(doc.get("correctness_passed"), bool)
        return {"mode": "single_case", "correctness_passed": doc["correctness_passed"]}
    assert doc["schema_version"] == 2
    assert doc.get("mode") == "official_matrix"
    for field in ("environment", "settings"):
        assert isinstance(doc.get(field), dict), field
    requested = doc["requested_case_ids"]
    assert requested and all(isinstance(c, int) for c in requested)
    cases = doc["cases"]
    assert isinstance(doc["complete"], bool) and isinstance(doc["all_cases_executed"], bool)
    assert doc["complete"] == (len(cases) == len(requested))
    assert not doc["all_cases_executed"] or doc["complete"]
    passed = doc["correctness_passed"]
    assert passed is None or isinstance(passed, bool)
    if passed is True:
        assert doc["complete"] and doc["all_cases_executed"]
    assert doc["failure_category"] is None or isinstance(doc["failure_category"], str)
    return {"mode": "official_matrix", "correctness_passed": passed}


def test_flags_and_defaults_follow_the_reference():
    args = runner.parse_args([])
    assert args.official_matrix and args.official_cases is None
    assert (args.batch_size, args.seq_len, args.d_model, args.heads, args.ffn_dim, args.layers) == (8, 128, 512, 8, 2048, 6)
    assert (args.rtol, args.atol, args.seed) == (0.02, 0.002, 1234)
    assert (args.warmup, args.repeats, args.benchmark_rounds, args.accuracy_trials) == (20, 100, 3, 5)
    assert args.dtype == "bfloat16" and args.device == "auto" and args.allow_tf32
    args = runner.parse_args(["--encoder-configs", "all"])
    assert args.encoder_configs == sorted(ENCODER_CONFIGS)


@pytest.mark.parametrize("argv, message", [
    (["--official-cases", "15"], "invalid official case IDs"),
    (["--official-cases", "2", "2"], "duplicates"),
    (["--no-official-matrix", "--official-cases", "2"], "requires --official-matrix"),
    (["--no-official-matrix", "--padding-ratio", "1.0"], "padding_ratio"),
    (["--no-official-matrix", "--repeats", "0"], "repeats"),
    (["--encoder-configs", "c9"], "unknown encoder"),
    ([], "requires a GPU"),
    (["--official-cases", "2", "--profile-candidate"], "requires a GPU"),
    (["--no-official-matrix", "--profile-candidate"], "focused case list"),
])
def test_validation_rejects_bad_arguments(argv, message):
    args = runner.parse_args(argv)
    with pytest.raises(ValueError, match=message):
        runner.validate_args(args, CPU, torch.float32)


def test_single_case_cli_writes_schema_1_and_exits_0(tmp_path):
    out = tmp_path / "single.json"
    cmd = [sys.executable, str(ROOT / "torch_transformer_benchmark.py"), "--no-official-matrix", *TINY,
           "--batch-size", "2", "--seq-len", "16", "--d-model", "32", "--heads", "2", "--ffn-dim", "64",
           "--layers", "1", "--causal", "--padding-ratio", "0.25", "--cpu-baseline-seconds", "0.2",
           "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "single_case", "correctness_passed": True}
    assert doc["config"]["causal"] is True and doc["settings"]["accuracy_rule"] == "strict_less_than_or"
    perf = doc["performance"]
    assert perf["optimized"]["median_ms"] > 0 and len(perf["optimized"]["samples_ms"]) == 2
    assert perf["cpu_baseline"]["unit"] == "tokens/s" and perf["cpu_baseline"]["value"] > 0
    assert not list(tmp_path.glob(".*.tmp"))  # atomic write leaves no temporary


def test_encoder_config_c1_runs_as_a_schema_2_matrix(tmp_path):
    out = tmp_path / "c1.json"
    args = runner.parse_args(["--encoder-configs", "c1", *TINY, "--json-output", str(out)])
    runner.validate_args(args, CPU, torch.float32)
    assert runner.run_encoder_configs(args, CPU, torch.float32) == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    (case,) = doc["cases"]
    assert case["case_id"] == 1 and case["status"] == "succeeded"
    assert case["config"] == {"batch_size": 2, "seq_len": 128, "d_model": 256, "num_heads": 4,
                              "ffn_dim": 1024, "num_layers": 2, "causal": False}
    assert doc["case_set"] == "mi355x_encoder_configs_c1_c5"


def test_matrix_classifies_out_of_memory_and_unsupported_shapes(tmp_path, monkeypatch):
    out = tmp_path / "matrix.json"
    calls = []

    def fake_case(config, args, device, dtype):
        calls.append(config)
        if len(calls) == 1:
            raise RuntimeError("HIP out of memory. Tried to allocate 12.00 GiB")
        raise UnsupportedShapeError("unsupported encoder shape: head_dim 16 (supported: 8, 32, 64, 128, 256)")

    monkeypatch.setattr(runner, "_run_benchmark_case_with_profile", fake_case)
    args = runner.parse_args(["--official-cases", "14", "2", "--device", "cpu", "--json-output", str(out)])
    rc = runner.run_official_matrix(args, CPU, torch.float32)
    assert rc == 3
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc)["correctness_passed"] is None
    assert doc["complete"] and not doc["all_cases_executed"] and doc["failure_category"] == "execution"
    first, second = doc["cases"]
    assert first["case_id"] == 14 and first["failure_category"] == "out_of_memory"
    assert second["status"] == "execution_failed" and second["failure_category"] == "unsupported_shape"


def test_matrix_other_runtime_errors_propagate(monkeypatch):
    def broken(config, args, device, dtype):
        raise RuntimeError("kernel launch failed")

    monkeypatch.setattr(runner, "_run_benchmark_case_with_profile", broken)
    args = runner.parse_args(["--official-cases", "2", "--device", "cpu"])
    with pytest.raises(RuntimeError, match="kernel launch failed"):
        runner.run_official_matrix(args, CPU, torch.float32)


def test_correctness_failure_exits_2_and_skips_timing(tmp_path, monkeypatch):
    from tiktoktechjam2026track3_amd import models

    real_forward = models.UserOptimizedTransformer.forward

    def wrong(self, x, mask=None):
        return real_forward(self, x, mask) + 1.0

    monkeypatch.setattr(models.UserOptimizedTransformer, "forward", wrong)
    out = tmp_path / "fail.json"
    args = runner.parse_args(["--no-official-matrix", *TINY, "--batch-size", "1", "--seq-len", "8",
                              "--d-model", "16", "--heads", "2", "--ffn-dim", "32", "--layers", "1",
                              "--json-output", str(out)])
    assert runner.run_single_case(args, CPU, torch.float32) == 2
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc)["correctness_passed"] is False
    assert doc["performance"] is None


def test_json_documents_have_no_non_finite_numbers(tmp_path):
    path = tmp_path / "doc.json"
    runner.write_json_document(path, {"a": float("nan"), "b": [1.0, float("inf")], "c": {"d": -math.inf}})
    assert json.loads(path.read_text()) == {"a": None, "b": [1.0, None], "c": {"d": None}}


def test_roofline_uses_algorithmic_flops():
    cfg = TransformerConfig(8, 1024, 1024, 16, 4096, 4, True)
    assert runner.forward_flops(cfg) == pytest.approx(0.893e12, rel=1e-3)
    perf = {"optimized": {"median_ms": 1.0}}
    roof = runner.roofline_summary(cfg, perf)
    assert roof["tokens_per_second"] == pytest.approx(8192 * 1000.0)
    assert roof["fraction_of_bf16_mfma_peak"] == pytest.approx(runner.forward_flops(cfg) / 1e-3 / 2.5e15)
