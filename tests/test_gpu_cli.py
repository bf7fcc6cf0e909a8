"""The CLI drop-in on the GPU: measurement configurations through the native
forward, the accuracy gate of the reference, timing, roofline and the bounded
candidate profile, written as a benchmarkctl-compatible schema 2 document."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

from tests.test_runner import benchmarkctl_summary

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def test_cli_encoder_configs_c2_c3_pass_the_gate_with_profile(tmp_path):
    out = tmp_path / "result.json"
    cmd = [sys.executable, "-u", str(ROOT / "torch_transformer_benchmark.py"), "--encoder-configs", "c2", "c3",
           "--rtol", "1.6e-2", "--atol", "1e-2", "--accuracy-trials", "2", "--warmup", "3", "--repeats", "10",
           "--benchmark-rounds", "2", "--profile-candidate", "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    print(proc.stdout[-3000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    assert doc["requested_case_ids"] == [2, 3]
    for case in doc["cases"]:
        assert case["status"] == "succeeded"
        assert case["accuracy"]["failed_elements"] == 0
        roof = case["performance"]["roofline"]
        assert 0 < roof["fraction_of_bf16_mfma_peak"] < 1
        profile = case["candidate_profile"]
        assert profile["profiled_replays"] == 3 and len(profile["replay_wall_time"]["samples_ms"]) == 3
    assert doc["environment"]["compute_units"] > 0


def test_cli_official_cases_at_head_dims_8_to_256_pass(tmp_path):
    """Official cases 2 (head dim 32), 8 (256), 9 (128), 10 (64), 11 (8) and
    12 (32, 32 tokens) with the reference runner's default gate and inputs."""
    out = tmp_path / "official.json"
    cmd = [sys.executable, "-u", str(ROOT / "torch_transformer_benchmark.py"), "--official-cases", "2", "8", "9",
           "10", "11", "12", "--accuracy-trials", "2", "--warmup", "2", "--repeats", "5", "--benchmark-rounds", "1",
           "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    print(proc.stdout[-3000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    assert doc["requested_case_ids"] == [2, 8, 9, 10, 11, 12]
    for case in doc["cases"]:
        assert case["status"] == "succeeded"
        assert case["accuracy"]["failed_elements"] == 0


def test_cli_remaining_official_cases_1_to_13_pass(tmp_path):
    """With the test above, cases 1-13 of the official matrix through the CLI:
    1, 3-6 and 13 (head dim 32 at 1 to 10000 sequences and 1024 tokens) and 7
    (d_model 32, head dim 8).  Case 14 is c5's shape, whose baseline cannot
    materialise its scores; the encoder tests cover it."""
    out = tmp_path / "official.json"
    cmd = [sys.executable, "-u", str(ROOT / "torch_transformer_benchmark.py"), "--official-cases", "1", "3", "4",
           "5", "6", "7", "13", "--accuracy-trials", "1", "--warmup", "2", "--repeats", "3", "--benchmark-rounds",
           "1", "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    print(proc.stdout[-3000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    for case in doc["cases"]:
        assert case["status"] == "succeeded"
        assert case["accuracy"]["failed_elements"] == 0


def test_cli_encoder_config_c1_on_the_gpu_box(tmp_path):
    """c1 (B=2, S=128, D=256, H=4, FFN=1024, L=2, fp32, seed 0) is the
    reference's CPU smoke case: on the GPU box the CLI still runs it through
    the candidate's CPU path (the reference's CPU fallback contract) and holds
    it to the reference gate against the baseline, bit for bit."""
    out = tmp_path / "c1.json"
    cmd = [sys.executable, "-u", str(ROOT / "torch_transformer_benchmark.py"), "--encoder-configs", "c1",
           "--rtol", "1.6e-2", "--atol", "1e-2", "--accuracy-trials", "2", "--warmup", "1", "--repeats", "3",
           "--benchmark-rounds", "1", "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    print(proc.stdout[-3000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    (case,) = doc["cases"]
    assert case["status"] == "succeeded"
    assert case["accuracy"]["failed_elements"] == 0 and case["accuracy"]["max_abs_error"] == 0.0
    assert case["config"]["d_model"] == 256 and case["config"]["num_layers"] == 2
    print(f"[c1] {json.dumps(case['accuracy'])}", flush=True)


def test_cli_profile_candidate_with_rocprof_evidence(tmp_path):
    """--profile-candidate --rocprof on c2 and c3: rocprofv3 child processes
    (kernel trace, FETCH_SIZE, WRITE_SIZE, MFMA busy) replay the focused cases
    before the CLI touches the GPU; each case's profile then carries per-kernel
    time, HBM bytes and GB/s and MFMA utilisation of the HIP kernels."""
    out = tmp_path / "result.json"
    cmd = [sys.executable, "-u", str(ROOT / "torch_transformer_benchmark.py"), "--encoder-configs", "c2", "c3",
           "--rtol", "1.6e-2", "--atol", "1e-2", "--accuracy-trials", "1", "--warmup", "2", "--repeats", "5",
           "--benchmark-rounds", "1", "--profile-candidate", "--rocprof", "--rocprof-dir", str(tmp_path / "prof"),
           "--rocprof-timeout", "240", "--json-output", str(out)]
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=900)
    print(proc.stdout[-3000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    doc = json.loads(out.read_text())
    assert benchmarkctl_summary(doc) == {"mode": "official_matrix", "correctness_passed": True}
    for case in doc["cases"]:
        roc = case["candidate_profile"]["rocprof"]
        names = [k["kernel"] for k in roc["kernels"]]
        print(case["case_id"], [(k["name"][:40], k["calls"], round(k["avg_us"], 2), k["mfma_busy"],
                                 k["hbm_gbps"]) for k in roc["kernels"][:6]], flush=True)
        assert any("attn_fwd_kernel" in n for n in names)
        assert any("gemm" in n for n in names)
        assert not any("spin_kernel" in n or "copyBuffer" in n for n in names)
        assert 0 < roc["calibration"]["fetch_bytes_per_unit"] and 0 < roc["calibration"]["write_bytes_per_unit"]
        layers = case["config"]["num_layers"]
        attn = next(k for k in roc["kernels"] if "attn_fwd_kernel" in k["kernel"])
        assert attn["calls"] == 3 * layers  # three profiled forwards, one attention launch per layer
        gemm = max((k for k in roc["kernels"] if "gemm" in k["kernel"]), key=lambda k: k["total_ms"])
        assert 0 < gemm["mfma_busy"] <= 1
        assert gemm["hbm_gbps"] > 0 and gemm["fetched_bytes_per_call"] > 0
