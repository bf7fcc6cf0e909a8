"""Command line, orchestration and JSON results of the encoder benchmark.

Drop-in for transformer_benchmark/runner.py of the reference: the same flags
(runner.py:80-158), the same validation (:161-207), seeding and model build
order (:304-333: seed, baseline built first, candidate, strict weight copy,
then .to(device, dtype).eval()), accuracy then timing then the optional
bounded profile (:341-396), JSON schema 1 for one case and 2 for a matrix,
written atomically after every case (:261-293, :463-499), out-of-memory
classified as an execution failure (:502-531) and exit codes 0 / 2 / 3
(:544-559), so the reference's unchanged benchmarkctl can drive it.

Additions for this build, none of which changes the fields benchmarkctl
validates:
  * ``--encoder-configs c1 .. c5`` runs the five measurement configurations
    (shape, dtype, device, causal/padding, seed per configuration) as a
    schema 2 matrix with case ids 1..5;
  * every timed case reports ``roofline``: algorithmic FLOPs per forward,
    tokens/s and the fraction of MI355X dense bf16 MFMA peak at the
    candidate's median latency;
  * ``--cpu-baseline-seconds N`` times the baseline forward on the host CPU
    for about N seconds on one sequence of the case (sequences are
    independent, so tokens/s carries over) and reports it beside the GPU
    figure; a sequence too long for the host is reported as not run, with
    the reason;
  * a shape the HIP kernels do not cover is a case result with status
    ``execution_failed`` and failure category ``unsupported_shape``;
  * ``--profile-candidate --rocprof`` adds rocprofv3 evidence per kernel
    (time, HBM bytes and GB/s, MFMA utilisation) to each focused case's
    bounded profile, under ``candidate_profile.rocprof``; the profiled
    program runs as child processes started before this process touches the
    GPU (``--rocprof-child`` is their mode).
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import platform
import sys
import tempfile
import time
from dataclasses import asdict
from pathlib import Path
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from .cases import ENCODER_CONFIGS, OFFICIAL_TEST_CASES, TransformerConfig, generate_random_case
from .correctness import AccuracySummary, run_accuracy_tests
from .models import BaselineTransformer, UnsupportedShapeError, UserOptimizedTransformer, copy_model_weights
from .profiling import (
    PROFILE_CANDIDATE_REPLAYS,
    PROFILE_MAX_CASES,
    PROFILE_MAX_EVENTS,
    PROFILE_WARMUP_REPLAYS,
    ROCPROF_PASSES,
    calibration_copy,
    profile_candidate,
    region_marker,
    run_rocprof_passes,
    summarize_rocprof,
)
from .timing import benchmark_models, warmup_model

MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
ENCODER_CONFIG_NAMES = tuple(sorted(ENCODER_CONFIGS))


def resolve_device(device_arg: str) -> torch.device:
    """`--device`: "auto" takes the GPU when one is visible, else the CPU; an
    explicit GPU device without a visible GPU is an error (reference
    runner.py:48-54)."""
    have_gpu = torch.cuda.is_available()
    chosen = torch.device(("cuda" if have_gpu else "cpu") if device_arg == "auto" else device_arg)
    if chosen.type == "cuda" and not have_gpu:
        raise RuntimeError(f"--device {device_arg} needs a GPU, and torch.cuda.is_available() is False")
    return chosen


def resolve_dtype(dtype_name: str) -> torch.dtype:
    return {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[dtype_name]


def release_case_memory(device: torch.device) -> None:
    """Between cases: collect the finished case's objects, and on a GPU return
    the caching allocator's free blocks, so the next case starts from the
    device's full memory (reference runner.py:66-69)."""
    gc.collect()
    if device.type != "cuda":
        return
    torch.cuda.empty_cache()


def maybe_compile(model: nn.Module, enabled: bool, mode: str) -> nn.Module:
    """`--compile-baseline` / `--compile-user`: wrap the model in torch.compile
    with the chosen mode (reference runner.py:72-77)."""
    compile_fn = getattr(torch, "compile", None) if enabled else None
    if enabled and compile_fn is None:
        raise RuntimeError("--compile-* needs torch.compile, which this PyTorch build lacks")
    return compile_fn(model, mode=mode) if enabled else model


def parse_args(argv: Optional[Sequence[str]] = None) -> argparse.Namespace:
    parser = argparse.ArgumentParser(description="Compare a baseline and an MI355X-native Transformer encoder")
    parser.add_argument("--official-matrix", action=argparse.BooleanOptionalAction, default=True,
                        help="run the declared 14-case matrix (enabled by default)")
    parser.add_argument("--official-cases", type=int, nargs="+", metavar="ID",
                        help="run only these one-based official case IDs")
    parser.add_argument("--encoder-configs", nargs="+", metavar="NAME",
                        help=f"run these measurement configurations ({', '.join(ENCODER_CONFIG_NAMES)} or all)")
    parser.add_argument("--batch-size", type=int, default=8)
    parser.add_argument("--seq-len", type=int, default=128)
    parser.add_argument("--d-model", type=int, default=512)
    parser.add_argument("--heads", type=int, default=8)
    parser.add_argument("--ffn-dim", type=int, default=2048)
    parser.add_argument("--layers", type=int, default=6)
    parser.add_argument("--causal", action="store_true")
    parser.add_argument("--device", default="auto", help="auto, cpu, cuda, cuda:0, ...")
    parser.add_argument("--dtype", choices=("float32", "float16", "bfloat16"), default="bfloat16")
    parser.add_argument("--padding-ratio", type=float, default=0.0)
    parser.add_argument("--input-scale", type=float, default=1.0)
    parser.add_argument("--accuracy-trials", type=int, default=5)
    parser.add_argument("--rtol", type=float, default=0.02)
    parser.add_argument("--atol", type=float, default=0.002)
    parser.add_argument("--seed", type=int, default=1234)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--repeats", type=int, default=100)
    parser.add_argument("--benchmark-rounds", type=int, default=3)
    parser.add_argument("--benchmark-on-failure", action="store_true")
    parser.add_argument("--profile-candidate", action="store_true",
                        help="after correctness and timing, collect a bounded candidate-only profile "
                             "for an explicit focused case list")
    parser.add_argument("--rocprof", action="store_true",
                        help="with --profile-candidate, also collect rocprofv3 kernel time, HBM traffic and "
                             "MFMA utilisation per kernel (child processes, one per counter pass)")
    parser.add_argument("--rocprof-dir", type=Path,
                        help="directory for the rocprofv3 runs (default: a new temporary directory)")
    parser.add_argument("--rocprof-timeout", type=float, default=900.0,
                        help="seconds each rocprofv3 pass may take")
    parser.add_argument("--rocprof-child", action="store_true", help=argparse.SUPPRESS)
    parser.add_argument("--compile-baseline", action="store_true")
    parser.add_argument("--compile-user", action="store_true")
    parser.add_argument("--compile-mode", choices=("default", "reduce-overhead", "max-autotune"), default="default")
    parser.add_argument("--non-strict-weight-copy", action="store_true")
    parser.add_argument("--matmul-precision", choices=("highest", "high", "medium"), default="high")
    parser.add_argument("--allow-tf32", action=argparse.BooleanOptionalAction, default=True,
                        help="enable/disable TF32 for both implementations")
    parser.add_argument("--cpu-baseline-seconds", type=float, default=0.0,
                        help="also time the baseline on the host CPU for about this many seconds")
    parser.add_argument("--json-output", type=Path, help="write a versioned machine-readable result to this path")
    args = parser.parse_args(argv)
    if args.encoder_configs and "all" in args.encoder_configs:
        args.encoder_configs = list(ENCODER_CONFIG_NAMES)
    return args


def validate_args(args: argparse.Namespace, device: torch.device, dtype: torch.dtype) -> None:
    if args.encoder_configs:
        unknown = sorted(set(args.encoder_configs) - set(ENCODER_CONFIG_NAMES))
        if unknown:
            raise ValueError(f"unknown encoder configurations: {unknown}")
        if len(set(args.encoder_configs)) != len(args.encoder_configs):
            raise ValueError("--encoder-configs must not contain duplicates")
        if args.official_cases:
            raise ValueError("--encoder-configs and --official-cases are exclusive")
    if args.official_cases and not args.official_matrix:
        raise ValueError("--official-cases requires --official-matrix")
    if args.official_cases:
        invalid = sorted({c for c in args.official_cases if not 1 <= c <= len(OFFICIAL_TEST_CASES)})
        if invalid:
            raise ValueError(f"invalid official case IDs: {invalid}")
        if len(set(args.official_cases)) != len(args.official_cases):
            raise ValueError("--official-cases must not contain duplicates")
    if (args.official_matrix and not args.encoder_configs and args.official_cases is None
            and device.type != "cuda"):
        raise ValueError(
            "the full official matrix requires a GPU; use --official-cases for a "
            "CPU subset or --no-official-matrix for a custom CPU smoke test"
        )
    validate_profile_focus(args)
    if args.profile_candidate:
        if device.type != "cuda" and not args.encoder_configs:
            raise ValueError("--profile-candidate requires a GPU device")
        if args.benchmark_on_failure:
            raise ValueError("--profile-candidate cannot be combined with --benchmark-on-failure")
    if not 0.0 <= args.padding_ratio < 1.0:
        raise ValueError("padding_ratio must be in [0, 1)")
    if args.input_scale <= 0:
        raise ValueError("input_scale must be positive")
    if args.accuracy_trials <= 0:
        raise ValueError("accuracy_trials must be positive")
    if args.rtol < 0 or args.atol < 0:
        raise ValueError("rtol and atol must be non-negative")
    if args.warmup < 0:
        raise ValueError("warmup must be non-negative")
    if args.repeats <= 0 or args.benchmark_rounds <= 0:
        raise ValueError("repeats and benchmark_rounds must be positive")
    if args.cpu_baseline_seconds < 0:
        raise ValueError("cpu_baseline_seconds must be non-negative")
    if device.type == "cpu" and dtype == torch.float16:
        print("[warning] float16 CPU kernels may be unsupported or slow")


def validate_profile_focus(args: argparse.Namespace) -> None:
    """The checks on --profile-candidate / --rocprof that need no device."""
    if args.rocprof and not args.profile_candidate:
        raise ValueError("--rocprof requires --profile-candidate")
    if args.profile_candidate:
        focused = args.encoder_configs or (args.official_cases if args.official_matrix else None)
        if not focused:
            raise ValueError("--profile-candidate requires an explicit focused case list")
        if len(focused) > PROFILE_MAX_CASES:
            raise ValueError(f"--profile-candidate accepts at most {PROFILE_MAX_CASES} focused cases")
    if args.rocprof_timeout <= 0:
        raise ValueError("rocprof_timeout must be positive")


def environment_metadata(device: torch.device, dtype: torch.dtype) -> Dict[str, object]:
    meta: Dict[str, object] = {
        "python_version": platform.python_version(),
        "platform": platform.platform(),
        "device": str(device),
        "dtype": str(dtype),
        "torch_version": torch.__version__,
        "cuda_version": torch.version.cuda,
        "hip_version": getattr(torch.version, "hip", None),
        "gpu": torch.cuda.get_device_name(device) if device.type == "cuda" else None,
        "pytorch_cuda_alloc_conf": os.environ.get("PYTORCH_CUDA_ALLOC_CONF"),
        "host_cpu_count": os.cpu_count(),
        "host_torch_threads": torch.get_num_threads(),
    }
    if device.type == "cuda":
        props = torch.cuda.get_device_properties(device)
        meta["gpu_arch"] = getattr(props, "gcnArchName", None)
        meta["compute_units"] = props.multi_processor_count
        meta["gpu_memory_bytes"] = props.total_memory
    return meta


def settings_metadata(args: argparse.Namespace) -> Dict[str, object]:
    settings: Dict[str, object] = {
        "seed": args.seed,
        "padding_ratio": args.padding_ratio,
        "input_scale": args.input_scale,
        "accuracy_trials": args.accuracy_trials,
        "rtol": args.rtol,
        "atol": args.atol,
        "accuracy_rule": "strict_less_than_or",
        "warmup": args.warmup,
        "repeats": args.repeats,
        "benchmark_rounds": args.benchmark_rounds,
        "benchmark_on_failure": args.benchmark_on_failure,
        "matmul_precision": args.matmul_precision,
        "allow_tf32": args.allow_tf32,
        "compile_baseline": args.compile_baseline,
        "compile_user": args.compile_user,
        "cpu_baseline_seconds": args.cpu_baseline_seconds,
    }
    if args.encoder_configs:
        settings["encoder_configs"] = list(args.encoder_configs)
    if args.profile_candidate:
        settings["candidate_profile"] = {
            "warmup_replays": PROFILE_WARMUP_REPLAYS,
            "profiled_replays": PROFILE_CANDIDATE_REPLAYS,
            "event_limit": PROFILE_MAX_EVENTS,
        }
        if args.rocprof:
            settings["candidate_profile"]["rocprof_passes"] = [name for name, _ in ROCPROF_PASSES]
    return settings


def json_safe(value: Any) -> Any:
    """A copy of a result document that strict JSON accepts: NaN and +-inf
    become null at any depth of dicts, lists and tuples (tuples become
    lists, as json.dumps writes them anyway)."""
    if isinstance(value, dict):
        return dict(zip(value.keys(), map(json_safe, value.values())))
    if isinstance(value, (list, tuple)):
        return list(map(json_safe, value))
    return None if isinstance(value, float) and (math.isnan(value) or math.isinf(value)) else value


def write_json_document(path: Optional[Path], result: Dict[str, object]) -> None:
    if path is None:
        return
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_name(f".{path.name}.tmp")
    temporary.write_text(json.dumps(json_safe(result), indent=2, allow_nan=False) + "\n", encoding="utf-8")
    temporary.replace(path)


def configure_runtime(args: argparse.Namespace, device: torch.device) -> None:
    torch.set_float32_matmul_precision(args.matmul_precision)
    if device.type == "cuda":
        torch.backends.cuda.matmul.allow_tf32 = args.allow_tf32
        torch.backends.cudnn.allow_tf32 = args.allow_tf32


# ------------------------------------------------------------ measurement ----

def forward_flops(config: TransformerConfig) -> float:
    """Algorithmic FLOPs of one forward: GEMMs 8TD^2 + 4TDF per layer,
    attention 4BDS^2 (non-causal) or 4BDS(S+1)/2 (causal-live); padding is
    not subtracted."""
    t = config.batch_size * config.seq_len
    d, f, s = config.d_model, config.ffn_dim, config.seq_len
    attn = 4.0 * config.batch_size * d * s * ((s + 1) / 2 if config.causal else s)
    return config.num_layers * (8.0 * t * d * d + 4.0 * t * d * f + attn)


def roofline_summary(config: TransformerConfig, performance: Dict[str, object]) -> Dict[str, object]:
    median_ms = performance["optimized"]["median_ms"]  # type: ignore[index]
    flops = forward_flops(config)
    achieved = flops / (median_ms * 1e-3) / 1e12
    return {
        "flops_per_forward": flops,
        "tokens_per_second": config.batch_size * config.seq_len * 1000.0 / median_ms,
        "achieved_tflops": achieved,
        "peak_tflops": MFMA_PEAK_TFLOPS,
        "fraction_of_bf16_mfma_peak": achieved / MFMA_PEAK_TFLOPS,
    }


def cpu_baseline(baseline_cpu: nn.Module, config: TransformerConfig, dtype: torch.dtype, seed: int,
                 padding_ratio: float, input_scale: float, budget_s: float) -> Dict[str, object]:
    """The baseline forward on the host CPU for about budget_s seconds, on one
    sequence of the case (sequences are independent, so tokens/s carries
    over); beyond 8192 tokens one sequence's score rows are too large for the
    host, which is stated instead of extrapolated."""
    if config.seq_len > 8192:
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "port",
                "sample": f"not run: one sequence of {config.seq_len} tokens needs "
                          f"{4.0 * config.d_model * config.seq_len ** 2 / 1e12:.0f} TFLOP of attention "
                          "per layer on the host"}
    one = TransformerConfig(1, config.seq_len, config.d_model, config.num_heads, config.ffn_dim,
                            config.num_layers, config.causal)
    x, mask = generate_random_case(one, torch.device("cpu"), dtype, seed + 300000, padding_ratio, input_scale)
    runs = 0
    t0 = time.perf_counter()
    with torch.inference_mode():
        while True:
            baseline_cpu(x, mask)
            runs += 1
            if time.perf_counter() - t0 >= budget_s:
                break
    elapsed = time.perf_counter() - t0
    return {"value": runs * config.seq_len / elapsed, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{runs} forward(s) of one sequence ({config.seq_len} tokens), {elapsed:.1f} s"}


# ------------------------------------------------------------------ cases ----

def build_models(config: TransformerConfig, args: argparse.Namespace,
                 device: torch.device) -> Tuple[nn.Module, nn.Module]:
    """Seed, then the baseline, then the candidate, then the strict weight
    copy (runner.py:304-326 of the reference); both still on the host."""
    config.validate()
    torch.manual_seed(args.seed)
    if device.type == "cuda":
        torch.cuda.manual_seed_all(args.seed)
    baseline = BaselineTransformer(config)
    optimized = UserOptimizedTransformer(config)
    copy_model_weights(baseline, optimized, strict=not args.non_strict_weight_copy)
    return baseline, optimized


def _run_benchmark_case_with_profile(
    config: TransformerConfig, args: argparse.Namespace, device: torch.device, dtype: torch.dtype,
) -> Tuple[AccuracySummary, Optional[Dict[str, object]], Optional[Dict[str, object]]]:
    baseline, optimized = build_models(config, args, device)
    baseline_cpu = None
    if args.cpu_baseline_seconds > 0:
        baseline_cpu = BaselineTransformer(config)
        baseline_cpu.load_state_dict(baseline.state_dict())
        baseline_cpu = baseline_cpu.to(dtype=dtype).eval()
    baseline = baseline.to(device=device, dtype=dtype).eval()
    optimized = optimized.to(device=device, dtype=dtype).eval()
    baseline = maybe_compile(baseline, args.compile_baseline, args.compile_mode)
    optimized = maybe_compile(optimized, args.compile_user, args.compile_mode)

    print("=== Configuration ===")
    print(config)
    print(f"device={device}, dtype={dtype}, torch={torch.__version__}")
    if device.type == "cuda":
        print(f"gpu={torch.cuda.get_device_name(device)}")

    accuracy = run_accuracy_tests(
        baseline=baseline, optimized=optimized, config=config, device=device, dtype=dtype,
        trials=args.accuracy_trials, seed=args.seed, padding_ratio=args.padding_ratio,
        input_scale=args.input_scale, rtol=args.rtol, atol=args.atol,
    )
    if not accuracy.passed and not args.benchmark_on_failure:
        print("\nPerformance benchmark skipped because accuracy validation failed.")
        print("Use --benchmark-on-failure to benchmark an incorrect implementation anyway.")
        return accuracy, None, None
    release_case_memory(device)
    performance = benchmark_models(
        baseline=baseline, optimized=optimized, config=config, device=device, dtype=dtype,
        seed=args.seed, padding_ratio=args.padding_ratio, input_scale=args.input_scale,
        warmup=args.warmup, repeats=args.repeats, rounds=args.benchmark_rounds,
    )
    if device.type == "cuda":
        # which path the candidate's GPU calls took (the native forward, or the
        # logged native-torch fallback per reason), so no figure is read as
        # the kernels' when it was not
        module = getattr(optimized, "_orig_mod", optimized)
        performance["candidate_backend"] = {
            "native_calls": int(getattr(module, "native_calls", 0)),
            "fallback_calls": dict(getattr(module, "fallback_calls", {})),
        }
        performance["roofline"] = roofline_summary(config, performance)
        print(f"roofline: {performance['roofline']['fraction_of_bf16_mfma_peak']:.2%} of bf16 MFMA peak")
    if baseline_cpu is not None:
        performance["cpu_baseline"] = cpu_baseline(
            baseline_cpu, config, dtype, args.seed, args.padding_ratio, args.input_scale,
            args.cpu_baseline_seconds)
        print(f"cpu baseline: {performance['cpu_baseline']}")
    candidate_profile = None
    if args.profile_candidate and accuracy.passed:
        print("\n=== Bounded candidate profile ===")
        candidate_profile = profile_candidate(
            optimized=optimized, config=config, device=device, dtype=dtype, seed=args.seed,
            padding_ratio=args.padding_ratio, input_scale=args.input_scale,
        )
        print(f"recorded {len(candidate_profile['events'])} bounded events from "
              f"{PROFILE_CANDIDATE_REPLAYS} candidate replays")
    return accuracy, performance, candidate_profile


def run_benchmark_case(
    config: TransformerConfig, args: argparse.Namespace, device: torch.device, dtype: torch.dtype,
) -> Tuple[AccuracySummary, Optional[Dict[str, object]]]:
    accuracy, performance, _ = _run_benchmark_case_with_profile(config, args, device, dtype)
    return accuracy, performance


def config_from_args(args: argparse.Namespace) -> TransformerConfig:
    return TransformerConfig(
        batch_size=args.batch_size, seq_len=args.seq_len, d_model=args.d_model, num_heads=args.heads,
        ffn_dim=args.ffn_dim, num_layers=args.layers, causal=args.causal,
    )


def official_case_result(case_id: int, config: TransformerConfig, accuracy: AccuracySummary,
                         performance: Optional[Dict[str, object]],
                         candidate_profile: Optional[Dict[str, object]] = None) -> Dict[str, object]:
    result: Dict[str, object] = {
        "case_id": case_id,
        "config": asdict(config),
        "status": "succeeded" if accuracy.passed else "correctness_failed",
        "failure_category": None if accuracy.passed else "correctness",
        "correctness_passed": accuracy.passed,
        "accuracy": asdict(accuracy),
        "performance": performance,
    }
    if candidate_profile is not None:
        result["candidate_profile"] = candidate_profile
    return result


def execution_failed_result(case_id: int, config: TransformerConfig, failure_category: str,
                            error: BaseException) -> Dict[str, object]:
    return {
        "case_id": case_id,
        "config": asdict(config),
        "status": "execution_failed",
        "failure_category": failure_category,
        "correctness_passed": None,
        "accuracy": None,
        "performance": None,
        "error": str(error),
    }


def write_json_result(path: Optional[Path], config: TransformerConfig, args: argparse.Namespace,
                      device: torch.device, dtype: torch.dtype, accuracy: AccuracySummary,
                      performance: Optional[Dict[str, object]]) -> None:
    write_json_document(path, {
        "schema_version": 1,
        "config": asdict(config),
        "environment": environment_metadata(device, dtype),
        "settings": settings_metadata(args),
        "correctness_passed": accuracy.passed,
        "accuracy": asdict(accuracy),
        "performance": performance,
    })


def write_matrix_result(path: Optional[Path], args: argparse.Namespace, device: torch.device,
                        dtype: torch.dtype, requested_case_ids: List[int],
                        case_results: List[Dict[str, object]], case_set: str) -> None:
    complete = len(case_results) == len(requested_case_ids)
    all_cases_executed = complete and all(r["status"] != "execution_failed" for r in case_results)
    if not all_cases_executed:
        correctness_passed: Optional[bool] = None
        failure_category: Optional[str] = "execution" if complete else None
    elif all(r["correctness_passed"] is True for r in case_results):
        correctness_passed, failure_category = True, None
    else:
        correctness_passed, failure_category = False, "correctness"
    write_json_document(path, {
        "schema_version": 2,
        "mode": "official_matrix",
        "case_set": case_set,
        "requested_case_ids": requested_case_ids,
        "complete": complete,
        "all_cases_executed": all_cases_executed,
        "environment": environment_metadata(device, dtype),
        "settings": settings_metadata(args),
        "failure_category": failure_category,
        "correctness_passed": correctness_passed,
        "cases": case_results,
    })


def is_out_of_memory_error(error: BaseException) -> bool:
    return "out of memory" in str(error).lower()


def _run_matrix(cases: List[Tuple[int, TransformerConfig, argparse.Namespace, torch.device, torch.dtype]],
                args: argparse.Namespace, device: torch.device, dtype: torch.dtype, case_set: str,
                rocprof: Optional[Dict[int, Dict[str, object]]] = None) -> int:
    requested = [case_id for case_id, *_ in cases]
    results: List[Dict[str, object]] = []
    for position, (case_id, config, case_args, case_device, case_dtype) in enumerate(cases, start=1):
        print(f"\n######## Case {case_id} ({position}/{len(cases)}) ########")
        try:
            accuracy, performance, profile = _run_benchmark_case_with_profile(
                config, case_args, case_device, case_dtype)
            if profile is not None and rocprof is not None and case_id in rocprof:
                profile["rocprof"] = rocprof[case_id]
            result = official_case_result(case_id, config, accuracy, performance, profile)
        except UnsupportedShapeError as error:
            print(f"[unsupported shape] case {case_id}: {error}")
            result = execution_failed_result(case_id, config, "unsupported_shape", error)
        except RuntimeError as error:
            if not is_out_of_memory_error(error):
                raise
            print(f"[out of memory] case {case_id}: {error}")
            result = execution_failed_result(case_id, config, "out_of_memory", error)
        results.append(result)
        release_case_memory(case_device)
        write_matrix_result(args.json_output, args, device, dtype, requested, results, case_set)
    if any(r["status"] == "execution_failed" for r in results):
        return 3
    if any(r["correctness_passed"] is not True for r in results):
        return 2
    return 0


def official_cases(args: argparse.Namespace, device: torch.device, dtype: torch.dtype):
    requested = args.official_cases or list(range(1, len(OFFICIAL_TEST_CASES) + 1))
    return [(cid, OFFICIAL_TEST_CASES[cid - 1], args, device, dtype) for cid in requested]


def run_official_matrix(args: argparse.Namespace, device: torch.device, dtype: torch.dtype,
                        rocprof: Optional[Dict[int, Dict[str, object]]] = None) -> int:
    return _run_matrix(official_cases(args, device, dtype), args, device, dtype, "competition_appendix_3_7",
                       rocprof)


def encoder_config_case(name: str, args: argparse.Namespace) -> Tuple[TransformerConfig, argparse.Namespace,
                                                                      torch.device, torch.dtype]:
    """A measurement configuration's shape, seed, masking, dtype and device."""
    spec = ENCODER_CONFIGS[name]
    case_args = argparse.Namespace(**vars(args))
    case_args.seed = spec.seed
    case_args.padding_ratio = spec.padding_ratio
    case_device = resolve_device("cpu" if spec.device_type == "cpu" else "cuda")
    return spec.config, case_args, case_device, spec.dtype


def encoder_cases(args: argparse.Namespace):
    cases = []
    for name in args.encoder_configs:
        config, case_args, case_device, case_dtype = encoder_config_case(name, args)
        cases.append((ENCODER_CONFIG_NAMES.index(name) + 1, config, case_args, case_device, case_dtype))
    return cases


def run_encoder_configs(args: argparse.Namespace, device: torch.device, dtype: torch.dtype,
                        rocprof: Optional[Dict[int, Dict[str, object]]] = None) -> int:
    return _run_matrix(encoder_cases(args), args, device, dtype, "mi355x_encoder_configs_c1_c5", rocprof)


def profiled_case_ids(args: argparse.Namespace) -> List[int]:
    """Case ids of the focused cases that run on the GPU, in run order,
    decided without touching the GPU."""
    if args.encoder_configs:
        return [ENCODER_CONFIG_NAMES.index(n) + 1 for n in args.encoder_configs
                if ENCODER_CONFIGS[n].device_type != "cpu"]
    return list(args.official_cases or [])


def collect_rocprof(args: argparse.Namespace, argv: Sequence[str]) -> Dict[int, Dict[str, object]]:
    """Run the rocprofv3 passes over child processes that replay the focused
    cases (before this process touches the GPU) and summarise them per case."""
    case_ids = profiled_case_ids(args)
    if not case_ids:
        return {}
    out_dir = str(args.rocprof_dir) if args.rocprof_dir else tempfile.mkdtemp(prefix="rocprof_candidate_")
    print(f"=== rocprofv3 candidate profile ({len(case_ids)} case(s), output {out_dir}) ===", flush=True)
    commands = run_rocprof_passes(out_dir, list(argv), args.rocprof_timeout,
                                  log=lambda line: print(line, flush=True))
    summaries = summarize_rocprof({name: os.path.join(out_dir, name) for name, _ in ROCPROF_PASSES},
                                  commands, len(case_ids))
    for summary in summaries:
        summary["output_dir"] = out_dir
    return dict(zip(case_ids, summaries))


def run_rocprof_child(args: argparse.Namespace) -> int:
    """The profiled program of one rocprofv3 pass: for every focused GPU
    case, two warmup calls, then three candidate calls between two marker
    dispatches; a calibration copy of known size comes first."""
    device = resolve_device(args.device)
    dtype = resolve_dtype(args.dtype)
    configure_runtime(args, device)
    cases = encoder_cases(args) if args.encoder_configs else official_cases(args, device, dtype)
    calibration_copy()
    for case_id, config, case_args, case_device, case_dtype in cases:
        if case_device.type != "cuda":
            continue
        _, optimized = build_models(config, case_args, case_device)
        optimized = optimized.to(device=case_device, dtype=case_dtype).eval()
        x, mask = generate_random_case(config, case_device, case_dtype, case_args.seed + 200000,
                                       case_args.padding_ratio, case_args.input_scale)
        warmup_model(optimized, x, mask, PROFILE_WARMUP_REPLAYS, case_device)
        region_marker()
        with torch.inference_mode():
            for _ in range(PROFILE_CANDIDATE_REPLAYS):
                optimized(x, mask)
        region_marker()
        torch.cuda.synchronize(case_device)
        print(f"profiled case {case_id}", flush=True)
        del optimized, x, mask
        release_case_memory(case_device)
    return 0


def run_single_case(args: argparse.Namespace, device: torch.device, dtype: torch.dtype) -> int:
    config = config_from_args(args)
    accuracy, performance = run_benchmark_case(config, args, device, dtype)
    write_json_result(args.json_output, config, args, device, dtype, accuracy, performance)
    return 0 if accuracy.passed else 2


def main(argv: Optional[Sequence[str]] = None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    args = parse_args(argv)
    if args.rocprof_child:
        return run_rocprof_child(args)
    rocprof = None
    if args.rocprof:
        # before anything below touches the GPU
        validate_profile_focus(args)
        rocprof = collect_rocprof(args, argv)
    device = resolve_device(args.device)
    dtype = resolve_dtype(args.dtype)
    validate_args(args, device, dtype)
    configure_runtime(args, device)
    if args.encoder_configs:
        return run_encoder_configs(args, device, dtype, rocprof)
    if args.official_matrix:
        return run_official_matrix(args, device, dtype, rocprof)
    return run_single_case(args, device, dtype)


if __name__ == "__main__":
    raise SystemExit(main())
