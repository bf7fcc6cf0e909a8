"""Elementwise correctness gate between the baseline and the candidate forward.

Mirrors transformer_benchmark/correctness.py of the reference:
``compare_outputs`` (correctness.py:40-109) applies the strict OR rule
``|opt - ref| < atol  OR  |opt - ref| < rtol * |ref|`` to finite elements only
(non-finite elements fail), reports the maximum absolute/relative error, the
worst index and the failing output-feature columns; ``run_accuracy_tests``
(correctness.py:112-188) runs trials with seeds ``seed + trial`` under
``torch.inference_mode``.  In addition each result reports whether the looser
allclose form ``|opt - ref| <= atol + rtol * |ref|`` holds.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Tuple

import torch
import torch.nn as nn

from .cases import TransformerConfig, generate_random_case


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float
    allclose_passed: bool = True


@dataclass
class AccuracySummary:
    passed: bool
    rtol: float
    atol: float
    max_abs_error: float
    max_relative_error: float
    failed_elements: int
    total_elements: int
    trials: List[AccuracyResult] = field(default_factory=list)


def _unravel(flat: int, shape: Tuple[int, ...]) -> Tuple[int, ...]:
    index = []
    for size in reversed(shape):
        index.append(flat % size)
        flat //= size
    return tuple(reversed(index))


def compare_outputs(
    reference: torch.Tensor,
    optimized: torch.Tensor,
    rtol: float,
    atol: float,
) -> AccuracyResult:
    if reference.shape != optimized.shape:
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, "
            f"optimized={tuple(optimized.shape)}"
        )
    if reference.dtype != optimized.dtype:
        print(
            f"[warning] dtype mismatch: baseline={reference.dtype}, "
            f"optimized={optimized.dtype}"
        )

    ref = reference.detach().float()
    opt = optimized.detach().float()
    err = (opt - ref).abs()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    # Strict OR rule: each element passes on either bound, never on their sum.
    ok = finite & ((err < atol) | (err < rtol * ref.abs()))
    failed = ~ok
    failed_count = int(failed.sum().item())
    allclose_ok = bool((finite & (err <= atol + rtol * ref.abs())).all().item())

    worst = _unravel(int(err.reshape(-1).argmax().item()), tuple(reference.shape))
    rel = err / ref.abs().clamp_min(1e-12)

    if reference.ndim == 0:
        failed_dims = [0] if failed_count else []
    elif reference.ndim == 1:
        failed_dims = torch.nonzero(failed, as_tuple=False).flatten().tolist()
    else:
        per_feature = failed.any(dim=tuple(range(reference.ndim - 1)))
        failed_dims = torch.nonzero(per_feature, as_tuple=False).flatten().tolist()

    return AccuracyResult(
        passed=failed_count == 0,
        total_elements=reference.numel(),
        failed_elements=failed_count,
        max_abs_error=float(err.max().item()),
        max_relative_error=float(rel.max().item()),
        mean_abs_error=float(err.mean().item()),
        failed_feature_dims=failed_dims,
        worst_index=worst,
        reference_at_worst=float(ref[worst].item()),
        optimized_at_worst=float(opt[worst].item()),
        allclose_passed=allclose_ok,
    )


def run_accuracy_tests(
    baseline: nn.Module,
    optimized: nn.Module,
    config: TransformerConfig,
    device: torch.device,
    dtype: torch.dtype,
    trials: int,
    seed: int,
    padding_ratio: float,
    input_scale: float,
    rtol: float,
    atol: float,
) -> AccuracySummary:
    print("\n=== Accuracy check ===")
    print(f"criterion: abs_error < {atol:g} OR relative_error < {rtol:.2%}")

    summary = AccuracySummary(
        passed=True, rtol=rtol, atol=atol, max_abs_error=0.0, max_relative_error=0.0,
        failed_elements=0, total_elements=0, trials=[],
    )
    with torch.inference_mode():
        for trial in range(trials):
            x, mask = generate_random_case(
                config=config, device=device, dtype=dtype, seed=seed + trial,
                padding_ratio=padding_ratio, input_scale=input_scale,
            )
            reference = baseline(x, mask)
            candidate = optimized(x, mask)
            result = compare_outputs(reference, candidate, rtol=rtol, atol=atol)
            del reference, candidate, x, mask
            summary.trials.append(result)
            summary.passed = summary.passed and result.passed
            summary.max_abs_error = max(summary.max_abs_error, result.max_abs_error)
            summary.max_relative_error = max(summary.max_relative_error, result.max_relative_error)
            summary.failed_elements += result.failed_elements
            summary.total_elements += result.total_elements

            print(
                f"trial {trial + 1:02d}/{trials}: {'PASS' if result.passed else 'FAIL'} | "
                f"max_abs={result.max_abs_error:.6g} | "
                f"max_rel={result.max_relative_error:.6g} | "
                f"failed={result.failed_elements}/{result.total_elements}"
            )
            if not result.passed:
                shown = result.failed_feature_dims[:16]
                more = "..." if len(result.failed_feature_dims) > len(shown) else ""
                print(
                    f"  worst_index={result.worst_index}, "
                    f"baseline={result.reference_at_worst:.8g}, "
                    f"optimized={result.optimized_at_worst:.8g}"
                )
                print(f"  failed output feature dims={shown}{more}")

    print(
        f"summary: {'PASS' if summary.passed else 'FAIL'} | "
        f"max_abs={summary.max_abs_error:.6g} | max_rel={summary.max_relative_error:.6g} | "
        f"failed={summary.failed_elements}/{summary.total_elements}"
    )
    return summary
