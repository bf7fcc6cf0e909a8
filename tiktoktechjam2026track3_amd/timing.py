"""Warmup and steady-state latency measurement (interface of
transformer_benchmark/timing.py:17-195).

The protocol is the reference's: a fixed timing input generated with
``seed + 100000``, ``warmup`` untimed calls of each model, then ``rounds``
rounds of ``repeats`` timed calls with the baseline/candidate order alternating
between rounds.  On a GPU every call is bracketed by a pair of device events
recorded on the current stream (hipEvent on ROCm, which torch exposes as
``torch.cuda.Event``); on the CPU by ``time.perf_counter_ns``.  Latency is the
median sample; throughput is ``batch * seq_len * 1000 / median_ms`` tokens/s.
"""

from __future__ import annotations

import math
import statistics
import time
from dataclasses import dataclass
from typing import Dict, List

import torch
import torch.nn as nn

from .cases import TransformerConfig, generate_random_case

TIMING_SEED_OFFSET = 100000  # timing.py:123


def percentile(values: List[float], q: float) -> float:
    """Linear-interpolated percentile, q in [0, 1] (timing.py:17-30)."""
    if not values:
        raise ValueError("values must not be empty")
    ordered = sorted(values)
    pos = (len(ordered) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    if lo == hi:
        return ordered[lo]
    frac = pos - lo
    return ordered[lo] * (1.0 - frac) + ordered[hi] * frac


@dataclass
class TimingResult:
    samples_ms: List[float]

    @property
    def mean_ms(self) -> float:
        return statistics.fmean(self.samples_ms)

    @property
    def median_ms(self) -> float:
        return statistics.median(self.samples_ms)

    @property
    def p90_ms(self) -> float:
        return percentile(self.samples_ms, 0.90)

    @property
    def min_ms(self) -> float:
        return min(self.samples_ms)

    def summary(self, tokens_per_call: int) -> Dict[str, object]:
        return {
            "samples_ms": list(self.samples_ms),
            "median_ms": self.median_ms,
            "mean_ms": self.mean_ms,
            "p90_ms": self.p90_ms,
            "min_ms": self.min_ms,
            "tokens_per_second": tokens_per_call * 1000.0 / self.median_ms,
        }


def warmup_model(
    model: nn.Module,
    x: torch.Tensor,
    valid_mask: torch.Tensor,
    iterations: int,
    device: torch.device,
) -> None:
    """Untimed calls, then a device synchronisation (timing.py:53-64)."""
    with torch.inference_mode():
        for _ in range(iterations):
            model(x, valid_mask)
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def benchmark_once(
    model: nn.Module,
    x: torch.Tensor,
    valid_mask: torch.Tensor,
    iterations: int,
    device: torch.device,
) -> List[float]:
    """Per-call latency samples in milliseconds (timing.py:67-99)."""
    samples: List[float] = []
    with torch.inference_mode():
        if device.type == "cuda":
            events = [
                (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(iterations)
            ]
            torch.cuda.synchronize(device)
            for start, end in events:
                start.record()
                model(x, valid_mask)
                end.record()
            torch.cuda.synchronize(device)
            samples = [start.elapsed_time(end) for start, end in events]
        else:
            for _ in range(iterations):
                t0 = time.perf_counter_ns()
                model(x, valid_mask)
                samples.append((time.perf_counter_ns() - t0) / 1e6)
    return samples


def benchmark_models(
    baseline: nn.Module,
    optimized: nn.Module,
    config: TransformerConfig,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float,
    warmup: int,
    repeats: int,
    rounds: int,
) -> Dict[str, object]:
    """Alternating-order latency comparison (timing.py:102-195)."""
    print("\n=== Performance benchmark ===")
    print("timing excludes random-data generation and uses a fixed input")
    if device.type == "cuda":
        print("GPU latency is measured with hipEvents on the current stream")

    x, valid_mask = generate_random_case(
        config, device, dtype, seed + TIMING_SEED_OFFSET, padding_ratio, input_scale
    )
    warmup_model(baseline, x, valid_mask, warmup, device)
    warmup_model(optimized, x, valid_mask, warmup, device)

    base_samples: List[float] = []
    opt_samples: List[float] = []
    for round_index in range(rounds):
        order = [(baseline, base_samples), (optimized, opt_samples)]
        if round_index % 2:
            order.reverse()
        for model, sink in order:
            sink.extend(benchmark_once(model, x, valid_mask, repeats, device))

    tokens = config.batch_size * config.seq_len
    base = TimingResult(base_samples)
    opt = TimingResult(opt_samples)
    speedup = base.median_ms / opt.median_ms
    for label, res in (("baseline ", base), ("optimized", opt)):
        print(
            f"{label}: median={res.median_ms:.4f} ms | mean={res.mean_ms:.4f} ms | "
            f"p90={res.p90_ms:.4f} ms | min={res.min_ms:.4f} ms | "
            f"throughput={tokens * 1000.0 / res.median_ms:.2f} token/s"
        )
    print(f"speedup  : {speedup:.3f}x based on median latency")
    return {
        "baseline": base.summary(tokens),
        "optimized": opt.summary(tokens),
        "speedup": speedup,
        "warmup": warmup,
        "repeats": repeats,
        "rounds": rounds,
    }
