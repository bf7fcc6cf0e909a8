#!/usr/bin/env python3
"""Encoder-forward benchmark on one MI355X; prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c5] [--also c2,c3,c4]

A step is one forward of ``UserOptimizedTransformer`` (the drop-in candidate
of transformer_benchmark/models.py:922-1239) over one batch of synthetic input
already resident in HBM.  The headline workload is BASELINE configuration c5
(B=32, S=100000, D=1024, H=16, FFN=1024, L=2, bf16, non-causal, weights seeded
with 4, timing input seeded with 4 + 100000 as in timing.py:123): the largest
configuration, which fits one GPU only because scores are never materialised.
The configurations named by ``--also`` (default c2, c3, c4) are measured in the
same run with the same protocol and reported under ``"configs"``; c1 is the
reference's CPU smoke case and runs through the CLI tests instead.

Reported beside each configuration's throughput:
  * ``roofline``: the kernel with the largest share of the forward's time.
    Each kernel's launches, with the inputs a forward driven launch by launch
    through the C ABI gives them (the sequence enc_encoder_forward_bf16
    issues), are timed back to back between hipEvents on the stream they run
    on (torch's current stream).  A kernel whose algorithmic FLOPs per byte
    fall below the ridge point (2.5 PFLOP/s / 8 TB/s = 312) is HBM-bound:
    achieved = algorithmic bytes per launch / mean launch duration against
    8 TB/s; otherwise achieved = algorithmic FLOPs per launch / mean duration
    against the MI355X dense bf16 MFMA peak (2.5 PFLOP/s).  ``traffic`` is the
    HBM bytes per launch measured with rocprofv3 counters (profiles/traffic.json);
  * ``cpu_baseline``: the oracle's restatement of the reference forward
    (oracle/encoder_oracle.py) timed on the host CPU for a bounded sample: c2
    whole forwards, c3 and c4 one sequence's forward, c5 one sequence's work
    for a block of rows of one layer, extrapolated (the sample says which).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "fwd latency ms + tokens/s + % bf16 MFMA peak per encoder config, 1 GPU"
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
HBM_PEAK_GBS = 8000.0


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--config", default="c5", choices=["c2", "c3", "c4", "c5"],
                   help="headline workload")
    p.add_argument("--also", default="c2,c3,c4",
                   help="comma-separated configurations also measured and reported under 'configs' ('' for none)")
    p.add_argument("--kernel-reps", type=int, default=10,
                   help="rounds over the layers' launches when timing each kernel (c5: at most 1)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="finish with a device copy of this many MiB (rocprof counter calibration)")
    return p.parse_args(argv)


# --------------------------------------------------------------- kernels ----

def profiled_forward(cfg, model, x, mask, native, torch, record):
    """The native forward's launch sequence (enc_encoder_forward_bf16 issues the
    same kernels in the same order) driven launch by launch through the C ABI,
    with ``record(name, (flops, bytes), fn)`` wrapping every launch."""
    b, s, d = cfg.batch_size, cfg.seq_len, cfg.d_model
    h, f, hd = cfg.num_heads, cfg.ffn_dim, cfg.d_model // cfg.num_heads
    t = b * s
    kv_len = row_mask = None
    if mask is not None and not bool(mask.all()):
        kv_len = native.mask_lengths(mask)
        row_mask = mask.reshape(-1)
    if cfg.causal:
        attn_flops = 4.0 * b * d * s * (s + 1) / 2  # causal-live, padding not subtracted
    else:
        attn_flops = 4.0 * b * d * s * s
    e = 2.0  # bf16 bytes
    # (algorithmic FLOPs, algorithmic HBM bytes) per launch: every operand read
    # once and every result written once
    ln_work = (0.0, 2 * e * t * d + 2 * e * d)
    qkv_work = (2.0 * t * 3 * d * d, e * (t * d + 3 * d * d + 3 * d + 3 * t * d))
    attn_work = (attn_flops, e * 4 * t * d)
    out_work = (2.0 * t * d * d, e * (t * d + d * d + d + 2 * t * d))
    ffn_in_work = (2.0 * t * f * d, e * (t * d + f * d + f + t * f))
    ffn_out_work = (2.0 * t * d * f, e * (t * f + d * f + d + 2 * t * d))
    xa = x.reshape(t, d)
    for layer in model.layers:
        attn = layer.attention
        xn = record("layernorm", ln_work,
                    lambda: native.layernorm(xa, layer.norm1.weight, layer.norm1.bias, layer.norm1.eps))
        q, k, v_t = record("qkv_proj", qkv_work,
                           lambda: native.qkv_proj(xn.view(b, s, d), attn.qkv_proj.weight,
                                                   attn.qkv_proj.bias, h))
        ctx = record("attention", attn_work,
                     lambda: native.attention(q, k, v_t, hd**-0.5, cfg.causal, kv_len=kv_len))
        xb = record("out_proj_residual", out_work,
                    lambda: native.linear(ctx.view(t, d), attn.out_proj.weight, attn.out_proj.bias,
                                          native.ENC_EPI_BIAS_RESIDUAL_KEEP, residual=xa,
                                          row_mask=row_mask))
        xn2 = record("layernorm", ln_work,
                     lambda: native.layernorm(xb, layer.norm2.weight, layer.norm2.bias, layer.norm2.eps))
        hid = record("ffn_in_gelu", ffn_in_work,
                     lambda: native.linear(xn2, layer.ffn_in.weight, layer.ffn_in.bias,
                                           native.ENC_EPI_BIAS_GELU))
        xa = record("ffn_out_residual", ffn_out_work,
                    lambda: native.linear(hid, layer.ffn_out.weight, layer.ffn_out.bias,
                                          native.ENC_EPI_BIAS_RESIDUAL_ZERO, residual=xb,
                                          row_mask=row_mask))
    fn = model.final_norm
    return record("layernorm", ln_work,
                  lambda: native.layernorm(xa, fn.weight, fn.bias, fn.eps, row_mask=row_mask)).view(b, s, d)


def kernel_profile(cfg, model, x, mask, native, torch, reps):
    """Mean launch duration of each kernel of the forward.

    One launch-by-launch forward keeps, per kernel, the launch closures of all
    layers with their real inputs.  Each kernel is then timed alone: the GPU
    gets a busy-wait first, so ``reps`` rounds over the layers' launches queue
    up behind it and run back to back between one pair of hipEvents on the
    current stream; the duration is the elapsed time over the launch count
    (inter-launch gaps included, so it slightly overstates the kernel)."""
    launches = {}

    def record(name, work, fn):
        flops, nbytes = work
        # below the ridge point (peak FLOP/s over peak bytes/s) HBM bounds it
        bound = "mfma" if flops / nbytes >= MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"
        entry = launches.setdefault(name, {"flops": flops, "bytes": nbytes, "bound": bound, "fns": []})
        entry["fns"].append(fn)
        return fn()

    out = profiled_forward(cfg, model, x, mask, native, torch, record)
    torch.cuda.synchronize()
    stats = {}
    per_step = {name: len(v["fns"]) for name, v in launches.items()}
    for name, entry in launches.items():
        fns = entry["fns"]
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        try:
            torch.cuda._sleep(20_000_000)
        except Exception:  # the busy-wait only keeps host latency out of the pair
            pass
        start.record()
        for _ in range(reps):
            for fn in fns:
                fn()
        end.record()
        torch.cuda.synchronize()
        stats[name] = {"flops": entry["flops"], "bytes": entry["bytes"], "bound": entry["bound"],
                       "per_step": per_step[name],
                       "mean_ms": start.elapsed_time(end) / (reps * len(fns)),
                       "launches": reps * len(fns)}
    return stats, out


def load_traffic(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE runs, scaled by the copy-kernel calibration), if recorded in
    profiles/traffic.json by ``python -m tiktoktechjam2026track3_amd.profiling``."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        table = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = table.get(f"{kernel}@{workload}")
    return None if entry is None else entry.get("bytes_per_launch")


def copy_calibration(mib, torch):
    """A device-to-device copy of exactly ``mib`` MiB, so a rocprofv3 --pmc run
    of this process reads FETCH_SIZE / WRITE_SIZE for a kernel of known traffic
    (the largest __amd_rocclr_copyBuffer dispatch)."""
    n = mib * 1024 * 1024
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


# ----------------------------------------------------------- CPU baseline ----

def host_cpu():
    """CPU model and logical core count of the host (the GPU box's, in a GPU run)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def _cpu_record(value, sample, torch, estimate=False):
    model, count = host_cpu()
    record = {"value": value, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
              "sample": sample, "cpu_model": model, "cpu_count": count}
    if estimate:
        record["estimate"] = True
    return record


def cpu_baseline(spec, baseline_sd, budget_s, torch):
    """The oracle's reference forward on the host CPU at the config's dtype, for
    a bounded sample of about budget_s seconds.  c2 runs whole forwards; c3
    and c4 one sequence (sequences are independent, so tokens/s carries over);
    c5 one sequence's layer work for a block of rows, extrapolated."""
    if spec.name == "c5":
        return cpu_baseline_c5_estimate(spec, baseline_sd, budget_s, torch)
    from oracle.encoder_oracle import encoder_forward, generate_case

    cfg = spec.config
    batch = cfg.batch_size if spec.name == "c2" else 1
    sd = {k: v.to(torch.bfloat16) for k, v in baseline_sd.items()}
    x, mask = generate_case(batch, cfg.seq_len, cfg.d_model, torch.device("cpu"), torch.bfloat16,
                            spec.seed + 100000, spec.padding_ratio)
    m = None if bool(mask.all()) else mask
    runs = 0
    t0 = time.perf_counter()
    with torch.inference_mode():
        while True:
            encoder_forward(sd, x, m, cfg.causal, cfg.num_heads, cfg.num_layers)
            runs += 1
            if time.perf_counter() - t0 >= budget_s:
                break
    elapsed = time.perf_counter() - t0
    return _cpu_record(runs * batch * cfg.seq_len / elapsed,
                       f"{runs} forward(s) of {spec.name} with batch {batch} (of {cfg.batch_size}), bf16, "
                       f"oracle restatement on torch CPU ops, {elapsed:.1f} s", torch)


def cpu_baseline_c5_estimate(spec, baseline_sd, budget_s, torch, token_block=2048, query_block=64):
    """c5 on the CPU, extrapolated: a whole c5 forward is ~2700 TFLOP (hours on
    the host), so one sequence's first layer is sampled.  Its row-local work
    (LayerNorms, the six projections, GELU and residuals) is timed on a block
    of token_block tokens, and its attention on a block of query_block query
    rows against all 100000 keys (the oracle's row-blocked restatement); the
    per-layer time of a sequence is t_rows * S / token_block +
    t_attn * S / query_block, and a forward is L layers of B sequences."""
    import torch.nn.functional as F

    from oracle.encoder_oracle import attention_rows, generate_case

    cfg = spec.config
    s, d, h = cfg.seq_len, cfg.d_model, cfg.num_heads
    hd = d // h
    sd = {k: v.to(torch.bfloat16) for k, v in baseline_sd.items()}
    x, _ = generate_case(1, s, d, torch.device("cpu"), torch.bfloat16, spec.seed + 100000, 0.0)
    p, a = "layers.0.", "layers.0.attention."

    def row_work(rows):
        hn = F.layer_norm(rows, (d,), sd[p + "norm1.weight"], sd[p + "norm1.bias"], 1e-5)
        q = F.linear(hn, sd[a + "q_proj.weight"], sd[a + "q_proj.bias"])
        k = F.linear(hn, sd[a + "k_proj.weight"], sd[a + "k_proj.bias"])
        v = F.linear(hn, sd[a + "v_proj.weight"], sd[a + "v_proj.bias"])
        y = rows + F.linear(q + k + v, sd[a + "out_proj.weight"], sd[a + "out_proj.bias"])
        h2 = F.layer_norm(y, (d,), sd[p + "norm2.weight"], sd[p + "norm2.bias"], 1e-5)
        hid = F.gelu(F.linear(h2, sd[p + "ffn_in.weight"], sd[p + "ffn_in.bias"]), approximate="none")
        return y + F.linear(hid, sd[p + "ffn_out.weight"], sd[p + "ffn_out.bias"])

    with torch.inference_mode():
        hn = F.layer_norm(x, (d,), sd[p + "norm1.weight"], sd[p + "norm1.bias"], 1e-5)

        def heads(t):
            return t.view(1, t.shape[1], h, hd).transpose(1, 2).contiguous()

        k = heads(F.linear(hn, sd[a + "k_proj.weight"], sd[a + "k_proj.bias"]))
        v = heads(F.linear(hn, sd[a + "v_proj.weight"], sd[a + "v_proj.bias"]))
        q = heads(F.linear(hn[:, :query_block], sd[a + "q_proj.weight"], sd[a + "q_proj.bias"]))
        positions = torch.arange(query_block)
        t_rows, t_attn, n_rows, n_attn = 0.0, 0.0, 0, 0
        t0 = time.perf_counter()
        while True:
            t1 = time.perf_counter()
            row_work(x[:, :token_block])
            t_rows += time.perf_counter() - t1
            n_rows += 1
            t1 = time.perf_counter()
            attention_rows(q, k, v, hd**-0.5, False, None, positions)
            t_attn += time.perf_counter() - t1
            n_attn += 1
            if time.perf_counter() - t0 >= budget_s:
                break
    per_layer = (t_rows / n_rows) * s / token_block + (t_attn / n_attn) * s / query_block
    forward_s = per_layer * cfg.num_layers * cfg.batch_size
    value = cfg.batch_size * s / forward_s
    return _cpu_record(
        value,
        f"extrapolated estimate: one c5 sequence, layer 0, bf16 oracle ops on the CPU: row-local work on "
        f"{token_block} tokens ({t_rows / n_rows:.3f} s, x{n_rows}) and attention for {query_block} query rows "
        f"against all {s} keys ({t_attn / n_attn:.3f} s, x{n_attn}), scaled to {s} rows, {cfg.num_layers} layers "
        f"and {cfg.batch_size} sequences: {forward_s / 3600:.1f} h per forward",
        torch, estimate=True)


# ------------------------------------------------------------------ main ----

def measure_config(name, args, torch, native, reps):
    """Warmup, K timed forwards, the per-kernel profile and the roofline of the
    dominant kernel for one configuration."""
    import contextlib

    from tiktoktechjam2026track3_amd.cases import ENCODER_CONFIGS, generate_random_case
    from tiktoktechjam2026track3_amd.models import (
        BaselineTransformer, UserOptimizedTransformer, copy_model_weights,
    )

    spec = ENCODER_CONFIGS[name]
    cfg = spec.config
    device = torch.device("cuda:0")
    torch.manual_seed(spec.seed)
    baseline = BaselineTransformer(cfg)
    candidate = UserOptimizedTransformer(cfg)
    candidate.native_only = True  # a timed figure is never the torch fallback's
    copy_model_weights(baseline, candidate)
    baseline_sd = {k: v.detach().clone() for k, v in baseline.state_dict().items()}
    del baseline
    candidate = candidate.to(device=device, dtype=torch.bfloat16).eval()
    x, mask = generate_random_case(cfg, device, torch.bfloat16, spec.seed + 100000, spec.padding_ratio, 1.0)
    tokens = cfg.batch_size * cfg.seq_len

    # the model's one-line capture notice goes to stderr: stdout carries only the JSON line
    with torch.inference_mode(), contextlib.redirect_stdout(sys.stderr):
        for _ in range(args.warmup):
            candidate(x, mask)
        torch.cuda.synchronize()
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(args.steps)]
        torch.cuda.synchronize()
        for start, end in pairs:
            start.record()
            candidate(x, mask)
            end.record()
        torch.cuda.synchronize()
        total_ms = pairs[0][0].elapsed_time(pairs[-1][1])
        per_call = [a.elapsed_time(b) for a, b in pairs]
        print(f"[bench] {name}: {args.steps} forwards, median {statistics.median(per_call):.3f} ms",
              file=sys.stderr, flush=True)

        graph_out = candidate(x, mask)
        candidate._hip.workspace = None  # the launch-by-launch forward allocates its own buffers
        stats, prof_out = kernel_profile(cfg, candidate, x, mask, native, torch, reps)
        if not torch.equal(prof_out, graph_out):
            print(f"warning: {name}: launch-by-launch forward differs from the model forward", file=sys.stderr)
        del graph_out, prof_out
    del candidate, x, mask
    torch.cuda.empty_cache()

    timed = []
    for kname, v in stats.items():
        timed.append((v["per_step"] * v["mean_ms"], kname, v["per_step"], v["mean_ms"], v["launches"],
                      v["flops"], v["bytes"], v["bound"]))
    timed.sort(reverse=True)
    ms_per_step = total_ms / args.steps
    median_ms = statistics.median(per_call)
    d, f, s, b = cfg.d_model, cfg.ffn_dim, cfg.seq_len, cfg.batch_size
    attn = 4.0 * b * d * s * (s + 1) / 2 if cfg.causal else 4.0 * b * d * s * s
    flops = cfg.num_layers * (8.0 * tokens * d * d + 4.0 * tokens * d * f + attn)

    _, kname, kcount, kmean, ktimed, kflops, kbytes, kbound = timed[0]
    if kbound == "mfma":
        achieved, peak, unit = kflops / (kmean * 1e-3) / 1e12, MFMA_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = kbytes / (kmean * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
    roofline = {
        "bound": kbound,
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 5),
        "traffic": load_traffic(kname, spec.name),
        "kernel": kname,
        "launch_ms_mean": round(kmean, 5),
        "launches_per_step": kcount,
        "launches_timed": ktimed,
        "flops_per_launch": kflops,
        "bytes_per_launch": kbytes,
    }
    breakdown = {}
    for share, kn, count, mean, _, k_flops, k_bytes, bound in timed:
        rate = k_flops / (mean * 1e-3) / 1e12 if bound == "mfma" else k_bytes / (mean * 1e-3) / 1e9
        breakdown[kn] = {"mean_ms": round(mean, 5), "per_step": count, "bound": bound,
                         "achieved": round(rate, 2), "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                         "share_est": round(share / ms_per_step, 4)}
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(spec, baseline_sd, args.cpu_seconds, torch)
    return {
        "workload": spec.name,
        "value": tokens * args.steps / (total_ms / 1e3),
        "ms_per_step": ms_per_step,
        "latency_ms_median": median_ms,
        "tokens_per_s_median": tokens / (median_ms * 1e-3),
        "pct_bf16_mfma_peak": 100.0 * flops / (median_ms * 1e-3) / (MFMA_PEAK_TFLOPS * 1e12),
        "flops_per_forward": flops,
        "config": {
            "workload": spec.name,
            "batch": b, "seq_len": s, "d_model": d, "num_heads": cfg.num_heads,
            "ffn_dim": f, "num_layers": cfg.num_layers, "causal": cfg.causal,
            "padding_ratio": spec.padding_ratio, "parallelism": "single GPU",
        },
        "roofline": roofline,
        "kernels": breakdown,
        "cpu_baseline": cpu,
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the encoder would shard over the batch across GPUs, which this build "
              "does not run)", file=sys.stderr)
        return 2

    sys.path.insert(0, str(ROOT))
    from tiktoktechjam2026track3_amd.runtime_environment import configure_pre_torch_environment

    configure_pre_torch_environment()
    import torch

    from tiktoktechjam2026track3_amd import native

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        return 3
    native.load_library()  # fails loudly if the HIP library is missing
    also = [c for c in (a.strip() for a in args.also.split(",")) if c and c != args.config]
    for c in also:
        if c not in ("c2", "c3", "c4", "c5"):
            print(f"unknown configuration {c!r} in --also", file=sys.stderr)
            return 2

    head = measure_config(args.config, args, torch, native,
                          min(args.kernel_reps, 1) if args.config == "c5" else args.kernel_reps)
    others = {}
    for c in also:
        others[c] = measure_config(c, args, torch, native, min(args.kernel_reps, 1) if c == "c5" else args.kernel_reps)
        others[c].pop("config")
    if args.copy_calibration_mib > 0:
        copy_calibration(args.copy_calibration_mib, torch)

    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x ~ N(0,1) seeded, default-init weights seeded (no checkpoints)",
        "config": head["config"],
        "latency_ms_median": head["latency_ms_median"],
        "pct_bf16_mfma_peak": head["pct_bf16_mfma_peak"],
        "flops_per_forward": head["flops_per_forward"],
        "roofline": head["roofline"],
        "kernels": head["kernels"],
        "cpu_baseline": head["cpu_baseline"],
        "configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
