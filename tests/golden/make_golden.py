"""Write golden vectors by running the reference's own Python in this container.

Run once, from the repository root, where /root/reference is mounted:

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's ``transformer_benchmark`` package (torch-CPU only;
no Triton/CUDA path is reachable on CPU) and records, as plain arrays and JSON:

  * default-init weights per seed for several shapes, including the five
    measurement configurations (checksums + leading values; full tensors for
    tiny shapes) -- pins the module construction order of models.py:20-33,
    719-725, 896-907;
  * generate_random_case outputs (cases.py:60-98) on CPU -- pins the RNG order;
  * BaselineTransformer forward outputs on CPU in fp32 and bf16 (models.py:
    909-919) for tiny shapes (full) and for c1 (sampled rows + checksums);
  * compare_outputs verdicts on boundary cases (correctness.py:40-109) and
    timing.percentile values (timing.py:17-30).

Nothing from the reference is copied into the repository: only these numbers.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REFERENCE = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().float().numpy().tobytes()).hexdigest()


def summary(t: torch.Tensor) -> dict:
    f = t.detach().double()
    return {
        "shape": list(t.shape),
        "sum": float(f.sum()),
        "sumsq": float((f * f).sum()),
        "head": [float(v) for v in t.detach().float().reshape(-1)[:8]],
        "sha256_fp32": sha(t),
    }


def main() -> None:
    sys.path.insert(0, str(REFERENCE))
    from transformer_benchmark.cases import TransformerConfig, generate_random_case
    from transformer_benchmark.correctness import compare_outputs
    from transformer_benchmark.models import BaselineTransformer
    from transformer_benchmark.timing import percentile

    torch.set_num_threads(8)
    cpu = torch.device("cpu")
    arrays: dict[str, np.ndarray] = {}
    meta: dict = {"weights": {}, "inputs": {}, "forward": {}, "compare": [], "percentile": []}

    # ---- weights --------------------------------------------------------
    weight_cases = {
        "tiny_d32": ((1, 8, 32, 4, 64, 2, True), 0),
        "tiny_d64": ((2, 16, 64, 1, 128, 1, False), 5),
        "c1": ((2, 128, 256, 4, 1024, 2, False), 0),
        "c2": ((1, 128, 512, 8, 2048, 6, False), 1),
        "c3": ((8, 1024, 1024, 16, 4096, 4, True), 2),
        "c4": ((4, 8192, 1024, 16, 4096, 2, True), 3),
        "c5": ((32, 100000, 1024, 16, 1024, 2, False), 4),
    }
    for name, (shape, seed) in weight_cases.items():
        cfg = TransformerConfig(*shape)
        torch.manual_seed(seed)
        model = BaselineTransformer(cfg)
        entry = {"config": list(shape), "seed": seed, "params": {}}
        for key, value in model.state_dict().items():
            entry["params"][key] = summary(value)
            if name.startswith("tiny"):
                arrays[f"w/{name}/{key}"] = value.numpy().astype(np.float32)
        meta["weights"][name] = entry

    # ---- inputs ---------------------------------------------------------
    input_cases = {
        "tiny_pad": ((3, 16, 32, 4, 64, 2, True), 11, 0.5, 1.0),
        "tiny_nopad": ((2, 8, 32, 4, 64, 2, False), 12, 0.0, 2.0),
        "c1": ((2, 128, 256, 4, 1024, 2, False), 0, 0.0, 1.0),
        "c4_cpu": ((4, 8192, 1024, 16, 4096, 2, True), 3, 0.5, 1.0),
    }
    for name, (shape, seed, pad, scale) in input_cases.items():
        cfg = TransformerConfig(*shape)
        x, mask = generate_random_case(cfg, cpu, torch.float32, seed, pad, scale)
        meta["inputs"][name] = {
            "config": list(shape), "seed": seed, "padding_ratio": pad, "input_scale": scale,
            "x": summary(x), "lengths": mask.sum(1).tolist(),
        }
        if name.startswith("tiny"):
            arrays[f"in/{name}/x"] = x.numpy()
            arrays[f"in/{name}/mask"] = mask.numpy()
        else:
            arrays[f"in/{name}/x_row0"] = x[0, :4].numpy()

    # ---- forward outputs ----------------------------------------------
    fwd_cases = {
        # name: (config, weight seed, input seed, padding, dtype)
        "tiny_causal_pad_fp32": ((3, 16, 32, 4, 64, 2, True), 21, 11, 0.5, torch.float32),
        "tiny_noncausal_fp32": ((2, 16, 64, 1, 128, 1, False), 22, 13, 0.0, torch.float32),
        "tiny_causal_pad_bf16": ((3, 16, 32, 4, 64, 2, True), 21, 11, 0.5, torch.bfloat16),
        "tiny_hd64_pad_bf16": ((2, 32, 128, 2, 256, 2, True), 23, 14, 0.4, torch.bfloat16),
        "c1": ((2, 128, 256, 4, 1024, 2, False), 0, 0, 0.0, torch.float32),
    }
    for name, (shape, wseed, xseed, pad, dtype) in fwd_cases.items():
        cfg = TransformerConfig(*shape)
        torch.manual_seed(wseed)
        model = BaselineTransformer(cfg).to(dtype=dtype).eval()
        x, mask = generate_random_case(cfg, cpu, dtype, xseed, pad, 1.0)
        with torch.inference_mode():
            y = model(x, mask)
        entry = {
            "config": list(shape), "weight_seed": wseed, "input_seed": xseed,
            "padding_ratio": pad, "dtype": str(dtype), "y": summary(y),
        }
        if name == "c1":
            rows = [0, 1, 63, 127]
            entry["sample_rows"] = rows
            arrays[f"fwd/{name}/y_rows"] = y[:, rows, :].float().numpy()
        else:
            arrays[f"fwd/{name}/y"] = y.float().numpy()
        meta["forward"][name] = entry

    # ---- correctness rule and percentile KATs ---------------------------
    ref = torch.tensor([1.0, 1.0, 0.5, 0.0, 2.0, float("nan"), 1.0, -3.0])
    opt = torch.tensor([1.016, 1.0159, 0.5099, 0.0099, 2.0, float("nan"), float("inf"), -3.05])
    for rtol, atol in ((0.016, 0.01), (0.02, 0.002)):
        res = compare_outputs(ref, opt, rtol=rtol, atol=atol)
        meta["compare"].append({
            "ref": [float(v) for v in ref], "opt": [float(v) for v in opt], "rtol": rtol, "atol": atol,
            "passed": res.passed, "failed_elements": res.failed_elements,
            "failed_feature_dims": res.failed_feature_dims,
        })
    for values, q in (([3.0, 1.0, 2.0], 0.9), ([5.0], 0.5), ([1.0, 2.0, 3.0, 4.0], 0.9), ([10.0, 0.0], 0.25)):
        meta["percentile"].append({"values": values, "q": q, "result": percentile(values, q)})

    meta["torch_version"] = torch.__version__
    np.savez_compressed(HERE / "reference_vectors.npz", **arrays)
    (HERE / "reference_vectors.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(f"wrote {len(arrays)} arrays and metadata to {HERE}")


if __name__ == "__main__":
    main()
