"""Host-side contracts that need no GPU.

The C-ABI library loads here and exports every entry point its header
declares.  The candidate module keeps the reference's plugin contracts
(transformer_benchmark/models.py, tests/test_models.py of the reference): CPU
fallback op order, the packed Q/K/V state dict, mask classification and graph
replay returning independent clones.  The rocprof summary tool parses the CSV
layout rocprofv3 writes.
"""

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from tiktoktechjam2026track3_amd import native, profiling
from tiktoktechjam2026track3_amd.cases import OFFICIAL_TEST_CASES, TransformerConfig
from tiktoktechjam2026track3_amd.correctness import compare_outputs
from tiktoktechjam2026track3_amd.models import (
    BaselineTransformer,
    UnsupportedShapeError,
    UserOptimizedTransformer,
    classify_mask,
    copy_model_weights,
)

ROOT = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------------ C ABI ----

def declared_entry_points():
    text = (ROOT / "include" / "mi355x_encoder.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(enc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    lib = ctypes.CDLL(str(native.LIBRARY_PATH))
    names = declared_entry_points()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_binding_covers_the_header_exactly():
    assert sorted(name for name, _, _ in native.SIGNATURES) == declared_entry_points()


def test_library_reports_version_and_errors_without_a_gpu():
    lib = native.load_library()
    assert lib.enc_version() >> 16 == 1
    # argument validation happens before any device call
    rc = lib.enc_layernorm_bf16(None, None, None, None, 4, 256, 1e-5, None, None)
    assert rc == native.ENC_ERR_INVALID
    assert b"null" in lib.enc_last_error()
    rc = lib.enc_linear_bf16(None, None, None, None, None, 4, 100, 64, 0, None, None)
    assert rc in (native.ENC_ERR_INVALID, native.ENC_ERR_UNSUPPORTED)
    assert lib.enc_encoder_workspace_bytes(1, 128, 512, 8, 2048) > 0
    assert lib.enc_encoder_workspace_bytes(1, 128, 500, 8, 2048) == -1  # D % H != 0


# -------------------------------------------------------- plugin contracts ----

def _pair(config, seed):
    torch.manual_seed(seed)
    baseline = BaselineTransformer(config).eval()
    optimized = UserOptimizedTransformer(config).eval()
    copy_model_weights(baseline, optimized)
    return baseline, optimized


def test_cpu_candidate_is_bitwise_the_baseline_in_fp32():
    """The CPU path runs the baseline's op sequence (reference
    tests/test_models.py:53-67 pins the same property with torch.equal)."""
    config = TransformerConfig(4, 8, 16, 4, 32, 1, True)
    baseline, optimized = _pair(config, 4321)
    x = torch.randn(4, 8, 16)
    mask = torch.ones(4, 8, dtype=torch.bool)
    mask[1, -3:] = False
    x = x.masked_fill(~mask[..., None], 0)
    with torch.inference_mode():
        assert torch.equal(baseline(x, mask), optimized(x, mask))


def test_cpu_candidate_with_padding_passes_reference_gate():
    config = TransformerConfig(1, 128, 128, 4, 128, 2, True)
    baseline, optimized = _pair(config, 1234)
    x = torch.randn(1, 128, 128)
    mask = torch.ones(1, 128, dtype=torch.bool)
    mask[:, -32:] = False
    x = x.masked_fill(~mask[..., None], 0)
    with torch.inference_mode():
        result = compare_outputs(baseline(x, mask), optimized(x, mask), rtol=0.02, atol=0.002)
    assert result.passed
    assert optimized._cuda_graph is None


def test_legacy_qkv_state_dict_is_packed_q_then_k_then_v():
    config = TransformerConfig(1, 8, 16, 4, 32, 1, False)
    baseline, optimized = _pair(config, 7)
    attn_b = baseline.layers[0].attention
    attn_o = optimized.layers[0].attention
    expected_w = torch.cat([attn_b.q_proj.weight, attn_b.k_proj.weight, attn_b.v_proj.weight])
    expected_b = torch.cat([attn_b.q_proj.bias, attn_b.k_proj.bias, attn_b.v_proj.bias])
    assert torch.equal(attn_o.qkv_proj.weight, expected_w)
    assert torch.equal(attn_o.qkv_proj.bias, expected_b)


def test_packed_state_dict_round_trips_strictly():
    config = TransformerConfig(1, 8, 16, 4, 32, 2, False)
    _, optimized = _pair(config, 8)
    other = UserOptimizedTransformer(config)
    other.load_state_dict(optimized.state_dict(), strict=True)
    for (k1, v1), (k2, v2) in zip(optimized.state_dict().items(), other.state_dict().items()):
        assert k1 == k2 and torch.equal(v1, v2)


def test_incomplete_or_ambiguous_legacy_state_is_rejected():
    config = TransformerConfig(1, 8, 16, 4, 32, 1, False)
    baseline, _ = _pair(config, 9)
    sd = baseline.state_dict()
    incomplete = {k: v for k, v in sd.items() if "v_proj.bias" not in k}
    with pytest.raises(RuntimeError, match="incomplete legacy"):
        UserOptimizedTransformer(config).load_state_dict(incomplete)
    ambiguous = dict(sd)
    ambiguous["layers.0.attention.qkv_proj.weight"] = torch.zeros(48, 16)
    with pytest.raises(RuntimeError, match="ambiguous"):
        UserOptimizedTransformer(config).load_state_dict(ambiguous)


def test_mask_classes():
    assert classify_mask(torch.ones(2, 8, dtype=torch.bool)) == "all_true"
    prefix = torch.arange(8)[None, :] < torch.tensor([[5], [8]])
    assert classify_mask(prefix) == "prefix"
    general = prefix.clone()
    general[0, 1] = False
    assert classify_mask(general) == "general"


def test_mask_classification_tracks_mutation_and_inference_tensors():
    config = TransformerConfig(1, 128, 128, 4, 128, 4, True)
    optimized = UserOptimizedTransformer(config).eval()
    mask = torch.ones(1, 128, dtype=torch.bool)
    assert optimized._mask_is_all_true(mask)
    mask[0, -1] = False
    assert not optimized._mask_is_all_true(mask)
    with torch.inference_mode():
        inference_mask = torch.ones(1, 128, dtype=torch.bool)
        assert optimized._mask_is_all_true(inference_mask)
        inference_mask[0, -1] = False
        assert not optimized._mask_is_all_true(inference_mask)


def test_graph_replay_returns_independent_outputs():
    """Replays hand back clones of the static output (reference
    tests/test_models.py:666-691)."""
    config = TransformerConfig(1, 8, 16, 4, 32, 1, True)
    optimized = UserOptimizedTransformer(config).eval()
    static_output = torch.zeros(1)

    class FakeGraph:
        def replay(self) -> None:
            static_output.add_(1)

    optimized._cuda_graph = FakeGraph()
    optimized._cuda_graph_output = static_output
    optimized._cuda_graph_signature = ("stable",)
    optimized._cuda_graph_eligible = lambda _x, _mask: True
    optimized._cuda_graph_live_signature = lambda _x, _mask, _kind: ("stable",)
    x = torch.zeros(1, 8, 16)
    mask = torch.ones(1, 8, dtype=torch.bool)
    first = optimized(x, mask)
    second = optimized(x, mask)
    assert first is not second
    assert first.item() == 1.0 and second.item() == 2.0


def test_native_path_rejects_shapes_the_kernels_do_not_cover():
    config = TransformerConfig(1, 8, 128, 8, 128, 1, False)  # head_dim 16
    model = UserOptimizedTransformer(config)
    with pytest.raises(UnsupportedShapeError, match="head_dim 16"):
        model._check_native_supported(torch.zeros(1, 8, 128, dtype=torch.bfloat16))
    odd_ffn = UserOptimizedTransformer(TransformerConfig(1, 8, 128, 4, 48, 1, False))  # ffn_dim 48
    with pytest.raises(UnsupportedShapeError, match="multiple of 32"):
        odd_ffn._check_native_supported(torch.zeros(1, 8, 128, dtype=torch.bfloat16))
    # every official case's shape is covered (head dims 8 to 256, d_model 32 to 1024)
    for case in OFFICIAL_TEST_CASES:
        small = TransformerConfig(1, 8, case.d_model, case.num_heads, case.ffn_dim, 1, case.causal)
        UserOptimizedTransformer(small)._check_native_supported(
            torch.zeros(1, 8, case.d_model, dtype=torch.bfloat16))
    with pytest.raises(UnsupportedShapeError, match="bfloat16"):
        model._check_native_supported(torch.zeros(1, 8, 128))


def test_dispatch_rule_autograd_dtype_and_native_only():
    # the native forward runs only where every reference route would run its
    # custom kernels (no autograd history, BF16, a covered shape); the rest
    # takes the logged torch fallback, or raises under native_only
    config = TransformerConfig(1, 8, 128, 4, 128, 1, False)
    model = UserOptimizedTransformer(config)
    x = torch.randn(1, 8, 128).bfloat16()
    with torch.no_grad():
        assert model._fallback_reason(x) is None
        assert "bfloat16" in model._fallback_reason(x.float())
    assert "autograd" in model._fallback_reason(x)  # grad enabled, parameters require grad
    for p in model.parameters():
        p.requires_grad_(False)
    assert model._fallback_reason(x) is None
    assert "autograd" in model._fallback_reason(x.float().requires_grad_())
    model = model.bfloat16().eval()
    model.native_only = True
    with pytest.raises(UnsupportedShapeError, match="native_only"):
        model._forward_fallback(x, None, "a reason")
    model.native_only = False
    with torch.inference_mode():
        out = model._forward_fallback(x, None, "a reason")
        out2 = model._forward_fallback(x, None, "a reason")
        ref = model._forward_eager(x, None)
    assert torch.equal(out, ref) and torch.equal(out2, ref)
    assert model.fallback_calls == {"a reason": 2} and model.native_calls == 0
    # the test session runs strict (tests/conftest.py)
    assert UserOptimizedTransformer.native_only


# --------------------------------------------------------------- profiling ----

def _write_csv(path: Path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    lines = [",".join(f'"{h}"' for h in header)]
    for row in rows:
        lines.append(",".join(f'"{v}"' if isinstance(v, str) else str(v) for v in row))
    path.write_text("\n".join(lines) + "\n")


def test_profiling_summary_scales_counters_by_the_copy_calibration(tmp_path):
    stats_header = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"]
    _write_csv(tmp_path / "trace" / "run_kernel_stats.csv", stats_header, [
        ["void enc::(anonymous namespace)::gemm_big_kernel<256, 128>(unsigned short const*)", 4, 400.0, 100.0, 80.0, 90, 110, 1.0],
        ["at::cuda::(anonymous namespace)::spin_kernel(long)", 1, 1e9, 1e9, 10.0, 1, 1, 0.0],
        ["__amd_rocclr_copyBuffer", 2, 100.0, 50.0, 20.0, 40, 60, 1.0],
    ])
    pmc_header = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
                  "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
                  "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    gemm = "void enc::(anonymous namespace)::gemm_big_kernel<256, 128>(unsigned short const*)"
    for kind, counter, gemm_vals, copy_val in (("fetch", "FETCH_SIZE", (100.0, 300.0), 1024.0 * 8),
                                               ("write", "WRITE_SIZE", (50.0, 50.0), 1024.0 * 16)):
        rows = [[i, i, "Agent 1", 1, 1, 1, 256, 1, gemm, 256, 0, 0, 64, 0, 32, counter, v, 0, 1]
                for i, v in enumerate(gemm_vals)]
        rows.append([9, 9, "Agent 1", 1, 1, 1, 256, 2, "__amd_rocclr_copyBuffer", 256, 0, 0, 8, 0, 8, counter, copy_val, 0, 1])
        rows.append([10, 10, "Agent 1", 1, 1, 1, 256, 2, "__amd_rocclr_copyBuffer", 256, 0, 0, 8, 0, 8, counter, 3.0, 0, 1])
        _write_csv(tmp_path / kind / "run_counter_collection.csv", pmc_header, rows)
    out = tmp_path / "summary.md"
    traffic = tmp_path / "traffic.json"
    rc = profiling.main([
        "--trace", str(tmp_path / "trace"), "--fetch", str(tmp_path / "fetch"), "--write", str(tmp_path / "write"),
        "--copy-mib", "16", "--workload", "cX", "--label", "gemm=gemm_big_kernel<256, 128>",
        "--algorithmic-bytes", "gemm=1000000", "--out", str(out), "--traffic", str(traffic),
    ])
    assert rc == 0
    table = json.loads(traffic.read_text())["gemm@cX"]
    # fetch: 16 MiB copy read 8192 units -> 2048 bytes per unit; mean 200 units
    assert table["fetched"] == 200 * 2048
    # write: 16 MiB copy wrote 16384 units -> 1024 bytes per unit; mean 50 units
    assert table["written"] == 50 * 1024
    assert table["bytes_per_launch"] == 200 * 2048 + 50 * 1024
    text = out.read_text()
    assert "gemm_big_kernel<256, 128>" in text and "spin_kernel" not in text


def test_profiling_summary_reports_mfma_utilisation(tmp_path):
    stats_header = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"]
    gemm = "void enc::(anonymous namespace)::gemm_big_kernel<256, 128>(unsigned short const*)"
    _write_csv(tmp_path / "trace" / "run_kernel_stats.csv", stats_header, [[gemm, 2, 200.0, 100.0, 100.0, 90, 110, 1.0]])
    pmc_header = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
                  "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
                  "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    rows = []
    # dispatch 1: busy 1024 SIMDs x 400 cycles of 8 XCDs x 1000 active -> 40%; dispatch 2: 60%
    for i, busy in ((1, 409600.0), (2, 614400.0)):
        rows.append([i, i, "Agent 1", 1, 1, 1, 256, 1, gemm, 256, 0, 0, 64, 0, 32, "SQ_VALU_MFMA_BUSY_CYCLES", busy, 0, 1])
        rows.append([i, i, "Agent 1", 1, 1, 1, 256, 1, gemm, 256, 0, 0, 64, 0, 32, "GRBM_GUI_ACTIVE", 8000.0, 0, 1])
    _write_csv(tmp_path / "mfma" / "run_counter_collection.csv", pmc_header, rows)
    util, n = profiling.mfma_utilisation(str(tmp_path / "mfma"), "gemm_big_kernel<256, 128>", 1024, 8)
    assert n == 2 and util == pytest.approx(0.5)
    out = tmp_path / "summary.md"
    assert profiling.main(["--trace", str(tmp_path / "trace"), "--mfma", str(tmp_path / "mfma"), "--workload", "cX",
                           "--label", "gemm=gemm_big_kernel<256, 128>", "--out", str(out)]) == 0
    assert "| gemm (`gemm_big_kernel<256, 128>`) | 2 | 50.0% |" in out.read_text()


def test_noalloc_entry_point_rejects_large_shapes_before_any_device_call():
    """The workspace-size check of enc_encoder_forward_bf16_noalloc runs before
    any HIP call (here there is no GPU): a c3-sized forward needs more than the
    library's scratch array."""
    lib = native.load_library()
    layers = 1
    table = (ctypes.c_void_p * (12 * layers + 2))(*([1] * (12 * layers + 2)))
    fake = ctypes.c_void_p(16)
    rc = lib.enc_encoder_forward_bf16_noalloc(
        fake, fake, ctypes.cast(table, ctypes.c_void_p), 8, 1024, 1024, 16, 4096, layers, 1e-5, 1,
        None, None, None, 0, None,
    )
    assert rc == native.ENC_ERR_UNSUPPORTED
    assert b"scratch array" in lib.enc_last_error()
    assert lib.enc_encoder_workspace_bytes(8, 1024, 1024, 16, 4096) > native.NOALLOC_SCRATCH_BYTES


def test_prepack_argument_checks_match_the_python_rule():
    """enc_prepack_weight_bf16 rejects every shape without a packed form before
    any device call, exactly where native.prepack_rows says there is none."""
    lib = native.load_library()
    fake_w, fake_p = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    for n in (32, 96, 128, 200, 256, 384, 1000, 1024, 1536, 3072):
        for k in (16, 32, 48, 1024):
            if native.prepack_rows(n, k):
                assert native.prepack_rows(n, k) == (256 if n % 256 == 0 else 128)
                continue
            rc = lib.enc_prepack_weight_bf16(fake_w, fake_p, n, k, None)
            assert rc == native.ENC_ERR_UNSUPPORTED, (n, k)
    assert lib.enc_prepack_weight_bf16(fake_w, fake_w, 256, 32, None) == native.ENC_ERR_INVALID  # aliasing
    assert lib.enc_prepack_weight_bf16(None, fake_p, 256, 32, None) == native.ENC_ERR_INVALID


def test_encoder_packed_flag_needs_the_packed_pointers():
    """With ENC_FWD_PACKED_WEIGHTS the table holds 4 more pointers per layer;
    a null one among them, or a shape without a packed form, is rejected
    before any device call."""
    lib = native.load_library()
    layers = 2
    n_ptrs = 16 * layers + 2
    ptrs = [64 * (i + 1) for i in range(n_ptrs)]
    ptrs[12 * layers + 2 + 5] = 0  # layer 1's packed out_proj weight
    table = (ctypes.c_void_p * n_ptrs)(*ptrs)
    fake = ctypes.c_void_p(16)
    ws = ctypes.c_void_p(1 << 20)
    rc = lib.enc_encoder_forward_bf16(fake, fake, ws, 1 << 40, ctypes.cast(table, ctypes.c_void_p), 1, 2048, 1024,
                                      16, 4096, layers, 1e-5, 1, None, None, None, native.ENC_FWD_PACKED_WEIGHTS,
                                      None)
    assert rc == native.ENC_ERR_INVALID and b"index 31" in lib.enc_last_error()
    table = (ctypes.c_void_p * (16 + 2))(*([64] * 18))
    rc = lib.enc_encoder_forward_bf16(fake, fake, ws, 1 << 40, ctypes.cast(table, ctypes.c_void_p), 1, 2048, 1024,
                                      16, 4000, 1, 1e-5, 1, None, None, None, native.ENC_FWD_PACKED_WEIGHTS, None)
    assert rc == native.ENC_ERR_UNSUPPORTED and b"packed weights" in lib.enc_last_error()
    with pytest.raises(ValueError, match="18 device pointers"):
        native._forward_flags(False, True, True, torch.zeros(14, dtype=torch.int64), 1)


def test_ffn_entry_point_checks_arguments_before_any_device_call():
    lib = native.load_library()
    p = [ctypes.c_void_p(4096 * (i + 1)) for i in range(7)]
    hidden = ctypes.c_void_p(1 << 30)
    rc = lib.enc_ffn_fused_bf16(*p[:7], hidden, 128, 512, 2000, None, None)
    assert rc == native.ENC_ERR_UNSUPPORTED and b"multiples of 32" in lib.enc_last_error()
    rc = lib.enc_ffn_fused_bf16(*p[:6], None, hidden, 128, 512, 2048, None, None)
    assert rc == native.ENC_ERR_INVALID and b"null" in lib.enc_last_error()
    # hidden overlapping the input rows (h at 4096, 128 x 512 bf16 = 128 KiB)
    rc = lib.enc_ffn_fused_bf16(*p[:7], ctypes.c_void_p(4096 + 1024), 128, 512, 2048, None, None)
    assert rc == native.ENC_ERR_INVALID and b"overlap" in lib.enc_last_error()
    assert lib.enc_ffn_fused_bf16(*p[:7], hidden, 0, 512, 2048, None, None) == native.ENC_OK
