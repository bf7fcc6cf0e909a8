"""enc_encoder_forward_bf16_noalloc (the entry point that allocates nothing)
against enc_encoder_forward_bf16 with a caller workspace, through the C ABI.

Both run the same kernels over the same inputs, so the outputs must be equal
bit for bit; the second call uses a smaller input (the array keeps the first
call's contents) and a prefix mask.  A shape whose workspace exceeds the
library's scratch array is rejected before anything is launched.
"""

import pytest
import torch

from tiktoktechjam2026track3_amd import native
from tiktoktechjam2026track3_amd.cases import ENCODER_CONFIGS, TransformerConfig, generate_random_case
from tiktoktechjam2026track3_amd.models import BaselineTransformer, UserOptimizedTransformer, copy_model_weights

pytestmark = pytest.mark.gpu


def _model(cfg, seed, device):
    torch.manual_seed(seed)
    baseline = BaselineTransformer(cfg)
    candidate = UserOptimizedTransformer(cfg)
    copy_model_weights(baseline, candidate)
    return candidate.to(device=device, dtype=torch.bfloat16).eval()


def _both(model, x, mask, rows=None):
    cfg = model.config
    table, eps, packed = model._native_weights(x.device, x.shape[0] * x.shape[1] if rows is None else rows)
    kv_len = row_mask = None
    if mask is not None and not bool(mask.all()):
        kv_len = native.mask_lengths(mask)
        row_mask = mask.contiguous().view(torch.uint8)
    b, s, d = x.shape
    workspace = torch.empty(native.encoder_workspace_bytes(b, s, d, cfg.num_heads, cfg.ffn_dim),
                            device=x.device, dtype=torch.uint8)
    ref = torch.empty_like(x)
    native.encoder_forward(x, ref, workspace, table, cfg.num_heads, cfg.ffn_dim, cfg.num_layers, eps,
                           cfg.causal, kv_len, None, row_mask, packed_weights=packed)
    out = torch.full_like(x, float("nan"))
    native.encoder_forward_noalloc(x, out, table, cfg.num_heads, cfg.ffn_dim, cfg.num_layers, eps,
                                   cfg.causal, kv_len, None, row_mask, packed_weights=packed)
    torch.cuda.synchronize()
    return ref, out


def test_noalloc_forward_matches_workspace_forward(device):
    spec = ENCODER_CONFIGS["c2"]
    model = _model(spec.config, spec.seed, device)
    with torch.inference_mode():
        x, mask = generate_random_case(spec.config, device, torch.bfloat16, spec.seed + 100000, 0.0, 1.0)
        ref, out = _both(model, x, mask)
        print(f"[noalloc] c2 first call equal={torch.equal(ref, out)}", flush=True)
        assert torch.equal(ref, out)
        # second call, smaller input (64 tokens, prefix padding): the array still
        # holds the first call's activations
        small = TransformerConfig(1, 64, 512, 8, 2048, 6, True)
        x2, mask2 = generate_random_case(small, device, torch.bfloat16, 5, 0.3, 1.0)
        model.config = small
        ref2, out2 = _both(model, x2, mask2)
        print(f"[noalloc] smaller second call equal={torch.equal(ref2, out2)}", flush=True)
        assert torch.equal(ref2, out2)
        assert torch.all(out2[~mask2] == 0)


@pytest.mark.parametrize("packed", [False, True], ids=["plain_weights", "packed_weights"])
def test_noalloc_forward_at_a_wide_tile_shape(device, packed):
    """2304 tokens at d_model 1024 / ffn 4096 (a 52 MB workspace, within the
    64 MiB array): the wide GEMM tiles, the 256 x 256 GELU tile (which keeps
    three words in scratch), the GELU table and, with packed_weights, the
    tile-packed weights.  Bitwise against the workspace forward, twice; the
    second no-allocation call leaves the device's free memory unchanged."""
    from tiktoktechjam2026track3_amd import linear_order

    cfg = TransformerConfig(1, 2304, 1024, 16, 4096, 1, True)
    need = native.encoder_workspace_bytes(1, 2304, 1024, 16, 4096)
    assert need <= native.NOALLOC_SCRATCH_BYTES
    model = _model(cfg, 11, device)
    rows = 2304 if packed else 0  # 0 rows: below the packing threshold, plain weights only
    with torch.inference_mode():
        linear_order.ensure_encoder(2304, 1024, 4096, device)
        x, mask = generate_random_case(cfg, device, torch.bfloat16, 12, 0.3, 1.0)
        ref, out = _both(model, x, mask, rows)
        assert torch.equal(ref, out)
        table, eps, used_packed = model._native_weights(device, rows)
        assert used_packed == packed
        kv_len = native.mask_lengths(mask)
        row_mask = mask.contiguous().view(torch.uint8)
        out2 = torch.full_like(x, float("nan"))
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info(device)[0]
        native.encoder_forward_noalloc(x, out2, table, cfg.num_heads, cfg.ffn_dim, cfg.num_layers, eps,
                                       cfg.causal, kv_len, None, row_mask, packed_weights=used_packed)
        torch.cuda.synchronize()
        free_after = torch.cuda.mem_get_info(device)[0]
    print(f"[noalloc] wide tiles packed={packed}: equal={torch.equal(ref, out2)}, "
          f"free memory {free_before} -> {free_after}", flush=True)
    assert torch.equal(ref, out2)
    assert free_after == free_before


def test_noalloc_rejects_shapes_above_the_scratch_array(device):
    spec = ENCODER_CONFIGS["c3"]
    cfg = spec.config
    need = native.encoder_workspace_bytes(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim)
    assert need > native.NOALLOC_SCRATCH_BYTES
    model = _model(TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads, cfg.ffn_dim, 1,
                                     cfg.causal), spec.seed, device)
    table, eps, _ = model._native_weights(device)
    x = torch.zeros(cfg.batch_size, cfg.seq_len, cfg.d_model, device=device, dtype=torch.bfloat16)
    out = torch.empty_like(x)
    with pytest.raises(native.EncoderKernelError, match="scratch array") as info:
        native.encoder_forward_noalloc(x, out, table, cfg.num_heads, cfg.ffn_dim, 1, eps, cfg.causal,
                                       None, None, None)
    assert info.value.code == native.ENC_ERR_UNSUPPORTED
