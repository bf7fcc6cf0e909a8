"""ORACLE -- test infrastructure, never product code.

A from-scratch, functional restatement of the reference Transformer encoder
forward (transformer_benchmark/models.py of Sober7135/TikTokTechJam2026Track3)
written over a plain ``state_dict``, plus the reference's seeded weight init and
input generator.  It runs on whatever device its tensors live on: on the CPU
here, and on torch-ROCm on the GPU box, where it is the checker the HIP path is
compared against.  It is also the timed CPU baseline of ``bench.py``.

Functions and the reference lines they restate:
  init_state_dict   nn.Linear / nn.LayerNorm default init in the module
                    construction order of models.py:20-33, 719-725, 896-907
                    (torch.nn.init.kaiming_uniform_(a=sqrt(5)) + bias U(+-1/sqrt(fan_in)))
  generate_case     cases.py:60-98 (randn, then randint lengths, prefix mask)
  attention_rows    models.py:55-70 (scores, scale, causal/key -inf, fp32
                    softmax -> dtype, PV) for a set of query rows
  encoder_layer     models.py:43-80 + 727-738 (block with residuals, GELU FFN,
                    row masking)
  final_norm        models.py:916-918
  encoder_forward   models.py:909-919
  encoder_forward_sequences
                    models.py:909-919 for a subset of the batch, Linear and
                    LayerNorm on the whole batch (the reference's GEMM shapes)
  compare           correctness.py:63-67 strict OR rule

Parity pinning (tests/test_oracle.py): every function above is checked against
golden vectors written by running the reference itself in this container
(tests/golden/make_golden.py), and the forward additionally against the fp64
brute-force forms in oracle/numerics.py (closed-form LayerNorm, erf GELU,
explicit softmax attention) on tiny inputs.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import torch
import torch.nn.functional as F

# Query rows per score block when the oracle walks long sequences.
ORACLE_ATTENTION_BLOCK_ROWS = 1024

StateDict = Dict[str, torch.Tensor]


# ---------------------------------------------------------------- weights ----

def _kaiming_bound(fan_in: int) -> float:
    a = math.sqrt(5.0)
    gain = math.sqrt(2.0 / (1 + a**2))
    return math.sqrt(3.0) * (gain / math.sqrt(fan_in))


def _linear(out_features: int, in_features: int) -> tuple[torch.Tensor, torch.Tensor]:
    w = torch.empty(out_features, in_features)
    w.uniform_(-_kaiming_bound(in_features), _kaiming_bound(in_features))
    bound = 1.0 / math.sqrt(in_features)
    b = torch.empty(out_features)
    b.uniform_(-bound, bound)
    return w, b


def init_state_dict(
    d_model: int, num_heads: int, ffn_dim: int, num_layers: int, seed: Optional[int] = None
) -> StateDict:
    """Default-init weights in the reference's construction order (CPU, fp32)."""
    if seed is not None:
        torch.manual_seed(seed)
    sd: StateDict = {}
    for i in range(num_layers):
        p = f"layers.{i}."
        sd[p + "norm1.weight"] = torch.ones(d_model)
        sd[p + "norm1.bias"] = torch.zeros(d_model)
        for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
            w, b = _linear(d_model, d_model)
            sd[f"{p}attention.{name}.weight"] = w
            sd[f"{p}attention.{name}.bias"] = b
        sd[p + "norm2.weight"] = torch.ones(d_model)
        sd[p + "norm2.bias"] = torch.zeros(d_model)
        sd[p + "ffn_in.weight"], sd[p + "ffn_in.bias"] = _linear(ffn_dim, d_model)
        sd[p + "ffn_out.weight"], sd[p + "ffn_out.bias"] = _linear(d_model, ffn_dim)
    sd["final_norm.weight"] = torch.ones(d_model)
    sd["final_norm.bias"] = torch.zeros(d_model)
    return sd


def pack_qkv(sd: StateDict) -> StateDict:
    """Legacy q/k/v keys -> packed qkv_proj (rows q, then k, then v)."""
    out: StateDict = {}
    for key, value in sd.items():
        if ".attention.q_proj." in key:
            kind = key.rsplit(".", 1)[1]
            prefix = key.split("q_proj.")[0]
            out[f"{prefix}qkv_proj.{kind}"] = torch.cat(
                [sd[f"{prefix}{n}.{kind}"] for n in ("q_proj", "k_proj", "v_proj")], dim=0
            )
        elif ".attention.k_proj." in key or ".attention.v_proj." in key:
            continue
        else:
            out[key] = value
    return out


# ----------------------------------------------------------------- inputs ----

def generate_case(
    batch: int,
    seq_len: int,
    d_model: int,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float = 1.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(batch, seq_len, d_model, generator=gen, device=device, dtype=dtype)
    x = x * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(batch, seq_len, device=device, dtype=torch.bool)
    low = max(1, int(round(seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low, seq_len + 1, (batch,), generator=gen, device=device)
    mask = torch.arange(seq_len, device=device)[None, :] < lengths[:, None]
    return x.masked_fill(~mask[..., None], 0), mask


# -------------------------------------------------------------- attention ----

def attention_rows(
    q_rows: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal: bool,
    valid_token_mask: Optional[torch.Tensor],
    row_positions: torch.Tensor,
) -> torch.Tensor:
    """Context for the query rows ``q_rows`` [B, H, R, hd] at sequence positions
    ``row_positions`` [R]: bf16(softmax_fp32(bf16(q k^T) * scale masked)) @ v."""
    k_t = k.transpose(-2, -1)
    if k_t.is_cuda:
        # bf16 batched products with a transposed right operand are not run on
        # the GPU; the contiguous copy holds the same values
        k_t = k_t.contiguous()
    scores = torch.matmul(q_rows, k_t) * scale
    if causal:
        keys = torch.arange(k.shape[-2], device=k.device)
        future = keys[None, :] > row_positions.to(k.device)[:, None]
        scores = scores.masked_fill(future, float("-inf"))
    if valid_token_mask is not None:
        scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores.float(), dim=-1).to(dtype=q_rows.dtype)
    return torch.matmul(probs, v)


def even_block_rows(seq_len: int, limit: int = ORACLE_ATTENTION_BLOCK_ROWS) -> int:
    """Largest query-row block size <= limit that divides seq_len (at least
    half of limit), else limit.  Equal blocks give every block the same
    product shape, so the library accumulates each one the same way; a
    ragged last block can be given a different K order (e.g. at S = 100000
    with 1024-row blocks, the 672-row tail block's P.V product differs from
    the others' in the last bit)."""
    if seq_len <= limit:
        return seq_len
    for rows in range(limit, limit // 2 - 1, -1):
        if seq_len % rows == 0:
            return rows
    return limit


def _heads(t: torch.Tensor, num_heads: int) -> torch.Tensor:
    b, s, d = t.shape
    return t.view(b, s, num_heads, d // num_heads).transpose(1, 2).contiguous()


def encoder_layer(
    sd: StateDict,
    layer: int,
    x: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor],
    causal: bool,
    num_heads: int,
    rows: Optional[torch.Tensor] = None,
    eps: float = 1e-5,
    block_rows: int = ORACLE_ATTENTION_BLOCK_ROWS,
) -> torch.Tensor:
    """One encoder block.  With ``rows`` (1-D positions) only those sequence
    positions are produced ([B, len(rows), D]); keys/values still use all rows."""
    p = f"layers.{layer}."
    a = f"{p}attention."
    b, s, d = x.shape
    hd = d // num_heads
    scale = hd**-0.5
    h = F.layer_norm(x, (d,), sd[p + "norm1.weight"], sd[p + "norm1.bias"], eps)
    k = _heads(F.linear(h, sd[a + "k_proj.weight"], sd[a + "k_proj.bias"]), num_heads)
    v = _heads(F.linear(h, sd[a + "v_proj.weight"], sd[a + "v_proj.bias"]), num_heads)
    if rows is None:
        rows = torch.arange(s, device=x.device)
    rows = rows.to(x.device)
    x_rows = x[:, rows, :]
    h_rows = h[:, rows, :]
    q = _heads(F.linear(h_rows, sd[a + "q_proj.weight"], sd[a + "q_proj.bias"]), num_heads)
    r = rows.numel()
    context = torch.empty(b, num_heads, r, hd, device=x.device, dtype=x.dtype)
    for start in range(0, r, block_rows):
        stop = min(r, start + block_rows)
        context[:, :, start:stop] = attention_rows(
            q[:, :, start:stop], k, v, scale, causal, valid_token_mask, rows[start:stop]
        )
    context = context.transpose(1, 2).contiguous().view(b, r, d)
    attn = F.linear(context, sd[a + "out_proj.weight"], sd[a + "out_proj.bias"])
    row_mask = None if valid_token_mask is None else valid_token_mask[:, rows]
    if row_mask is not None:
        attn = attn.masked_fill(~row_mask[..., None], 0)
    y = x_rows + attn
    h2 = F.layer_norm(y, (d,), sd[p + "norm2.weight"], sd[p + "norm2.bias"], eps)
    ffn = F.linear(
        F.gelu(F.linear(h2, sd[p + "ffn_in.weight"], sd[p + "ffn_in.bias"]), approximate="none"),
        sd[p + "ffn_out.weight"],
        sd[p + "ffn_out.bias"],
    )
    y = y + ffn
    if row_mask is not None:
        y = y.masked_fill(~row_mask[..., None], 0)
    return y


def encoder_forward_sequences(
    sd: StateDict,
    x: torch.Tensor,
    sequences: Sequence[int],
    causal: bool,
    num_heads: int,
    num_layers: int,
    eps: float = 1e-5,
    block_rows: Optional[int] = None,
) -> torch.Tensor:
    """The reference forward (no mask) evaluated for the listed sequences only,
    with every Linear and LayerNorm run on the whole [B, S, D] batch exactly as
    the reference runs them (models.py:30-33, 721-725: nn.Linear flattens the
    batch into one [B*S, D] product, whose accumulation order the library picks
    for that whole shape).  Attention, whose score tensor would not fit, is the
    row-blocked restatement of models.py:55-70 for the listed sequences; the
    other sequences' contexts are left zero, which changes nothing for the
    listed ones because every Linear and LayerNorm row depends only on its own
    input row.  Returns [len(sequences), S, D]."""
    b, s, d = x.shape
    hd = d // num_heads
    scale = hd**-0.5
    rows = torch.arange(s, device=x.device)
    if block_rows is None:
        block_rows = even_block_rows(s)
    for layer in range(num_layers):
        p = f"layers.{layer}."
        a = f"{p}attention."
        h = F.layer_norm(x, (d,), sd[p + "norm1.weight"], sd[p + "norm1.bias"], eps)
        context = torch.zeros(b, s, d, device=x.device, dtype=x.dtype)
        q_all = F.linear(h, sd[a + "q_proj.weight"], sd[a + "q_proj.bias"])
        k_all = F.linear(h, sd[a + "k_proj.weight"], sd[a + "k_proj.bias"])
        v_all = F.linear(h, sd[a + "v_proj.weight"], sd[a + "v_proj.bias"])
        del h
        for seq in sequences:
            q = _heads(q_all[seq : seq + 1], num_heads)
            k = _heads(k_all[seq : seq + 1], num_heads)
            v = _heads(v_all[seq : seq + 1], num_heads)
            ctx = torch.empty_like(q)
            for start in range(0, s, block_rows):
                stop = min(s, start + block_rows)
                ctx[:, :, start:stop] = attention_rows(
                    q[:, :, start:stop], k, v, scale, causal, None, rows[start:stop]
                )
            context[seq] = ctx.transpose(1, 2).reshape(s, d)
            del q, k, v, ctx
        del q_all, k_all, v_all
        x = x + F.linear(context, sd[a + "out_proj.weight"], sd[a + "out_proj.bias"])
        del context
        h2 = F.layer_norm(x, (d,), sd[p + "norm2.weight"], sd[p + "norm2.bias"], eps)
        hidden = F.gelu(F.linear(h2, sd[p + "ffn_in.weight"], sd[p + "ffn_in.bias"]), approximate="none")
        del h2
        x = x + F.linear(hidden, sd[p + "ffn_out.weight"], sd[p + "ffn_out.bias"])
        del hidden
    y = F.layer_norm(x, (d,), sd["final_norm.weight"], sd["final_norm.bias"], eps)
    return y[list(sequences)]


def final_norm(
    sd: StateDict, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor], eps: float = 1e-5
) -> torch.Tensor:
    y = F.layer_norm(x, (x.shape[-1],), sd["final_norm.weight"], sd["final_norm.bias"], eps)
    if valid_token_mask is not None:
        y = y.masked_fill(~valid_token_mask[..., None], 0)
    return y


def encoder_forward(
    sd: StateDict,
    x: torch.Tensor,
    valid_token_mask: Optional[torch.Tensor],
    causal: bool,
    num_heads: int,
    num_layers: int,
    eps: float = 1e-5,
    block_rows: int = ORACLE_ATTENTION_BLOCK_ROWS,
) -> torch.Tensor:
    """The full reference forward: L blocks then the final LayerNorm."""
    for layer in range(num_layers):
        x = encoder_layer(sd, layer, x, valid_token_mask, causal, num_heads, eps=eps, block_rows=block_rows)
    return final_norm(sd, x, valid_token_mask, eps)


# -------------------------------------------------------------- checking ----

def compare(reference: torch.Tensor, candidate: torch.Tensor, rtol: float, atol: float) -> Dict[str, object]:
    """Strict OR rule |c - r| < atol or |c - r| < rtol |r| on finite values."""
    ref = reference.detach().float()
    cand = candidate.detach().float()
    err = (cand - ref).abs()
    finite = torch.isfinite(ref) & torch.isfinite(cand)
    ok = finite & ((err < atol) | (err < rtol * ref.abs()))
    failed = int((~ok).sum().item())
    return {
        "passed": failed == 0,
        "failed": failed,
        "total": ref.numel(),
        "max_abs_error": float(err.max().item()) if err.numel() else 0.0,
        "allclose": bool((finite & (err <= atol + rtol * ref.abs())).all().item()),
    }


def select_rows(x: torch.Tensor, rows: Sequence[int]) -> torch.Tensor:
    return x[:, torch.as_tensor(list(rows), device=x.device), :]
