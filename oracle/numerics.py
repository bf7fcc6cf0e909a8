"""ORACLE -- test infrastructure, never product code.

Independent fp64 numpy forms of the encoder's pieces, written from their
mathematical definitions rather than from torch ops, used to pin the torch
oracle (oracle/encoder_oracle.py) on tiny inputs:

  layer_norm  y = (x - mean) / sqrt(var_biased + eps) * w + b      (nn.LayerNorm)
  gelu        0.5 x (1 + erf(x / sqrt 2))                          (F.gelu, exact)
  attention   explicit per-row softmax over allowed keys           (models.py:55-70)
  encoder     models.py:909-919 composed from the above

``bf16=True`` rounds at the reference's bf16 storage boundaries (every linear
output, the QK product and its scaled value, the probabilities, the context,
each residual sum, each LayerNorm/GELU output) using round-to-nearest-even on the
float32 bit pattern, so bf16 forwards can be checked too.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
from scipy.special import erf


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even); returns float64."""
    f = np.asarray(x, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(np.isfinite(f), out, f.astype(np.float64))


def _r(x: np.ndarray, bf16: bool) -> np.ndarray:
    return bf16_round(x) if bf16 else np.asarray(x, dtype=np.float64)


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * w + b


def gelu(x: np.ndarray) -> np.ndarray:
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    scale: float,
    causal: bool,
    key_valid: Optional[np.ndarray],
    bf16: bool = False,
) -> np.ndarray:
    """q, k, v: [B, H, S, hd] -> context [B, H, S, hd]; explicit loops over rows."""
    b_, h_, s_, _ = q.shape
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(b_):
        for h in range(h_):
            for i in range(s_):
                allowed = np.ones(s_, dtype=bool)
                if causal:
                    allowed[i + 1 :] = False
                if key_valid is not None:
                    allowed &= key_valid[b]
                if not allowed.any():
                    out[b, h, i] = np.nan
                    continue
                s = _r(_r(k[b, h] @ q[b, h, i], bf16) * scale, bf16)
                s = np.where(allowed, s, -np.inf)
                e = np.exp(s - s[allowed].max())
                p = _r(e / e.sum(), bf16)
                out[b, h, i] = _r(p @ v[b, h], bf16)
    return out


def encoder_forward(
    sd: Dict[str, np.ndarray],
    x: np.ndarray,
    valid_token_mask: Optional[np.ndarray],
    causal: bool,
    num_heads: int,
    num_layers: int,
    bf16: bool = False,
    eps: float = 1e-5,
) -> np.ndarray:
    """Reference forward from the definitions above (legacy q/k/v keys)."""
    x = np.asarray(x, dtype=np.float64)
    bsz, s, d = x.shape
    hd = d // num_heads
    row_valid = None if valid_token_mask is None else valid_token_mask[..., None]

    def lin(t: np.ndarray, name: str) -> np.ndarray:
        return _r(t @ sd[name + ".weight"].T + sd[name + ".bias"], bf16)

    def heads(t: np.ndarray) -> np.ndarray:
        return t.reshape(bsz, s, num_heads, hd).transpose(0, 2, 1, 3)

    for layer in range(num_layers):
        p = f"layers.{layer}."
        h = _r(layer_norm(x, sd[p + "norm1.weight"], sd[p + "norm1.bias"], eps), bf16)
        q = heads(lin(h, p + "attention.q_proj"))
        k = heads(lin(h, p + "attention.k_proj"))
        v = heads(lin(h, p + "attention.v_proj"))
        ctx = attention(q, k, v, hd**-0.5, causal, valid_token_mask, bf16)
        ctx = ctx.transpose(0, 2, 1, 3).reshape(bsz, s, d)
        attn = lin(ctx, p + "attention.out_proj")
        if row_valid is not None:
            attn = np.where(row_valid, attn, 0.0)
        x = _r(x + attn, bf16)
        h2 = _r(layer_norm(x, sd[p + "norm2.weight"], sd[p + "norm2.bias"], eps), bf16)
        f = _r(gelu(lin(h2, p + "ffn_in")), bf16)
        x = _r(x + lin(f, p + "ffn_out"), bf16)
        if row_valid is not None:
            x = np.where(row_valid, x, 0.0)
    y = _r(layer_norm(x, sd["final_norm.weight"], sd["final_norm.bias"], eps), bf16)
    if row_valid is not None:
        y = np.where(row_valid, y, 0.0)
    return y
