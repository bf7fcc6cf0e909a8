"""ctypes binding of libmi355x_encoder.so (the C ABI in include/mi355x_encoder.h).

The library is loaded once, under a lock, the way the reference loads its native
extensions (transformer_benchmark/native_softmax_bf16.py:16-17, 129-136) and binds
a C library through ctypes with explicit argtypes/restype and status codes mapped
to Python exceptions (transformer_benchmark/cublaslt_linear.py:57-60, 71-144).

There is no fallback: if the library is missing or fails to load, every call
raises ``NativeLibraryError`` naming the path and the build command.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libmi355x_encoder.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "mi355x_encoder.h"

ENC_OK = 0
ENC_ERR_INVALID = 1
ENC_ERR_UNSUPPORTED = 2
ENC_ERR_HIP = 3
ENC_ERR_OOM = 4

ENC_FWD_ONLINE_ATTENTION = 1
ENC_FWD_SKIP_FINAL_NORM = 2
ENC_FWD_PACKED_WEIGHTS = 4

ENC_EPI_BIAS = 0
ENC_EPI_BIAS_GELU = 1
ENC_EPI_BIAS_RESIDUAL_KEEP = 2
ENC_EPI_BIAS_RESIDUAL_ZERO = 3

# (name, restype, argtypes) for every exported symbol.
_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float
SIGNATURES = (
    ("enc_version", ctypes.c_int, ()),
    ("enc_last_error", ctypes.c_char_p, ()),
    ("enc_linear_order_register", ctypes.c_int, (_I32, _I64, _I64, _I64, _I32, _I32, _I32, _VP)),
    ("enc_linear_order_clear", ctypes.c_int, ()),
    ("enc_debug_gelu_table", ctypes.c_int, (_I32, _I32, _I32, _VP)),
    ("enc_layernorm_bf16", ctypes.c_int, (_VP, _VP, _VP, _VP, _I64, _I64, _F32, _VP, _VP)),
    ("enc_linear_bf16", ctypes.c_int, (_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP, _VP)),
    ("enc_prepack_weight_bf16", ctypes.c_int, (_VP, _VP, _I64, _I64, _VP)),
    (
        "enc_linear_prepacked_bf16",
        ctypes.c_int,
        (_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP, _VP),
    ),
    ("enc_ffn_fused_bf16", ctypes.c_int, (_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP, _VP)),
    ("enc_qkv_proj_bf16", ctypes.c_int, (_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP)),
    (
        "enc_attention_fwd_bf16",
        ctypes.c_int,
        (_VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _F32, _I32, _VP, _VP, _VP),
    ),
    (
        "enc_attention_online_fwd_bf16",
        ctypes.c_int,
        (_VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _F32, _I32, _VP, _VP, _VP),
    ),
    ("enc_selfcheck_expf", ctypes.c_int, (ctypes.c_uint32, ctypes.c_uint32, _VP, _VP)),
    ("enc_mask_lengths", ctypes.c_int, (_VP, _I64, _I64, _VP, _VP)),
    ("enc_encoder_workspace_bytes", ctypes.c_int64, (_I64, _I64, _I64, _I64, _I64)),
    (
        "enc_encoder_forward_bf16",
        ctypes.c_int,
        (_VP, _VP, _VP, _I64, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _VP, _VP, _VP, _I32, _VP),
    ),
    (
        "enc_encoder_forward_bf16_noalloc",
        ctypes.c_int,
        (_VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _I32, _VP, _VP, _VP, _I32, _VP),
    ),
)

# Bytes of the library's static scratch array (ENC_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024


class NativeLibraryError(RuntimeError):
    """libmi355x_encoder.so is missing or failed to load."""


class EncoderKernelError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, name: str, code: int, message: str) -> None:
        super().__init__(f"{name} failed with status {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load and bind the shared library (once per process)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise NativeLibraryError(
                f"{target} not found; build it with "
                "`python -m tiktoktechjam2026track3_amd.build_native`"
            )
        try:
            lib = ctypes.CDLL(str(target))
        except OSError as error:
            raise NativeLibraryError(f"failed to load {target}: {error}") from error
        for name, restype, argtypes in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = list(argtypes)
        if path is None:
            _lib = lib
        return lib


def library_loaded() -> bool:
    return _lib is not None


def _check(name: str, status: int) -> None:
    if status != ENC_OK:
        message = load_library().enc_last_error().decode("utf-8", "replace")
        raise EncoderKernelError(name, status, message)


def _ptr(tensor: Optional[torch.Tensor]) -> Optional[int]:
    return None if tensor is None else tensor.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ensure_order(rows: int, n: int, k: int, device: torch.device) -> None:
    """Make sure the library knows how the reference's nn.Linear reduces this
    shape on this device (measured once per shape, linear_order.py), and
    refuse a shape whose order it cannot reproduce."""
    from . import linear_order

    linear_order.require(linear_order.ensure(rows, n, k, device))


def _require(tensor: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if tensor.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {tensor.dtype}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def layernorm(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float,
    out: Optional[torch.Tensor] = None,
    row_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """bf16 LayerNorm over the last dimension (enc_layernorm_bf16)."""
    for tensor, name in ((x, "x"), (weight, "weight"), (bias, "bias")):
        _require(tensor, name, torch.bfloat16)
    width = x.shape[-1]
    if weight.numel() != width or bias.numel() != width:
        raise ValueError("weight and bias must have x.shape[-1] elements")
    out = torch.empty_like(x) if out is None else out
    mask = None
    if row_mask is not None:
        mask = row_mask.contiguous().view(torch.uint8)
        if mask.numel() != x.numel() // width:
            raise ValueError("row_mask must have one entry per row")
    _check(
        "enc_layernorm_bf16",
        load_library().enc_layernorm_bf16(
            x.data_ptr(), weight.data_ptr(), bias.data_ptr(), out.data_ptr(),
            x.numel() // width, width, float(eps), _ptr(mask), _stream(x.device),
        ),
    )
    return out


def prepack_rows(out_features: int, in_features: int) -> int:
    """Row-group height of the tile-packed weight layout (256 or 128), or 0
    when [out_features, in_features] has no packed form (the C ABI's rule)."""
    if out_features <= 0 or in_features <= 0 or in_features % 32:
        return 0
    return 256 if out_features % 256 == 0 else 128 if out_features % 128 == 0 else 0


def prepack_weight(weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The tile-packed copy of an nn.Linear weight (enc_prepack_weight_bf16),
    as a flat bf16 tensor of weight.numel() elements."""
    _require(weight, "weight", torch.bfloat16)
    n, k = weight.shape
    if prepack_rows(n, k) == 0:
        raise ValueError(f"weight {tuple(weight.shape)} has no packed form (out_features % 128, in_features % 32)")
    out = torch.empty(weight.numel(), device=weight.device, dtype=weight.dtype) if out is None else out
    if out.numel() != weight.numel() or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor of weight.numel() elements")
    _check(
        "enc_prepack_weight_bf16",
        load_library().enc_prepack_weight_bf16(weight.data_ptr(), out.data_ptr(), n, k, _stream(weight.device)),
    )
    return out


def linear(
    a: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    epilogue: int = ENC_EPI_BIAS,
    residual: Optional[torch.Tensor] = None,
    row_mask: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    packed_weight: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """epilogue(a . weight^T + bias) on MFMA (enc_linear_bf16; with
    ``packed_weight``, the prepack_weight copy of weight, through
    enc_linear_prepacked_bf16)."""
    for tensor, name in ((a, "a"), (weight, "weight"), (bias, "bias")):
        _require(tensor, name, torch.bfloat16)
    n, k = weight.shape
    if a.shape[-1] != k or bias.numel() != n:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, weight {tuple(weight.shape)}")
    rows = a.numel() // k
    _ensure_order(rows, n, k, a.device)
    out = torch.empty((*a.shape[:-1], n), device=a.device, dtype=a.dtype) if out is None else out
    if residual is not None:
        _require(residual, "residual", torch.bfloat16)
        if residual.shape != out.shape:
            raise ValueError("residual must have the output shape")
    mask = None if row_mask is None else row_mask.contiguous().view(torch.uint8)
    if packed_weight is not None:
        _require(packed_weight, "packed_weight", torch.bfloat16)
        if packed_weight.numel() != weight.numel():
            raise ValueError("packed_weight must hold weight.numel() elements")
        _check(
            "enc_linear_prepacked_bf16",
            load_library().enc_linear_prepacked_bf16(
                a.data_ptr(), weight.data_ptr(), packed_weight.data_ptr(), bias.data_ptr(), _ptr(residual),
                out.data_ptr(), rows, n, k, int(epilogue), _ptr(mask), _stream(a.device),
            ),
        )
        return out
    _check(
        "enc_linear_bf16",
        load_library().enc_linear_bf16(
            a.data_ptr(), weight.data_ptr(), bias.data_ptr(), _ptr(residual), out.data_ptr(),
            rows, n, k, int(epilogue), _ptr(mask), _stream(a.device),
        ),
    )
    return out


def ffn(
    h: torch.Tensor,
    w_in: torch.Tensor,
    b_in: torch.Tensor,
    w_out: torch.Tensor,
    b_out: torch.Tensor,
    residual: torch.Tensor,
    row_mask: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    hidden: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """residual + ffn_out(gelu(ffn_in(h))), masked rows zeroed
    (enc_ffn_fused_bf16); ``hidden`` is the [rows, ffn_dim] workspace."""
    for tensor, name in ((h, "h"), (w_in, "w_in"), (b_in, "b_in"), (w_out, "w_out"), (b_out, "b_out"),
                         (residual, "residual")):
        _require(tensor, name, torch.bfloat16)
    f, d = w_in.shape
    if h.shape[-1] != d or tuple(w_out.shape) != (d, f) or b_in.numel() != f or b_out.numel() != d:
        raise ValueError(f"shape mismatch: h {tuple(h.shape)}, w_in {tuple(w_in.shape)}, w_out {tuple(w_out.shape)}")
    if residual.shape != h.shape:
        raise ValueError("residual must have h's shape")
    rows = h.numel() // d
    _ensure_order(rows, f, d, h.device)
    _ensure_order(rows, d, f, h.device)
    out = torch.empty_like(h) if out is None else out
    hidden = torch.empty((rows, f), device=h.device, dtype=h.dtype) if hidden is None else hidden
    if hidden.numel() < rows * f or not hidden.is_contiguous():
        raise ValueError("hidden must be a contiguous workspace of rows * ffn_dim elements")
    mask = None if row_mask is None else row_mask.contiguous().view(torch.uint8)
    _check(
        "enc_ffn_fused_bf16",
        load_library().enc_ffn_fused_bf16(
            h.data_ptr(), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(), b_out.data_ptr(),
            residual.data_ptr(), out.data_ptr(), hidden.data_ptr(), rows, d, f, _ptr(mask), _stream(h.device),
        ),
    )
    return out


def debug_gelu_table(device: torch.device, ready: int = -1, entry: int = -1, value: int = -1) -> None:
    """Test hook (enc_debug_gelu_table): set the GELU table's ready flag and/or
    overwrite (value >= 0) or restore (value -1) one table entry."""
    _check("enc_debug_gelu_table", load_library().enc_debug_gelu_table(ready, entry, value, _stream(device)))


def vt_stride(seq_len: int) -> int:
    """Row stride of the transposed-V buffer: seq_len rounded up to 8."""
    return (seq_len + 7) // 8 * 8


def qkv_proj(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, num_heads: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed QKV projection; returns q, k [B,H,S,hd] and v_t [B,H,hd,ld_vt]."""
    for tensor, name in ((x, "x"), (weight, "weight"), (bias, "bias")):
        _require(tensor, name, torch.bfloat16)
    batch, seq_len, d_model = x.shape
    if tuple(weight.shape) != (3 * d_model, d_model) or bias.numel() != 3 * d_model:
        raise ValueError("qkv weight must be [3*d_model, d_model] with a [3*d_model] bias")
    _ensure_order(batch * seq_len, d_model, d_model, x.device)
    hd = d_model // num_heads
    q = torch.empty((batch, num_heads, seq_len, hd), device=x.device, dtype=x.dtype)
    k = torch.empty_like(q)
    v_t = torch.empty((batch, num_heads, hd, vt_stride(seq_len)), device=x.device, dtype=x.dtype)
    _check(
        "enc_qkv_proj_bf16",
        load_library().enc_qkv_proj_bf16(
            x.data_ptr(), weight.data_ptr(), bias.data_ptr(), q.data_ptr(), k.data_ptr(),
            v_t.data_ptr(), batch, seq_len, d_model, num_heads, _stream(x.device),
        ),
    )
    return q, k, v_t


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v_t: torch.Tensor,
    scale: float,
    causal: bool,
    kv_len: Optional[torch.Tensor] = None,
    key_mask: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    online: bool = False,
) -> torch.Tensor:
    """Streaming attention; returns context [B, S, H*hd].

    By default the three-sweep kernel that forms the reference's bf16
    probabilities bit for bit (enc_attention_fwd_bf16); ``online=True`` runs
    the one-pass online-softmax kernel (enc_attention_online_fwd_bf16).
    """
    for tensor, name in ((q, "q"), (k, "k"), (v_t, "v_t")):
        _require(tensor, name, torch.bfloat16)
    batch, heads, seq_len, hd = q.shape
    if tuple(k.shape) != tuple(q.shape):
        raise ValueError("q and k must have the same shape")
    if tuple(v_t.shape) != (batch, heads, hd, vt_stride(seq_len)):
        raise ValueError("v_t must be [B, H, hd, round_up(S, 8)]")
    out = (
        torch.empty((batch, seq_len, heads * hd), device=q.device, dtype=q.dtype)
        if out is None
        else out
    )
    if kv_len is not None:
        _require(kv_len, "kv_len", torch.int32)
    mask = None if key_mask is None else key_mask.contiguous().view(torch.uint8)
    name = "enc_attention_online_fwd_bf16" if online else "enc_attention_fwd_bf16"
    _check(
        name,
        getattr(load_library(), name)(
            q.data_ptr(), k.data_ptr(), v_t.data_ptr(), out.data_ptr(), batch, heads, seq_len, hd,
            float(scale), int(bool(causal)), _ptr(kv_len), _ptr(mask), _stream(q.device),
        ),
    )
    return out


def selfcheck_expf(lo_bits: int, hi_bits: int, device: torch.device) -> int:
    """Number of float bit patterns in [lo_bits, hi_bits] where the exact
    attention's inlined exponential differs from the device library's expf."""
    counter = torch.zeros(1, dtype=torch.int32, device=device)
    _check(
        "enc_selfcheck_expf",
        load_library().enc_selfcheck_expf(lo_bits, hi_bits, counter.data_ptr(), _stream(device)),
    )
    return int(counter.item())


def mask_lengths(mask: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-row count of valid tokens of a [B, S] bool mask, as int32 on device."""
    if mask.device.type != "cuda" or mask.dtype != torch.bool or mask.dim() != 2:
        raise ValueError("mask must be a [B, S] bool CUDA tensor")
    mask = mask.contiguous()
    batch, seq_len = mask.shape
    out = torch.empty((batch,), device=mask.device, dtype=torch.int32) if out is None else out
    _check(
        "enc_mask_lengths",
        load_library().enc_mask_lengths(
            mask.view(torch.uint8).data_ptr(), batch, seq_len, out.data_ptr(), _stream(mask.device)
        ),
    )
    return out


def encoder_workspace_bytes(batch: int, seq_len: int, d_model: int, num_heads: int, ffn_dim: int) -> int:
    size = load_library().enc_encoder_workspace_bytes(batch, seq_len, d_model, num_heads, ffn_dim)
    if size < 0:
        raise ValueError("invalid encoder shape")
    return int(size)


def _forward_flags(online_attention: bool, final_norm: bool, packed_weights: bool, weight_table: torch.Tensor,
                   num_layers: int) -> int:
    expected = 12 * num_layers + 2 + (4 * num_layers if packed_weights else 0)
    if weight_table.numel() != expected or weight_table.dtype != torch.int64 or weight_table.device.type != "cpu":
        raise ValueError(f"weight_table must be a CPU int64 tensor of {expected} device pointers")
    return ((ENC_FWD_ONLINE_ATTENTION if online_attention else 0) | (0 if final_norm else ENC_FWD_SKIP_FINAL_NORM)
            | (ENC_FWD_PACKED_WEIGHTS if packed_weights else 0))


def encoder_forward(
    x: torch.Tensor,
    out: torch.Tensor,
    workspace: torch.Tensor,
    weight_table: torch.Tensor,
    num_heads: int,
    ffn_dim: int,
    num_layers: int,
    eps: float,
    causal: bool,
    kv_len: Optional[torch.Tensor],
    key_mask: Optional[torch.Tensor],
    row_mask: Optional[torch.Tensor],
    online_attention: bool = False,
    final_norm: bool = True,
    packed_weights: bool = False,
) -> None:
    """Run the whole encoder through enc_encoder_forward_bf16.

    ``weight_table`` is a CPU int64 tensor of device pointers in the order the
    C ABI documents (with ``packed_weights``, followed by the packed copies of
    each layer's four projection weights, ENC_FWD_PACKED_WEIGHTS);
    ``key_mask``/``row_mask`` are uint8 [B, S] tensors.  With
    ``final_norm=False`` ``out`` receives the last block's output and the
    caller applies final_norm (ENC_FWD_SKIP_FINAL_NORM).
    """
    flags = _forward_flags(online_attention, final_norm, packed_weights, weight_table, num_layers)
    batch, seq_len, d_model = x.shape
    from . import linear_order

    for order in linear_order.ensure_encoder(batch * seq_len, d_model, ffn_dim, x.device):
        linear_order.require(order)
    table = ctypes.cast(weight_table.data_ptr(), ctypes.c_void_p)
    _check(
        "enc_encoder_forward_bf16",
        load_library().enc_encoder_forward_bf16(
            x.data_ptr(), out.data_ptr(), workspace.data_ptr(), workspace.numel(), table.value,
            batch, seq_len, d_model, num_heads, ffn_dim, num_layers, float(eps), int(bool(causal)),
            _ptr(kv_len), _ptr(key_mask), _ptr(row_mask),
            flags, _stream(x.device),
        ),
    )


def encoder_forward_noalloc(
    x: torch.Tensor,
    out: torch.Tensor,
    weight_table: torch.Tensor,
    num_heads: int,
    ffn_dim: int,
    num_layers: int,
    eps: float,
    causal: bool,
    kv_len: Optional[torch.Tensor],
    key_mask: Optional[torch.Tensor],
    row_mask: Optional[torch.Tensor],
    online_attention: bool = False,
    final_norm: bool = True,
    packed_weights: bool = False,
) -> None:
    """enc_encoder_forward_bf16_noalloc: the encoder forward over the library's
    own static scratch array (no workspace argument, no device allocation).
    Calls that overlap on one GPU share that array and must not run
    concurrently.  The reduction orders of the three product shapes must be
    known already (linear_order.ensure_encoder, or an earlier workspace
    forward at the same shape): measuring them allocates."""
    flags = _forward_flags(online_attention, final_norm, packed_weights, weight_table, num_layers)
    batch, seq_len, d_model = x.shape
    from . import linear_order

    for order in linear_order.known_encoder_orders(batch * seq_len, d_model, ffn_dim, x.device):
        linear_order.require(order)
    table = ctypes.cast(weight_table.data_ptr(), ctypes.c_void_p)
    _check(
        "enc_encoder_forward_bf16_noalloc",
        load_library().enc_encoder_forward_bf16_noalloc(
            x.data_ptr(), out.data_ptr(), table.value,
            batch, seq_len, d_model, num_heads, ffn_dim, num_layers, float(eps), int(bool(causal)),
            _ptr(kv_len), _ptr(key_mask), _ptr(row_mask),
            flags, _stream(x.device),
        ),
    )
