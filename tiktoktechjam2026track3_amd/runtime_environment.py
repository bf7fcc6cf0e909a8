"""Process environment that has to be in place before PyTorch is imported.

Counterpart of transformer_benchmark/runtime_environment.py:8-13 of the
reference, which switches torch's CUDA caching allocator to expandable
segments.  PyTorch-ROCm does not implement expandable segments (it warns
"expandable_segments not supported on this platform" and ignores the option),
so nothing is set for the allocator here; large configurations instead
allocate their activations and workspace once and reuse them across calls.
Callers keep calling this hook first so an environment setting can be added in
one place.
"""

from __future__ import annotations

# Variables the reference sets that the ROCm build deliberately leaves alone.
IGNORED_ON_ROCM = ("PYTORCH_CUDA_ALLOC_CONF",)


def configure_pre_torch_environment() -> None:
    """Environment for a PyTorch-ROCm process running the gfx950 kernels:
    currently nothing needs setting (see the module docstring)."""
    return None
