"""Process environment that has to be in place before PyTorch is imported.

Mirrors transformer_benchmark/runtime_environment.py:8-13 of the reference: the
caching allocator is switched to expandable segments (PyTorch-ROCm reads the same
``PYTORCH_CUDA_ALLOC_CONF`` variable) unless the caller already chose a setting.
Expandable segments matter here because the S=100000 configuration allocates
tens of GB of activations and workspace in a few large blocks.
"""

from __future__ import annotations

import os

PYTORCH_CUDA_ALLOC_CONF = "expandable_segments:True"


def configure_pre_torch_environment() -> None:
    """Select the fragmentation-resistant allocator unless explicitly configured."""
    if "PYTORCH_CUDA_ALLOC_CONF" not in os.environ:
        os.environ["PYTORCH_CUDA_ALLOC_CONF"] = PYTORCH_CUDA_ALLOC_CONF
