"""Forward-phase ranges for profilers, under the reference's names and switch.

swiftLLM marks the phases of each layer (``layer_<i>_qkv``,
``layer_<i>_store_kvcache``, ``layer_<i>_paged_attention``,
``layer_<i>_o_proj``, ``layer_<i>_ffn``) and the post-layer's
``post_lm_head`` with NVTX ranges when ``STARSD_ENABLE_FORWARD_PHASE_NVTX``
is 1/true/yes/on (swiftLLM/swiftllm/worker/layers/transformer_layer.py:46-65,
post_layer.py:22-40).  On ROCm torch's ``torch.cuda.nvtx`` calls emit roctx
ranges, which ``rocprofv3 --marker-trace`` records.  As in the reference, a
failing push or pop never stops the forward.
"""

from __future__ import annotations

import os
from contextlib import contextmanager

import torch

ENABLED = os.environ.get("STARSD_ENABLE_FORWARD_PHASE_NVTX", "0").lower() in {"1", "true", "yes", "on"}


@contextmanager
def forward_phase_range(name: str):
    """A named range around the enclosed work when ENABLED, else nothing."""
    if not ENABLED:
        yield
        return
    try:
        torch.cuda.nvtx.range_push(name)
    except Exception:
        yield
        return
    try:
        yield
    finally:
        try:
            torch.cuda.nvtx.range_pop()
        except Exception:
            pass
