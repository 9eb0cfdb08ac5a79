"""RMSNorm -- drop-ins for swiftLLM's ``rmsnorm_inplace`` (per head as
QK-norm, per row as the final norm) and ``fused_add_rmsnorm_inplace`` (the
two residual adds + norms of every layer).

Reference: swiftLLM/swiftllm/worker/kernels/rmsnorm.py:26-37 (wrapper),
:5-24 (kernel): ``x = fp16(x * 1/sqrt(mean(x^2) + eps) * w)`` in fp32;
:74-89 (wrapper), :39-72 (kernel): ``r = x + r`` (fp16), then the norm of r
into x.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import require, require_cuda, stream_of


def rmsnorm_inplace(input_and_output: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    x = input_and_output
    require_cuda(x, weight)
    require(x, torch.float16, "input_and_output")
    require(weight, torch.float16, "weight")
    if x.dim() != 2 or weight.shape != (x.shape[1],):
        raise ValueError("input_and_output must be [rows, hidden] and weight [hidden]")
    _lib.call("nsd_rmsnorm_inplace", x.data_ptr(), weight.data_ptr(), x.shape[0], x.shape[1],
              float(eps), stream_of(x))


def fused_add_rmsnorm_inplace(input_and_output: torch.Tensor, residual_io: torch.Tensor, weight: torch.Tensor,
                              eps: float) -> None:
    """rmsnorm.py:74-89: ``residual_io = input_and_output + residual_io`` and
    ``input_and_output = rms_norm(residual_io) * weight``, in place."""
    x, r = input_and_output, residual_io
    require_cuda(x, r, weight)
    for t, n in ((x, "input_and_output"), (r, "residual_io"), (weight, "weight")):
        require(t, torch.float16, n)
    if x.dim() != 2 or r.shape != x.shape or weight.shape != (x.shape[1],):
        raise ValueError("input_and_output and residual_io must be [rows, hidden], weight [hidden]")
    _lib.call("nsd_fused_add_rmsnorm_inplace", x.data_ptr(), r.data_ptr(), weight.data_ptr(), x.shape[0],
              x.shape[1], float(eps), stream_of(x))
