"""RMSNorm -- drop-in for swiftLLM's ``rmsnorm_inplace`` (used per head as QK-norm).

Reference: swiftLLM/swiftllm/worker/kernels/rmsnorm.py:26-37 (wrapper),
:5-24 (kernel): ``x = fp16(x * 1/sqrt(mean(x^2) + eps) * w)`` in fp32.
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
