"""SiLU-and-multiply -- drop-in for swiftLLM's ``silu_and_mul_inplace``.

Reference: swiftLLM/swiftllm/worker/kernels/silu_and_mul.py:25-34 (wrapper),
:5-23 (kernel): for x [tokens, 2*I] (the output of the stacked
``up_gate_proj``, up first, gate second, weight.py:151),
``x[:, :I] = x[:, :I] * fp16(silu(fp32(x[:, I:])))`` in place.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import require, require_cuda, stream_of


def silu_and_mul_inplace(x: torch.Tensor) -> None:
    require_cuda(x)
    require(x, torch.float16, "x")
    if x.dim() != 2 or x.shape[1] % 2:
        raise ValueError("x must be [tokens, 2 * ffn_inter_dim]")
    _lib.call("nsd_silu_and_mul_inplace", x.data_ptr(), x.shape[0], x.shape[1] // 2, stream_of(x))
