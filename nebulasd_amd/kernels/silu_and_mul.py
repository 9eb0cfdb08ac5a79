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


# Rows up to which one pass of the fused kernel (the weight streamed once)
# beats the library GEMM plus the separate SiLU-and-mul; above it a pass per
# 128 rows re-reads the weight.
FUSED_UP_GATE_MAX_ROWS = 128


def up_gate_silu_and_mul(x: torch.Tensor, up_gate: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The FFN's up/gate projection and SiLU-and-mul in one pass over the
    weight (transformer_layer.py:199-200: ``linear(o, up_gate_proj)`` then
    ``silu_and_mul_inplace``): returns [rows, I] with the values the
    reference leaves in ``up_gate_proj[:, :I]`` (fp16 GEMM outputs, then
    fp16(up * fp16(silu(gate)))).  x [rows, hidden], up_gate [2 * I, hidden]
    (up rows first), fp16.  Rows are processed in passes of 128, each reading
    the weight once."""
    require_cuda(x, up_gate)
    require(x, torch.float16, "x")
    require(up_gate, torch.float16, "up_gate")
    if x.dim() != 2 or up_gate.dim() != 2 or up_gate.shape[1] != x.shape[1] or up_gate.shape[0] % 2:
        raise ValueError("x must be [rows, hidden] and up_gate [2 * ffn_inter_dim, hidden]")
    inter = up_gate.shape[0] // 2
    if out is None:
        out = torch.empty((x.shape[0], inter), dtype=torch.float16, device=x.device)
    else:
        require_cuda(out)
        require(out, torch.float16, "out")
        if tuple(out.shape) != (x.shape[0], inter):
            raise ValueError("out must be [rows, ffn_inter_dim]")
    _lib.call("nsd_up_gate_silu_and_mul", x.data_ptr(), up_gate.data_ptr(), out.data_ptr(), x.shape[0], x.shape[1],
              inter, stream_of(x))
    return out
