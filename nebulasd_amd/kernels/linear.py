"""Split-k projection GEMMs of decode/verify batches and their consumers.

The reference's layer projections are ``F.linear`` calls
(swiftLLM/swiftllm/worker/kernels/linear.py:3-12; transformer_layer.py:107-109
q/k/v, :187 O, :201 down).  At decode/verify batch sizes (<= 128 rows)
``linear_partials`` streams the weight once with k split into ranges and
returns fp32 partial sums [splits, rows, n]; the projection is their sum in
split order rounded once to fp16 (``sum_partials``), which the next kernel of
the layer can take directly (``fused_add_rmsnorm_partials``, and
``qk_norm_rope_store_partials`` in ``prologue``) instead of a separate pass.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._util import require, require_cuda, stream_of

MAX_ROWS = 128  # rows one call serves


def linear_splits(rows: int, n_out: int, n_in: int) -> int:
    """Split count the current device uses for an n_out x n_in projection of
    ``rows`` rows (sizes the partials)."""
    s = ctypes.c_int()
    _lib.call("nsd_linear_splits", rows, n_out, n_in, ctypes.byref(s))
    return s.value


def linear_partials(x: torch.Tensor, w: torch.Tensor, partials: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 partial sums [splits, rows, n_out] of x [rows, n_in] . w[n_out, n_in]^T
    (fp16, rows <= 128, n_out a multiple of 16, n_in of 128)."""
    require_cuda(x, w, partials)
    require(x, torch.float16, "x")
    require(w, torch.float16, "w")
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
        raise ValueError("x must be [rows, n_in] and w [n_out, n_in]")
    rows, n_out, n_in = x.shape[0], w.shape[0], x.shape[1]
    splits = linear_splits(rows, n_out, n_in)
    if partials is None:
        partials = torch.empty((splits, rows, n_out), dtype=torch.float32, device=x.device)
    else:
        require(partials, torch.float32, "partials")
        if tuple(partials.shape) != (splits, rows, n_out):
            raise ValueError(f"partials must be [{splits}, {rows}, {n_out}]")
    _lib.call("nsd_linear_partials", x.data_ptr(), w.data_ptr(), partials.data_ptr(), rows, n_out, n_in,
              stream_of(x))
    return partials


def sum_partials(partials: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 [rows, n] = the sum of the splits of ``partials`` in split order."""
    require_cuda(partials, out)
    require(partials, torch.float32, "partials")
    if partials.dim() != 3:
        raise ValueError("partials must be [splits, rows, n]")
    splits, rows, n = partials.shape
    if out is None:
        out = torch.empty((rows, n), dtype=torch.float16, device=partials.device)
    elif out.dtype != torch.float16 or tuple(out.shape) != (rows, n) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp16 [{rows}, {n}]")
    _lib.call("nsd_sum_partials", partials.data_ptr(), splits, out.data_ptr(), rows, n, stream_of(partials))
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, w)`` for decode/verify batches (fp16 out, fp32 sums)."""
    return sum_partials(linear_partials(x, w))


def fused_add_rmsnorm_partials(partials: torch.Tensor, out: torch.Tensor, residual: torch.Tensor,
                               weight: torch.Tensor, eps: float) -> None:
    """``fused_add_rmsnorm_inplace`` (kernels/rmsnorm.py:74-89) whose input is
    the projection held in ``partials``: residual += fp16(sum of splits); out
    = the normalised residual (fp16 [rows, hidden])."""
    require_cuda(partials, out, residual, weight)
    require(partials, torch.float32, "partials")
    for t, n in ((out, "out"), (residual, "residual"), (weight, "weight")):
        require(t, torch.float16, n)
    splits, rows, hidden = partials.shape
    if tuple(out.shape) != (rows, hidden) or residual.shape != out.shape or tuple(weight.shape) != (hidden,):
        raise ValueError(f"out/residual must be [{rows}, {hidden}] and weight [{hidden}]")
    _lib.call("nsd_fused_add_rmsnorm_partials", partials.data_ptr(), splits, out.data_ptr(), residual.data_ptr(),
              weight.data_ptr(), rows, hidden, float(eps), stream_of(out))
