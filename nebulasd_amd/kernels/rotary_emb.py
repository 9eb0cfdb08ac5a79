"""RoPE -- drop-in for swiftLLM's ``rotary_embedding_inplace``.

Reference: swiftLLM/swiftllm/worker/kernels/rotary_emb.py:44-58 (wrapper),
:7-42 (kernel).  Rotate-half on halves [0, d/2) and [d/2, d) from the
per-token tables ``infer_state.position_cos/sin`` [num_tokens, d/2] fp16.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import require, require_cuda, stream_of


def rotary_embedding_inplace(q: torch.Tensor, k: torch.Tensor, infer_state) -> None:
    require_cuda(q, k, infer_state.position_cos, infer_state.position_sin)
    require(q, torch.float16, "q")
    require(k, torch.float16, "k")
    cos, sin = infer_state.position_cos, infer_state.position_sin
    require(cos, torch.float16, "position_cos")
    require(sin, torch.float16, "position_sin")
    n, hq, d = q.shape
    if k.shape[0] != n or k.shape[2] != d or cos.shape != (n, d // 2) or sin.shape != cos.shape:
        raise ValueError("q [T, Hq, d], k [T, Hkv, d] and cos/sin [T, d/2] disagree")
    _lib.call("nsd_rotary_embedding_inplace", q.data_ptr(), k.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), n, hq, k.shape[1], d, stream_of(q))
