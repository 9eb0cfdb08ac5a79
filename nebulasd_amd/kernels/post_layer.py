"""Post-layer: last-token gather, final RMSNorm, lm_head and argmax --
drop-in for swiftLLM's ``LlamaPostLayer.forward``.

Reference: swiftLLM/swiftllm/worker/layers/post_layer.py:49-79.  The
reference gathers each request's last token (prompt ends, then every decode
row, :53-60), normalises it (:63-67), computes the [rows, vocab] fp16 logits
with ``F.linear`` (:68) and takes ``torch.argmax`` (:69).  Here the lm_head
GEMV and the argmax are one gfx950 pass over the lm_head weight
(``nsd_lm_head_argmax``): the logits are never written.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import require, require_cuda, stream_of
from .rmsnorm import rmsnorm_inplace

_KEYS: dict = {}


def _keys(device: torch.device, stream: int, rows: int) -> torch.Tensor:
    """Zeroed 64-bit argmax keys, one buffer per (device, stream); every call
    leaves its keys zero, so calls in one stream reuse it in order."""
    k = (device, stream)
    buf = _KEYS.get(k)
    if buf is None or buf.numel() < rows:
        if buf is None and len(_KEYS) >= 16:
            _KEYS.clear()  # each dropped buffer is freed in its own stream's order
        buf = torch.zeros(max(rows, 256), dtype=torch.int64, device=device)
        _KEYS[k] = buf
    return buf


def lm_head_argmax(x: torch.Tensor, lm_head: torch.Tensor) -> torch.Tensor:
    """``torch.argmax(F.linear(x, lm_head), dim=1)`` for fp16 x [rows, hidden]
    and lm_head [vocab, hidden]: int64 [rows], in passes of 128 rows that
    each stream the weight once (faster than the library GEMM plus the
    argmax at every row count measured, 1-128, for the Qwen3-8B lm_head)."""
    require_cuda(x, lm_head)
    require(x, torch.float16, "x")
    require(lm_head, torch.float16, "lm_head")
    if x.dim() != 2 or lm_head.dim() != 2 or lm_head.shape[1] != x.shape[1]:
        raise ValueError("x must be [rows, hidden] and lm_head [vocab, hidden]")
    tokens = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    s = stream_of(x)
    keys = _keys(x.device, s, x.shape[0])
    _lib.call("nsd_lm_head_argmax", x.data_ptr(), lm_head.data_ptr(), x.shape[0], x.shape[1], lm_head.shape[0],
              keys.data_ptr(), tokens.data_ptr(), s)
    return tokens


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """``torch.argmax(logits, dim=1)`` for fp16 logits [rows, vocab]."""
    require_cuda(logits)
    require(logits, torch.float16, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be [rows, vocab]")
    tokens = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    _lib.call("nsd_argmax_rows", logits.data_ptr(), logits.shape[0], logits.shape[1], tokens.data_ptr(),
              stream_of(logits))
    return tokens


def last_token_indices(infer_state) -> torch.Tensor:
    """post_layer.py:53-59: the last token of every prompt, then every decode row."""
    dev = infer_state.prefill_seq_start_locs.device
    return torch.cat((infer_state.prefill_seq_start_locs + infer_state.prefill_seq_lens - 1,
                      torch.arange(infer_state.num_prefill_tokens, infer_state.num_tokens, device=dev,
                                   dtype=torch.int32)), dim=0)


def post_layer_forward(input_embds: torch.Tensor, infer_state, final_norm: torch.Tensor, lm_head: torch.Tensor,
                       eps: float) -> torch.Tensor:
    """post_layer.py:49-79: greedy next token of every request, int64 [batch_size]."""
    last_input = input_embds.index_select(0, last_token_indices(infer_state))
    rmsnorm_inplace(last_input, final_norm, eps)
    return lm_head_argmax(last_input, lm_head)
