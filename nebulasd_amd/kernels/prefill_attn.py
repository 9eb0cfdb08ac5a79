"""Prefill (prompt) attention -- drop-in for swiftLLM's prefill attention entry points.

Reference: ``flash_attn_varlen_func`` in
swiftLLM/swiftllm/worker/layers/transformer_layer.py:7-32 (the function the
layer calls at :151-164, one ``scaled_dot_product_attention`` per prompt
after a host copy of ``cu_seqlens``) and the Triton ``prefill_attention``
(swiftLLM/swiftllm/worker/kernels/prefill_attn.py:102-140).  Both compute
causal attention within each prompt of a packed batch; here one gfx950 launch
covers every prompt, with no host synchronisation.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import StatusWord, ptr, require, require_cuda, stream_of


def _longest_first(cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Prompt indices, longest first (device int32, computed on the device with
    no host synchronisation).  Kept on the ``cu_seqlens`` tensor object itself
    together with its version counter, so the layers of one forward share it
    and a new or modified tensor gets its own."""
    cached = getattr(cu_seqlens, "_nsd_longest_first", None)
    if cached is not None and cached[0] == cu_seqlens._version:
        return cached[1]
    lens = cu_seqlens[1:] - cu_seqlens[:-1]
    order = torch.argsort(lens, descending=True, stable=True).to(torch.int32)
    cu_seqlens._nsd_longest_first = (cu_seqlens._version, order)
    return order


def _launch(q, k, v, o, cu_seqlens, max_seqlen: int, softmax_scale: float,
            lse: torch.Tensor | None, validate: bool) -> None:
    require_cuda(q, k, v, o, cu_seqlens, lse)
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (o, "o")):
        require(t, torch.float16, n)
    require(cu_seqlens, torch.int32, "cu_seqlens")
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError("q must be [tokens, Hq, d]; k and v [tokens, Hkv, d]")
    tokens, hq, d = q.shape
    hkv = k.shape[1]
    if k.shape[0] < tokens or k.shape[2] != d:
        raise ValueError(f"k/v must hold at least the {tokens} tokens of q with head_dim {d}")
    if o.numel() != q.numel():
        raise ValueError("o must have as many elements as q")
    if lse is not None:
        require(lse, torch.float32, "lse")
        if lse.numel() != tokens * hq:
            raise ValueError("lse must be [tokens, Hq]")
    status = StatusWord(q.device) if validate else None
    order = _longest_first(cu_seqlens)
    _lib.call("nsd_prefill_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              ptr(lse), cu_seqlens.data_ptr(), order.data_ptr(), cu_seqlens.numel() - 1,
              int(max_seqlen), tokens,
              hq, hkv, d, float(softmax_scale), ptr(status.t) if status else None, stream_of(q))
    if status is not None:
        status.check("prefill_attention")


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                           max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float | None = None,
                           causal: bool = True, lse: torch.Tensor | None = None,
                           validate: bool = False) -> torch.Tensor:
    """Causal varlen attention, same signature and result as the reference's
    (transformer_layer.py:7-32): returns ``o`` [tokens, Hq, d] fp16.

    The reference is only ever called with ``cu_seqlens_q`` equal to
    ``cu_seqlens_k`` and ``causal=True`` (:154-163); other uses raise.
    ``lse`` (optional, fp32 [tokens, Hq]) receives ln(sum exp(score)).
    """
    if not causal:
        raise NotImplementedError("flash_attn_varlen_func: only causal prefill attention is supported")
    if cu_seqlens_k is not cu_seqlens_q and not torch.equal(cu_seqlens_k, cu_seqlens_q):
        raise NotImplementedError("flash_attn_varlen_func: cu_seqlens_k must equal cu_seqlens_q")
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    o = torch.empty_like(q)
    _launch(q, k, v, o, cu_seqlens_q, max(int(max_seqlen_q), int(max_seqlen_k)), scale, lse, validate)
    return o


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                      model_config, engine_config, infer_state, lse: torch.Tensor | None = None,
                      validate: bool = False) -> None:
    """Prefill attention of ``infer_state``'s prompts, written into ``o``.

    Same arguments as the reference's Triton prefill_attention
    (prefill_attn.py:102-140): q/k/v hold the forward's tokens (prompt tokens
    first), ``o`` [num_prefill_tokens, Hq, d] (or a view with as many
    elements) receives the prompts' rows.
    """
    npt = infer_state.num_prefill_tokens
    if infer_state.num_prefill_seqs == 0 or npt == 0:
        return
    hq, hkv, d = model_config.num_q_heads, model_config.num_kv_heads, model_config.head_dim
    if q.shape[1:] != (hq, d) or k.shape[1:] != (hkv, d):
        raise ValueError("q/k shapes do not match model_config")
    _launch(q[:npt], k[:npt], v[:npt], o[:npt], infer_state.prefill_seq_start_locs_with_end,
            infer_state.max_prefill_len, infer_state.softmax_scale, lse, validate)
