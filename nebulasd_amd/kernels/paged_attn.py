"""Paged verify/decode attention -- drop-in for swiftLLM's ``paged_attention``.

Reference: swiftLLM/swiftllm/worker/kernels/paged_attn.py:152-222 (wrapper),
:9-149 (Triton phases).  Same signature, argument meaning and in-place write
of ``o``; the extra keyword ``lse`` receives ln(sum exp(score)) per (row, q-head).
"""

from __future__ import annotations

import torch

from .. import _lib
from ..plan import plan_for
from ._util import StatusWord, cache_dims, check_block_table, ptr, require, require_cuda, stream_of


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table: torch.Tensor, model_config, engine_config, infer_state,
                    cur_layer: int, o: torch.Tensor, lse: torch.Tensor | None = None,
                    validate: bool = False) -> None:
    """Attention of the decode/verify rows of ``infer_state`` at layer ``cur_layer``.

    ``q``: [num_decoding_seqs, Hq, d] fp16 (the reference passes
    ``q[num_prefill_tokens:]``); ``o``: same number of elements, written in place.
    Rows are the reference's decode rows: row r reads ``block_table[seq_ids[r]]``
    for its first ``decoding_seq_lens[r]`` tokens (paged_attn.py:36-75).
    """
    require_cuda(q, k_cache, v_cache, block_table, o, lse)
    require(q, torch.float16, "q")
    require(k_cache, torch.float16, "k_cache")
    require(v_cache, torch.float16, "v_cache")
    check_block_table(block_table, engine_config)
    require(o, torch.float16, "o")
    if engine_config.block_size != k_cache.shape[3]:
        raise ValueError("engine_config.block_size does not match the cache layout")
    n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    rows = infer_state.num_decoding_seqs
    hq = model_config.num_q_heads
    if q.shape != (rows, hq, d) or o.numel() != rows * hq * d:
        raise ValueError(f"q must be [{rows}, {hq}, {d}] and o hold as many elements")
    if lse is not None:
        require(lse, torch.float32, "lse")
        if lse.numel() != rows * hq:
            raise ValueError("lse must hold num_decoding_seqs * num_q_heads floats")
    if rows == 0:
        return
    plan = plan_for(infer_state, model_config, engine_config, block_table)
    if plan.n_rows != rows:
        raise ValueError(f"the forward's attention plan covers {plan.n_rows} rows, q has {rows}")
    status = StatusWord(q.device) if validate else None
    _lib.call("nsd_paged_attention",
              q.data_ptr(), o.data_ptr(), ptr(lse), k_cache.data_ptr(), v_cache.data_ptr(),
              n_blocks, n_layers, int(cur_layer), hq, hkv, d, bs, block_table.data_ptr(),
              block_table.shape[0], block_table.shape[1], plan.host_ptr(), plan.dev.data_ptr(),
              plan.workspace.data_ptr(), plan.workspace.numel(),
              float(infer_state.softmax_scale), ptr(status.t) if status else None,
              stream_of(q))
    if status is not None:
        status.check("paged_attention")
