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


def paged_attention_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                          v_cache: torch.Tensor, block_table: torch.Tensor, q_norm: torch.Tensor | None,
                          k_norm: torch.Tensor | None, model_config, engine_config, infer_state,
                          cur_layer: int, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                          o: torch.Tensor, lse: torch.Tensor | None = None,
                          validate: bool = False) -> None:
    """The decode/verify rows' prologue and attention in one launch.

    Same results as ``qk_norm_rope_store(q, k, v, ...)`` then
    ``paged_attention(q, ...)`` (transformer_layer.py:114-145, :169-180):
    ``o`` (and ``lse``) and the K/V rows written into the cache are bit for
    bit those of the two calls; ``q`` is not written back.  q [rows, Hq, d],
    k/v [rows, Hkv, d] fp16 may be row-strided slices of one fused q/k/v
    projection.  Raises ``NativeLibraryError`` with NSD_ERR_UNSUPPORTED when
    the forward's plan splits a sequence's rows over several verify groups
    (then run the two calls).
    """
    require_cuda(q, k, v, k_cache, v_cache, block_table, cos_cache, sin_cache, q_norm, k_norm, o, lse)
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache"), (cos_cache, "cos_cache"),
                 (sin_cache, "sin_cache"), (o, "o")):
        require(t, torch.float16, n)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t.dtype != torch.float16:
            raise TypeError(f"{n} must be torch.float16, got {t.dtype}")
        if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2] or t.stride(0) % 8:
            raise ValueError(f"{n} must be [rows, heads, d] with contiguous heads (rows may be strided "
                             "by a multiple of 8 elements)")
        if t.data_ptr() % 16:
            raise ValueError(f"{n} must be 16-byte aligned")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("pass both q_norm and k_norm, or neither")
    if q_norm is not None:
        require(q_norm, torch.float16, "q_norm")
        require(k_norm, torch.float16, "k_norm")
    check_block_table(block_table, engine_config)
    n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
    rows = infer_state.num_decoding_seqs
    hq = model_config.num_q_heads
    if q.shape != (rows, hq, d) or k.shape != (rows, hkv, d) or v.shape != k.shape:
        raise ValueError(f"q [{rows},{hq},{d}], k/v [{rows},{hkv},{d}] expected")
    if o.numel() != rows * hq * d:
        raise ValueError("o must hold num_decoding_seqs * Hq * d elements")
    if lse is not None:
        require(lse, torch.float32, "lse")
        if lse.numel() != rows * hq:
            raise ValueError("lse must hold num_decoding_seqs * num_q_heads floats")
    if cos_cache.dim() != 2 or cos_cache.shape[1] != d // 2 or sin_cache.shape != cos_cache.shape:
        raise ValueError("cos/sin caches must be [max_positions, head_dim/2]")
    if rows == 0:
        return
    if getattr(infer_state, "ignore_kvcache", False):
        raise ValueError("infer_state.ignore_kvcache is set but the forward has decode rows")
    plan = plan_for(infer_state, model_config, engine_config, block_table)
    if plan.n_rows != rows:
        raise ValueError(f"the forward's attention plan covers {plan.n_rows} rows, q has {rows}")
    status = StatusWord(q.device) if validate else None
    _lib.call("nsd_paged_attention_fused",
              q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), None, 0,
              ptr(q_norm), ptr(k_norm), float(model_config.rms_norm_eps), cos_cache.data_ptr(),
              sin_cache.data_ptr(), cos_cache.shape[0], o.data_ptr(), ptr(lse), k_cache.data_ptr(),
              v_cache.data_ptr(), n_blocks, n_layers, int(cur_layer), hq, hkv, d, bs,
              block_table.data_ptr(), block_table.shape[0], block_table.shape[1], plan.host_ptr(),
              plan.dev.data_ptr(), plan.workspace.data_ptr(), plan.workspace.numel(),
              float(infer_state.softmax_scale), ptr(status.t) if status else None, stream_of(q))
    if status is not None:
        status.check("paged_attention_fused")
