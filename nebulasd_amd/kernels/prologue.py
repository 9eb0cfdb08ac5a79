"""Fused attention prologue: QK-RMSNorm + RoPE + KV store in one launch.

Replaces the sequence of swiftLLM/swiftllm/worker/layers/transformer_layer.py:114-145
(``rmsnorm_inplace(q)``, ``rmsnorm_inplace(k)``, ``rotary_embedding_inplace``,
``store_kvcache``) for the decode/verify rows of a forward.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import StatusWord, cache_dims, check_block_table, ptr, require, require_cuda, stream_of


def qk_norm_rope_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, block_table: torch.Tensor, q_norm: torch.Tensor | None,
                       k_norm: torch.Tensor | None, model_config, engine_config, infer_state,
                       cur_layer: int, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                       validate: bool = False, q_out: torch.Tensor | None = None) -> None:
    """Prologue of the decode/verify rows.

    ``q`` [rows, Hq, d], ``k``/``v`` [rows, Hkv, d] fp16 are the decode-row
    slices (``x[num_prefill_tokens:]``); q and k are normalised and rotated
    in place at position ``decoding_seq_lens - 1``; K (rotated) and V are
    stored into the cache slot of each row.  ``cos_cache``/``sin_cache`` are
    the full [max_positions, d/2] fp16 tables (model.py:242-252).  Pass
    ``q_norm = k_norm = None`` for models without QK-norm.

    q, k and v may be row-strided slices of one fused q/k/v projection
    ([rows, (Hq + 2*Hkv) * d] viewed per head); then q is left as it is and
    the normalised, rotated q goes to ``q_out`` (contiguous [rows, Hq, d],
    what ``paged_attention`` reads).  With contiguous q and no ``q_out`` q is
    processed in place, as in the reference.
    """
    require_cuda(q, k, v, k_cache, v_cache, block_table, cos_cache, sin_cache, q_norm, k_norm, q_out)
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache"), (cos_cache, "cos_cache"), (sin_cache, "sin_cache")):
        require(t, torch.float16, n)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t.dtype != torch.float16:
            raise TypeError(f"{n} must be torch.float16, got {t.dtype}")
        if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2] or t.stride(0) % 2:
            raise ValueError(f"{n} must be [rows, heads, d] with contiguous heads (rows may be strided)")
    if q_out is not None:
        require(q_out, torch.float16, "q_out")
        if q_out.shape != q.shape:
            raise ValueError("q_out must have q's shape")
    check_block_table(block_table, engine_config)
    if (q_norm is None) != (k_norm is None):
        raise ValueError("pass both q_norm and k_norm, or neither")
    if q_norm is not None:
        require(q_norm, torch.float16, "q_norm")
        require(k_norm, torch.float16, "k_norm")
    n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
    rows = infer_state.num_decoding_seqs
    hq = model_config.num_q_heads
    if q.shape != (rows, hq, d) or k.shape != (rows, hkv, d) or v.shape != k.shape:
        raise ValueError(f"q [{rows},{hq},{d}], k/v [{rows},{hkv},{d}] expected")
    if cos_cache.dim() != 2 or cos_cache.shape[1] != d // 2 or sin_cache.shape != cos_cache.shape:
        raise ValueError("cos/sin caches must be [max_positions, head_dim/2]")
    if rows == 0:
        return
    if getattr(infer_state, "ignore_kvcache", False):
        # the reference stores nothing then, and asserts there are no decode rows
        # (transformer_layer.py:133, :171); decode rows must store their K/V
        raise ValueError("infer_state.ignore_kvcache is set but the forward has decode rows")
    npf = infer_state.num_prefill_seqs
    status = StatusWord(q.device) if validate else None
    tail = (ptr(q_norm), ptr(k_norm), float(model_config.rms_norm_eps), cos_cache.data_ptr(), sin_cache.data_ptr(),
            cos_cache.shape[0], k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
            block_table.shape[0], block_table.shape[1], infer_state.seq_ids[npf:].data_ptr(),
            infer_state.decoding_seq_lens.data_ptr(), rows, n_blocks, n_layers, int(cur_layer),
            hq, hkv, d, bs, ptr(status.t) if status else None, stream_of(q))
    if q_out is None and q.is_contiguous() and k.is_contiguous() and v.is_contiguous():
        _lib.call("nsd_qk_norm_rope_store", q.data_ptr(), k.data_ptr(), v.data_ptr(), *tail)
    else:
        if q_out is None:
            raise ValueError("strided q needs q_out (a contiguous [rows, Hq, d] buffer)")
        _lib.call("nsd_qk_norm_rope_store_strided", q.data_ptr(), q.stride(0), q_out.data_ptr(), k.data_ptr(),
                  k.stride(0), v.data_ptr(), v.stride(0), *tail)
    if status is not None:
        status.check("qk_norm_rope_store")


def qk_norm_rope_store_partials(partials: torch.Tensor, q_out: torch.Tensor, k_cache: torch.Tensor,
                                v_cache: torch.Tensor, block_table: torch.Tensor, q_norm: torch.Tensor | None,
                                k_norm: torch.Tensor | None, model_config, engine_config, infer_state,
                                cur_layer: int, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                                validate: bool = False) -> None:
    """The prologue over the fused q/k/v projection of the decode/verify rows
    given as split partials [splits, rows, (Hq + 2*Hkv) * d] (``linear_partials``):
    q normalised and rotated into ``q_out`` [rows, Hq, d], K and V stored into
    the cache slots of the rows (transformer_layer.py:107-145)."""
    require_cuda(partials, q_out, k_cache, v_cache, block_table, cos_cache, sin_cache, q_norm, k_norm)
    require(partials, torch.float32, "partials")
    for t, n in ((q_out, "q_out"), (k_cache, "k_cache"), (v_cache, "v_cache"), (cos_cache, "cos_cache"),
                 (sin_cache, "sin_cache")):
        require(t, torch.float16, n)
    check_block_table(block_table, engine_config)
    if (q_norm is None) != (k_norm is None):
        raise ValueError("pass both q_norm and k_norm, or neither")
    n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
    rows, hq = infer_state.num_decoding_seqs, model_config.num_q_heads
    if partials.dim() != 3 or tuple(partials.shape[1:]) != (rows, (hq + 2 * hkv) * d):
        raise ValueError(f"partials must be [splits, {rows}, {(hq + 2 * hkv) * d}]")
    if tuple(q_out.shape) != (rows, hq, d):
        raise ValueError(f"q_out must be [{rows}, {hq}, {d}]")
    if rows == 0:
        return
    if getattr(infer_state, "ignore_kvcache", False):
        raise ValueError("infer_state.ignore_kvcache is set but the forward has decode rows")
    npf = infer_state.num_prefill_seqs
    status = StatusWord(q_out.device) if validate else None
    _lib.call("nsd_qk_norm_rope_store_partials", partials.data_ptr(), partials.shape[0], q_out.data_ptr(),
              ptr(q_norm), ptr(k_norm), float(model_config.rms_norm_eps), cos_cache.data_ptr(), sin_cache.data_ptr(),
              cos_cache.shape[0], k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
              block_table.shape[0], block_table.shape[1], infer_state.seq_ids[npf:].data_ptr(),
              infer_state.decoding_seq_lens.data_ptr(), rows, n_blocks, n_layers, int(cur_layer), hq, hkv, d, bs,
              ptr(status.t) if status else None, stream_of(q_out))
    if status is not None:
        status.check("qk_norm_rope_store_partials")
