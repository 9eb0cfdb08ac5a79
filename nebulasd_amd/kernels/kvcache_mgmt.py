"""KV-cache store -- drop-in for swiftLLM's ``store_kvcache``.

Reference: swiftLLM/swiftllm/worker/kernels/kvcache_mgmt.py:81-122 (wrapper),
:50-79 (decode/verify rows), :10-48 (prefill sequences).  Bit-exact copies
into the ``[num_blocks, num_layers, num_kv_heads, block_size, head_dim]`` cache.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import StatusWord, cache_dims, check_block_table, ptr, require, require_cuda, stream_of


def store_kvcache(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  block_table: torch.Tensor, model_config, engine_config, infer_state,
                  cur_layer: int, validate: bool = False) -> None:
    """Store every token's K/V of the forward at layer ``cur_layer``.

    ``k``/``v``: [num_tokens, Hkv, d] fp16 -- prefill tokens first, then one
    row per decode/verify row (kvcache_mgmt.py:104-122).
    """
    require_cuda(k, v, k_cache, v_cache, block_table)
    for t, n in ((k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        require(t, torch.float16, n)
    check_block_table(block_table, engine_config)
    require(infer_state.seq_ids, torch.int32, "infer_state.seq_ids")
    require(infer_state.decoding_seq_lens, torch.int32, "infer_state.decoding_seq_lens")
    n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
    if engine_config.block_size != bs:
        raise ValueError("engine_config.block_size does not match the cache layout")
    if k.shape[1:] != (hkv, d) or v.shape != k.shape:
        raise ValueError(f"k/v must be [tokens, {hkv}, {d}]")
    status = StatusWord(k.device) if validate else None
    st = stream_of(k)
    bt_rows, bt_stride = block_table.shape
    npf = infer_state.num_prefill_seqs
    if npf > 0:
        _lib.call("nsd_store_kvcache_prefill",
                  k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                  block_table.data_ptr(), bt_rows, bt_stride, infer_state.seq_ids.data_ptr(),
                  infer_state.prefill_seq_start_locs.data_ptr(),
                  infer_state.prefill_seq_lens.data_ptr(), npf, infer_state.max_prefill_len,
                  n_blocks, n_layers, int(cur_layer), hkv, d, bs,
                  ptr(status.t) if status else None, st)
    nd = infer_state.num_decoding_seqs
    if nd > 0:
        off = infer_state.num_prefill_tokens
        kd, vd = k[off:], v[off:]
        if kd.shape[0] != nd:
            raise ValueError("k/v hold fewer decode rows than infer_state.num_decoding_seqs")
        _lib.call("nsd_store_kvcache",
                  kd.data_ptr(), vd.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                  block_table.data_ptr(), bt_rows, bt_stride,
                  infer_state.seq_ids[npf:].data_ptr(), infer_state.decoding_seq_lens.data_ptr(),
                  nd, n_blocks, n_layers, int(cur_layer), hkv, d, bs,
                  ptr(status.t) if status else None, st)
    if status is not None:
        status.check("store_kvcache")
