"""gfx950 kernels behind swiftLLM's kernel entry points (swiftllm.worker.kernels)."""

from .block_mgmt import (gather_allocated_blocks_and_unset, set_block_table_and_num_seq_alloc_blocks,
                         unset_block_table_and_num_seq_alloc_blocks, write_block_table_ranges)
from .kvcache_mgmt import store_kvcache
from .linear import fused_add_rmsnorm_partials, linear, linear_partials, linear_splits, sum_partials
from .paged_attn import paged_attention, paged_attention_fused
from .post_layer import argmax_rows, lm_head_argmax, post_layer_forward
from .prefill_attn import flash_attn_varlen_func, prefill_attention
from .prologue import qk_norm_rope_store, qk_norm_rope_store_partials
from .rmsnorm import fused_add_rmsnorm_inplace, rmsnorm_inplace
from .rotary_emb import rotary_embedding_inplace
from .silu_and_mul import FUSED_UP_GATE_MAX_ROWS, silu_and_mul_inplace, up_gate_silu_and_mul

__all__ = ["paged_attention", "paged_attention_fused", "store_kvcache", "rotary_embedding_inplace", "rmsnorm_inplace",
           "qk_norm_rope_store", "flash_attn_varlen_func", "prefill_attention",
           "set_block_table_and_num_seq_alloc_blocks", "unset_block_table_and_num_seq_alloc_blocks",
           "gather_allocated_blocks_and_unset", "write_block_table_ranges", "fused_add_rmsnorm_inplace",
           "silu_and_mul_inplace", "up_gate_silu_and_mul", "FUSED_UP_GATE_MAX_ROWS", "lm_head_argmax",
           "argmax_rows", "post_layer_forward", "linear", "linear_partials", "linear_splits", "sum_partials",
           "fused_add_rmsnorm_partials", "qk_norm_rope_store_partials"]
