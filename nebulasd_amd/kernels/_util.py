"""Shared argument checks and pointer helpers for the kernel wrappers."""

from __future__ import annotations

import torch


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of the current torch stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("gfx950 kernels need GPU tensors (there is no CPU fallback)")


def require(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def check_block_table(block_table: torch.Tensor, engine_config) -> None:
    """The block table's row length must be ``engine_config.max_blocks_per_seq``:
    the reference kernels index rows with that stride (paged_attn.py:208,
    kvcache_mgmt.py:121), these wrappers with ``block_table.shape[1]``."""
    require(block_table, torch.int32, "block_table")
    if block_table.dim() != 2:
        raise ValueError("block_table must be [rows, max_blocks_per_seq]")
    if int(engine_config.max_blocks_per_seq) != block_table.shape[1]:
        raise ValueError(f"block_table rows hold {block_table.shape[1]} entries but "
                         f"engine_config.max_blocks_per_seq is {engine_config.max_blocks_per_seq}")


def cache_dims(k_cache: torch.Tensor):
    """(num_blocks, num_layers, num_kv_heads, block_size, head_dim) of a KV cache."""
    if k_cache.dim() != 5:
        raise ValueError("KV cache must be [num_blocks, num_layers, num_kv_heads, block_size, head_dim]")
    return tuple(int(x) for x in k_cache.shape)


class StatusWord:
    """Optional device status word; ``check()`` synchronises and raises on flags."""

    NAMES = {1: "block id outside the pool", 2: "seq_id/position outside the block table",
             4: "position outside the RoPE table"}

    def __init__(self, device):
        self.t = torch.zeros(1, dtype=torch.int32, device=device)

    def check(self, what: str) -> None:
        v = int(self.t.item())
        if v:
            bad = [n for b, n in self.NAMES.items() if v & b]
            raise RuntimeError(f"{what}: invalid metadata ({', '.join(bad)})")
