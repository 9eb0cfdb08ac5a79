"""Block-table metadata -- drop-ins for swiftLLM's block management kernels
and NebulaSD's bank metadata writer.

Reference: swiftLLM/swiftllm/worker/kernels/block_mgmt.py:5-127 (three
Triton kernels with their wrappers) and the metadata loop of
nebulasd/src/nebulasd/workers/dma_process.py:95-125 (host index/value
arrays, two H2D copies, ``index_copy_`` into the block table).  Same
signatures and in-place semantics; the integer writes are bit-exact.
"""

from __future__ import annotations

import torch

from .. import _lib
from ._util import StatusWord, ptr, require_cuda, stream_of


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def _check_table(num_seq_allocated_blocks, block_table):
    require_cuda(num_seq_allocated_blocks, block_table)
    if block_table.dtype != torch.int32 or not block_table.is_contiguous() or block_table.dim() != 2:
        raise TypeError("block_table must be a contiguous int32 [rows, max_blocks_per_seq] tensor")
    if num_seq_allocated_blocks is not None and (num_seq_allocated_blocks.dtype != torch.int32 or
                                                 num_seq_allocated_blocks.numel() < block_table.shape[0]):
        raise TypeError("num_seq_allocated_blocks must be int32 with one entry per block-table row")


def set_block_table_and_num_seq_alloc_blocks(num_seq_allocated_blocks: torch.Tensor,
                                             block_table: torch.Tensor, candidate_blocks: torch.Tensor,
                                             seq_ids: torch.Tensor, block_needed: torch.Tensor,
                                             validate: bool = False) -> None:
    """block_mgmt.py:28-45: append ``block_needed[i]`` blocks from
    ``candidate_blocks`` (consumed in batch order) to row ``seq_ids[i]``."""
    _check_table(num_seq_allocated_blocks, block_table)
    cand, sids, need = _i32(candidate_blocks), _i32(seq_ids), _i32(block_needed)
    status = StatusWord(block_table.device) if validate else None
    _lib.call("nsd_set_block_table", num_seq_allocated_blocks.data_ptr(), block_table.data_ptr(),
              block_table.shape[0], block_table.shape[1], cand.data_ptr(), cand.numel(),
              sids.data_ptr(), need.data_ptr(), sids.numel(), ptr(status.t) if status else None,
              stream_of(block_table))
    if status is not None:
        status.check("set_block_table_and_num_seq_alloc_blocks")


def unset_block_table_and_num_seq_alloc_blocks(num_seq_allocated_blocks: torch.Tensor,
                                               block_table: torch.Tensor, seq_ids: torch.Tensor,
                                               is_block_free: torch.Tensor,
                                               validate: bool = False) -> None:
    """block_mgmt.py:64-80: free every block of the rows ``seq_ids`` and zero
    their counts."""
    _check_table(num_seq_allocated_blocks, block_table)
    if is_block_free.dtype != torch.bool or not is_block_free.is_contiguous():
        raise TypeError("is_block_free must be a contiguous bool tensor")
    sids = _i32(seq_ids)
    status = StatusWord(block_table.device) if validate else None
    _lib.call("nsd_unset_block_table", num_seq_allocated_blocks.data_ptr(), block_table.data_ptr(),
              block_table.shape[0], block_table.shape[1], sids.data_ptr(), sids.numel(),
              is_block_free.data_ptr(), is_block_free.numel(), ptr(status.t) if status else None,
              stream_of(block_table))
    if status is not None:
        status.check("unset_block_table_and_num_seq_alloc_blocks")


def gather_allocated_blocks_and_unset(num_seq_allocated_blocks: torch.Tensor,
                                      block_table: torch.Tensor, seq_ids: torch.Tensor,
                                      is_block_free: torch.Tensor,
                                      validate: bool = False) -> torch.Tensor:
    """block_mgmt.py:108-127: the blocks of the rows ``seq_ids``, back to back,
    after which they are free and the rows' counts zero.  Like the
    reference, the output size is read back to the host once."""
    _check_table(num_seq_allocated_blocks, block_table)
    if is_block_free.dtype != torch.bool or not is_block_free.is_contiguous():
        raise TypeError("is_block_free must be a contiguous bool tensor")
    if seq_ids.numel() == 0:
        return torch.empty((0,), dtype=torch.int32, device=block_table.device)
    sids = _i32(seq_ids)
    total = int(num_seq_allocated_blocks[sids.long()].sum().item())
    out = torch.empty((total,), dtype=torch.int32, device=block_table.device)
    status = StatusWord(block_table.device) if validate else None
    _lib.call("nsd_gather_allocated_blocks_and_unset", num_seq_allocated_blocks.data_ptr(),
              block_table.data_ptr(), block_table.shape[0], block_table.shape[1], sids.data_ptr(),
              sids.numel(), is_block_free.data_ptr(), is_block_free.numel(), out.data_ptr(), total,
              ptr(status.t) if status else None, stream_of(block_table))
    if status is not None:
        status.check("gather_allocated_blocks_and_unset")
    return out


def write_block_table_ranges(block_table: torch.Tensor, rows, begins, counts,
                             num_seq_allocated_blocks: torch.Tensor | None = None,
                             validate: bool = False) -> None:
    """Bank metadata (dma_process.py:95-125; block_manager.py:685-691): row
    ``rows[i]`` gets the contiguous block ids ``begins[i] .. begins[i] +
    counts[i] - 1``.  ``rows``/``begins``/``counts``: host sequences (one small
    H2D copy) or device int32 tensors."""
    _check_table(num_seq_allocated_blocks, block_table)
    dev = block_table.device
    if isinstance(rows, torch.Tensor) and rows.is_cuda:
        r, b, c = _i32(rows), _i32(begins), _i32(counts)
    else:
        host = torch.tensor([list(rows), list(begins), list(counts)], dtype=torch.int32)
        packed = host.pin_memory().to(dev, non_blocking=True) if torch.cuda.is_available() else host.to(dev)
        r, b, c = packed[0], packed[1], packed[2]
    if not (r.numel() == b.numel() == c.numel()):
        raise ValueError("rows, begins and counts must have the same length")
    status = StatusWord(dev) if validate else None
    _lib.call("nsd_write_block_ranges", block_table.data_ptr(), block_table.shape[0],
              block_table.shape[1], r.data_ptr(), b.data_ptr(), c.data_ptr(), r.numel(),
              ptr(num_seq_allocated_blocks), ptr(status.t) if status else None, stream_of(block_table))
    if status is not None:
        status.check("write_block_table_ranges")
