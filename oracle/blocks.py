"""numpy restatement of the block-table metadata writes (the oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``; never by the product package.

All reference citations are relative to the reference repository root;
``K = swiftLLM/swiftllm/worker/kernels``.

How each function is pinned (``tests/test_oracle_blocks.py``):

* ``write_block_ranges`` -- the reference's own literal cases of
  ``swiftLLM/tests/test_block_manager_double_bank.py`` (committed as data in
  ``tests/golden/block_table_cases.json``) and equality with the reference's
  formulation (flat indices ``row * stride + arange(count)``, values
  ``arange(begin, begin + count)``, ``index_copy_``) run with torch.
* ``set_block_table`` / ``unset_block_table`` /
  ``gather_allocated_blocks_and_unset`` -- round trips (set then gather gives
  the candidates back in batch order and frees exactly them; set then unset
  frees exactly them and zeroes the counts), the untouched-rows canary, and
  planted mistakes (inclusive instead of exclusive offsets, a missing count
  update) that these checks reject.
"""

from __future__ import annotations

import numpy as np

__all__ = ["write_block_ranges", "set_block_table", "unset_block_table",
           "gather_allocated_blocks_and_unset"]


def write_block_ranges(block_table, rows, begins, counts, num_alloc=None):
    """nebulasd/src/nebulasd/workers/dma_process.py:111-121: for each
    (row, begin, count) the flat indices ``row * stride + arange(count)`` get
    the values ``arange(begin, begin + count)`` (index_copy_ into the
    flattened table); swiftLLM/swiftllm/worker/block_manager.py:685-691 also
    sets ``num_seq_allocated_blocks[row] = count``.  In place."""
    bt = block_table.reshape(-1)
    stride = block_table.shape[1]
    for row, begin, count in zip(rows, begins, counts):
        bt[row * stride: row * stride + count] = np.arange(begin, begin + count, dtype=block_table.dtype)
        if num_alloc is not None:
            num_alloc[row] = count


def set_block_table(num_alloc, block_table, candidate_blocks, seq_ids, block_needed):
    """K/block_mgmt.py:5-45: entry i (seq s) takes candidate_blocks
    [cumsum[i-1], cumsum[i]) (:41, :16) into block_table[s][num_alloc[s]:]
    (:17-21) and adds block_needed[i] to num_alloc[s] (:22).  In place."""
    cum = np.cumsum(np.asarray(block_needed, dtype=np.int64))
    for i, (s, need) in enumerate(zip(seq_ids, block_needed)):
        start = int(cum[i] - need)
        have = int(num_alloc[s])
        block_table[s, have:have + need] = candidate_blocks[start:start + need]
        num_alloc[s] = have + need


def unset_block_table(num_alloc, block_table, seq_ids, is_block_free):
    """K/block_mgmt.py:48-80: every block of row s (its first num_alloc[s]
    entries) becomes free (:58-60) and num_alloc[s] = 0 (:61).  In place."""
    for s in seq_ids:
        n = int(num_alloc[s])
        is_block_free[block_table[s, :n]] = True
        num_alloc[s] = 0


def gather_allocated_blocks_and_unset(num_alloc, block_table, seq_ids, is_block_free):
    """K/block_mgmt.py:83-127: the blocks of rows seq_ids[0], seq_ids[1], ...
    back to back at offsets cumsum(num_alloc[seq_ids]) (:118-119, :97-101),
    marked free, counts zeroed (:102-103).  Returns the gathered ids."""
    counts = [int(num_alloc[s]) for s in seq_ids]
    out = np.zeros(sum(counts), dtype=np.int32)
    off = 0
    for s, n in zip(seq_ids, counts):
        out[off:off + n] = block_table[s, :n]
        is_block_free[block_table[s, :n]] = True
        off += n
    for s in seq_ids:
        num_alloc[s] = 0
    return out
