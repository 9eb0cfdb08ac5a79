"""GPU parity of the block-table metadata kernels: bit-exact against the
numpy oracle and the reference's own torch formulation."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from nebulasd_amd.kernels import (gather_allocated_blocks_and_unset,
                                  set_block_table_and_num_seq_alloc_blocks,
                                  unset_block_table_and_num_seq_alloc_blocks, write_block_table_ranges)

pytestmark = pytest.mark.gpu


def _state(rng, n_seqs=64, stride=128, blocks=4096):
    bt = np.full((n_seqs, stride), -1, np.int32)
    na = rng.integers(0, 20, n_seqs).astype(np.int32)
    free = np.zeros(blocks, bool)
    perm = rng.permutation(blocks).astype(np.int32)
    k = 0
    for s in range(n_seqs):
        bt[s, :na[s]] = perm[k:k + na[s]]
        k += na[s]
    return bt, na, free, perm[k:]


def _dev(gpu, *arrays):
    return [torch.from_numpy(a.copy()).to(gpu) for a in arrays]


def test_write_block_ranges_bank_layout(gpu):
    """A bank switch's metadata: every row of a bank gets its contiguous range
    (dma_process.py:111-121), against the reference's index_copy_ on the GPU."""
    rng = np.random.default_rng(0)
    rows = rng.permutation(128)[:100].tolist()
    counts = rng.integers(0, 257, 100).tolist()
    begins = np.cumsum([0] + counts[:-1]).tolist()  # a bank's bump allocation
    bt0 = rng.integers(-9, 9, (128, 256)).astype(np.int32)
    na0 = np.zeros(128, np.int32)
    bt, na = _dev(gpu, bt0, na0)
    write_block_table_ranges(bt, rows, begins, counts, na, validate=True)
    ref = torch.from_numpy(bt0.copy()).to(gpu)
    ix = torch.cat([torch.arange(r * 256, r * 256 + n, device=gpu) for r, n in zip(rows, counts)])
    val = torch.cat([torch.arange(b, b + n, dtype=torch.int32, device=gpu) for b, n in zip(begins, counts)])
    ref.view(-1).index_copy_(0, ix, val)
    torch.cuda.synchronize()
    assert torch.equal(bt, ref)
    oracle.write_block_ranges(bt0, rows, begins, counts, na0)
    assert np.array_equal(bt.cpu().numpy(), bt0) and np.array_equal(na.cpu().numpy(), na0)


@pytest.mark.parametrize("seed", [1, 2])
def test_set_unset_gather_match_oracle(gpu, seed):
    rng = np.random.default_rng(seed)
    bt0, na0, free0, spare = _state(rng)
    seqs = rng.permutation(64)[:40].astype(np.int32)
    need = rng.integers(0, 30, 40).astype(np.int32)
    need = np.minimum(need, 128 - na0[seqs])
    cand = spare[:need.sum()].astype(np.int64)  # torch.nonzero gives int64 (block_manager.py:176)
    bt, na, free = _dev(gpu, bt0, na0, free0)
    set_block_table_and_num_seq_alloc_blocks(na, bt, torch.from_numpy(cand).to(gpu),
                                             torch.from_numpy(seqs).to(gpu), torch.from_numpy(need).to(gpu),
                                             validate=True)
    oracle.set_block_table(na0, bt0, cand.astype(np.int32), seqs.tolist(), need.tolist())
    torch.cuda.synchronize()
    assert np.array_equal(bt.cpu().numpy(), bt0) and np.array_equal(na.cpu().numpy(), na0)
    g_seqs = seqs[:25]
    out = gather_allocated_blocks_and_unset(na, bt, torch.from_numpy(g_seqs).to(gpu), free, validate=True)
    want = oracle.gather_allocated_blocks_and_unset(na0, bt0, g_seqs.tolist(), free0)
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == want.tolist()
    assert np.array_equal(free.cpu().numpy(), free0) and np.array_equal(na.cpu().numpy(), na0)
    u_seqs = seqs[25:]
    unset_block_table_and_num_seq_alloc_blocks(na, bt, torch.from_numpy(u_seqs).to(gpu), free, validate=True)
    oracle.unset_block_table(na0, bt0, u_seqs.tolist(), free0)
    torch.cuda.synchronize()
    assert np.array_equal(free.cpu().numpy(), free0) and np.array_equal(na.cpu().numpy(), na0)


def test_block_kernels_flag_bad_metadata(gpu):
    """Rows outside the table, counts past a row and block ids outside the
    pool are skipped and flagged, never written."""
    bt = torch.full((8, 16), -1, dtype=torch.int32, device=gpu)
    na = torch.zeros(8, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="invalid metadata"):
        write_block_table_ranges(bt, [3, 9], [0, 0], [4, 4], na, validate=True)  # row 9 past the table
    assert bt[3, :4].tolist() == [0, 1, 2, 3] and (bt[[0, 1, 2, 4, 5, 6, 7]] == -1).all()
    with pytest.raises(RuntimeError, match="invalid metadata"):
        write_block_table_ranges(bt, [1], [0], [17], na, validate=True)  # count past the row
    assert (bt[1] == -1).all()
    free = torch.zeros(10, dtype=torch.bool, device=gpu)
    bt[5, :3] = torch.tensor([2, 40, 7], dtype=torch.int32, device=gpu)  # 40 is past the pool
    na[5] = 3
    with pytest.raises(RuntimeError, match="invalid metadata"):
        unset_block_table_and_num_seq_alloc_blocks(na, bt, torch.tensor([5], device=gpu), free, validate=True)
    assert free.nonzero().flatten().tolist() == [2, 7] and na[5].item() == 0
