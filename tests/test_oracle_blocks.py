"""Pins for the block-table oracle (CPU only): the reference's literal cases,
the reference's own index_copy_ formulation run with torch, round trips, and
planted mistakes the checks must reject."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "block_table_cases.json").read_text())


def test_write_ranges_golden():
    for case in ("fill", "bump"):
        c = GOLDEN[case]
        bt = np.full((GOLDEN["max_seqs"], GOLDEN["max_blocks_per_seq"]), -7, np.int32)
        na = np.zeros(GOLDEN["max_seqs"], np.int32)
        oracle.write_block_ranges(bt, c["rows"], c["begins"], c["counts"], na)
        for row, want in c["expect_row"].items():
            assert bt[int(row), :len(want)].tolist() == want
            assert (bt[int(row), len(want):] == -7).all()
            assert na[int(row)] == c["expect_count"][row]
        untouched = [r for r in range(GOLDEN["max_seqs"]) if str(r) not in c["expect_row"]]
        assert (bt[untouched] == -7).all()


def reference_writer(block_table, rows, begins, counts):
    """dma_process.py:111-121 with torch: flat indices and values, index_copy_."""
    stride = block_table.shape[1]
    ix = np.concatenate([np.arange(r * stride, r * stride + n) for r, n in zip(rows, counts)]).astype(np.int64)
    val = np.concatenate([np.arange(b, b + n) for b, n in zip(begins, counts)]).astype(np.int32)
    t = torch.from_numpy(block_table.copy())
    t.view(-1).index_copy_(0, torch.from_numpy(ix), torch.from_numpy(val))
    return t.numpy()


def test_write_ranges_match_reference_formulation():
    rng = np.random.default_rng(0)
    bt = rng.integers(-100, 100, (64, 96)).astype(np.int32)
    rows = rng.permutation(64)[:20].tolist()
    counts = rng.integers(0, 97, 20).tolist()
    begins = rng.integers(0, 10_000, 20).tolist()
    want = reference_writer(bt, rows, begins, counts)
    oracle.write_block_ranges(bt, rows, begins, counts)
    np.testing.assert_array_equal(bt, want)


def _pool(rng, n_seqs=12, stride=40, blocks=400):
    bt = np.full((n_seqs, stride), -1, np.int32)
    na = rng.integers(0, 5, n_seqs).astype(np.int32)
    free = np.zeros(blocks, bool)
    used = rng.permutation(blocks)
    k = 0
    for s in range(n_seqs):
        bt[s, :na[s]] = used[k:k + na[s]]
        k += na[s]
    return bt, na, free, used[k:]


def test_set_then_gather_round_trip():
    rng = np.random.default_rng(1)
    bt, na, free, spare = _pool(rng)
    seqs = [7, 2, 9, 0]
    need = [3, 0, 5, 2]
    cand = spare[:sum(need)].astype(np.int32)
    before = na.copy()
    oracle.set_block_table(na, bt, cand, seqs, need)
    assert [int(na[s]) for s in seqs] == [int(before[s]) + n for s, n in zip(seqs, need)]
    out = oracle.gather_allocated_blocks_and_unset(na, bt, seqs, free)
    # each row's old blocks then its new candidates, rows in batch order
    pos, want = 0, []
    for s, n in zip(seqs, need):
        want += list(bt[s, :before[s]]) + list(cand[pos:pos + n])
        pos += n
    assert out.tolist() == want
    assert free.sum() == len(want) and free[out].all()
    assert all(na[s] == 0 for s in seqs)


def test_set_then_unset_frees_exactly_those_blocks():
    rng = np.random.default_rng(2)
    bt, na, free, spare = _pool(rng)
    seqs, need = [1, 5, 11], [4, 1, 6]
    cand = spare[:11].astype(np.int32)
    untouched = bt[[r for r in range(12) if r not in seqs]].copy()
    oracle.set_block_table(na, bt, cand, seqs, need)
    blocks = np.concatenate([bt[s, :na[s]] for s in seqs])
    oracle.unset_block_table(na, bt, seqs, free)
    assert set(np.nonzero(free)[0].tolist()) == set(blocks.tolist())
    assert all(na[s] == 0 for s in seqs)
    np.testing.assert_array_equal(bt[[r for r in range(12) if r not in seqs]], untouched)


def test_block_pins_reject_planted_mistakes():
    rng = np.random.default_rng(3)
    bt, na, free, spare = _pool(rng)
    seqs, need = [3, 4, 8], [2, 3, 4]
    cand = spare[:9].astype(np.int32)
    good_bt, good_na = bt.copy(), na.copy()
    oracle.set_block_table(good_na, good_bt, cand, seqs, need)
    # (1) inclusive instead of exclusive candidate offsets
    bad_bt, bad_na = bt.copy(), na.copy()
    cum = np.cumsum(need)
    for i, (s, n) in enumerate(zip(seqs, need)):
        start = int(cum[i])  # planted: should be cum[i] - n
        take = cand[start:start + n]
        bad_bt[s, bad_na[s]:bad_na[s] + len(take)] = take
        bad_na[s] += n
    assert not np.array_equal(bad_bt, good_bt)
    # (2) the count not updated: a second set would overwrite the first
    bad_bt2, bad_na2 = bt.copy(), na.copy()
    for i, (s, n) in enumerate(zip(seqs, need)):
        start = int(cum[i] - n)
        bad_bt2[s, bad_na2[s]:bad_na2[s] + n] = cand[start:start + n]
    assert not np.array_equal(bad_na2, good_na)
