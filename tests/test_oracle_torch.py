"""The PyTorch-CPU restatement (oracle/attention_torch.py), which ``bench.py``
times as the CPU baseline, against the pinned numpy oracle: random rows,
ragged lengths, rows of one sequence interleaved with others, GQA groups of
2 and 4, seq_len 1 and block-boundary lengths.  fp32 against float64:
o within 2e-5 abs, LSE within 2e-5 abs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle.attention_torch import paged_attention_rowwise


def case(seed, hq, hkv, rows_of):
    rng = np.random.default_rng(seed)
    d, bs, layers = 32, 16, 3
    n_seq = len(rows_of)
    max_len = max(max(v) for v in rows_of)
    width = (max_len + bs - 1) // bs
    n_blocks = n_seq * width + 3
    kc = rng.standard_normal((n_blocks, layers, hkv, bs, d)).astype(np.float16)
    vc = rng.standard_normal((n_blocks, layers, hkv, bs, d)).astype(np.float16)
    bt = rng.permutation(n_blocks)[:n_seq * width].reshape(n_seq, width).astype(np.int32)
    sids, lens = [], []
    for s, ls in enumerate(rows_of):
        for n in ls:
            sids.append(s)
            lens.append(n)
    return kc, vc, bt, sids, lens, rng, d


@pytest.mark.parametrize("seed,hq,hkv", [(0, 4, 2), (1, 8, 2), (2, 16, 8)])
def test_torch_restatement_matches_numpy_oracle(seed, hq, hkv):
    kc, vc, bt, sids, lens, rng, d = case(seed, hq, hkv, [[1], [15, 16, 17, 18, 19], [33], [64, 65]])
    # interleave: move the last sequence's first row to the front
    sids = [sids[-2]] + sids[:-2] + [sids[-1]]
    lens = [lens[-2]] + lens[:-2] + [lens[-1]]
    q = rng.standard_normal((len(sids), hq, d)).astype(np.float16)
    want_o, want_l = oracle.paged_attention(q, kc, vc, bt, sids, lens, layer=1)
    got_o, got_l = paged_attention_rowwise(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                                           torch.from_numpy(bt), sids, lens, 1)
    np.testing.assert_allclose(got_o.numpy(), want_o, atol=2e-5, rtol=0)
    np.testing.assert_allclose(got_l.numpy(), want_l, atol=2e-5, rtol=0)


def test_torch_restatement_catches_wrong_layer():
    """A planted mistake (reading another layer) is visible at this tolerance."""
    kc, vc, bt, sids, lens, rng, d = case(3, 4, 2, [[40, 41]])
    q = rng.standard_normal((2, 4, d)).astype(np.float16)
    want_o, _ = oracle.paged_attention(q, kc, vc, bt, sids, lens, layer=1)
    got_o, _ = paged_attention_rowwise(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                                       torch.from_numpy(bt), sids, lens, 2)
    assert np.abs(got_o.numpy() - want_o).max() > 1e-2
