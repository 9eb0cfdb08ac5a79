"""Shared test helpers: oracle inputs from device workloads and tolerance checks."""

from __future__ import annotations

import numpy as np
import torch

# Tolerances of the path (fp16 storage, fp32 math), written once here.
ATOL_O = 2e-3
RTOL_O = 1e-2
ATOL_LSE = 1e-4


def compact_cache(k_cache, v_cache, block_table, seq_ids, seq_lens, layer):
    """Referenced blocks of one layer as a small numpy cache + remapped table.

    Returns (k [n,1,Hkv,16,d] fp16, v, block_table [rows_of_table, nb] int64,
    layer 0) so the numpy oracle never touches the full pool.
    """
    bs = k_cache.shape[3]
    bt = block_table.cpu().numpy()
    need = {}
    for sid, sl in zip(seq_ids, seq_lens):
        need[sid] = max(need.get(sid, 0), (int(sl) + bs - 1) // bs)
    ids = sorted({int(bt[s, i]) for s, n in need.items() for i in range(n)})
    remap = {b: i for i, b in enumerate(ids)}
    idx = torch.tensor(ids, dtype=torch.long, device=k_cache.device)
    k_small = k_cache[idx, layer].unsqueeze(1).cpu().numpy()
    v_small = v_cache[idx, layer].unsqueeze(1).cpu().numpy()
    nb = max(need.values())
    bt_small = np.zeros((bt.shape[0], nb), dtype=np.int64)
    for s, n in need.items():
        bt_small[s, :n] = [remap[int(b)] for b in bt[s, :n]]
    return k_small, v_small, bt_small


def assert_close(got, want, atol, rtol, what):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(want))), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside atol={atol} "
                             f"rtol={rtol}; worst at {i}: got {got[i]}, want {want[i]}")
    return float(err.max())
