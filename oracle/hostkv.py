"""numpy restatement of the HostKV block-range copies (the oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``; never by the product package.

All reference citations are relative to the reference repository root;
``KV = nebulasd/src/nebulasd/kv``.

Caches and host planes are uint8 arrays ``[blocks, block_bytes]``: a block
is a byte image, the same on both sides (KV/cuda_transfer.py:41-46).

How each function is pinned (``tests/test_oracle_hostkv.py``):

* ``copy_block_ranges`` -- the reference's own copy benchmark fixture and
  byte check (nebulasd/tests/support/copy_benchmark.py:61-98: one guard
  block each side of every request, payload bytes ``pattern(plane, slot,
  iteration)``, guards 204 on the device and 221 on the host), both
  directions; equality with a block-by-block copy loop on random plans with
  adjacent, zero-count and overlapping regions; the reference's range errors
  (KV/transfer.py:23-26, KV/cuda_transfer.py:82-85).
* ``swap_blocks`` -- hand-built id lists whose runs are known (consecutive
  on both sides, broken on one side only, repeated ids), equality with a
  block-by-block loop, and swap-out followed by swap-in restoring the cache.
* Planted mistakes (a host offset off by one block, K and V planes swapped,
  a run that ignores the target side's break) that these checks reject.
"""

from __future__ import annotations

import numpy as np

__all__ = ["copy_block_ranges", "swap_blocks", "swap_runs", "benchmark_pattern",
           "fill_benchmark_buffers", "check_benchmark_buffers", "DEVICE_GUARD", "HOST_GUARD"]

DEVICE_GUARD = 204  # copy_benchmark.py:75
HOST_GUARD = 221    # copy_benchmark.py:76


def copy_block_ranges(k_cache, v_cache, host_k, host_v, regions, direction):
    """KV/cuda_transfer.py:92-106: for every region (gpu_begin, host_begin,
    count) in order, K plane then V plane, ``count`` blocks between device
    blocks [gpu_begin, gpu_begin + count) and host blocks [host_begin,
    host_begin + count) (host_begin is absolute: extent.offset_blocks +
    region.host_begin_block, :98).  "D2H" writes the host planes, "H2D" the
    caches.  Ranges are checked first (KV/transfer.py:23-26,
    KV/cuda_transfer.py:82-85); zero-count regions move nothing (:96-97).
    In place."""
    if direction not in ("D2H", "H2D"):
        raise ValueError("copy plan requires a direction and non-empty batch")
    for g, h, c in regions:
        if min(g, h, c) < 0:
            raise ValueError("negative copy range")
        if g + c > k_cache.shape[0]:
            raise ValueError("copy exceeds GPU KV cache")
        if h + c > host_k.shape[0]:
            raise ValueError("copy exceeds HostKV plane")
    for g, h, c in regions:
        if c == 0:
            continue
        for cache, host in ((k_cache, host_k), (v_cache, host_v)):
            if direction == "D2H":
                host[h:h + c] = cache[g:g + c]
            else:
                cache[g:g + c] = host[h:h + c]


def swap_runs(source_block_ids, target_block_ids):
    """swiftLLM/csrc/src/block_swapping.cpp:32-49: maximal runs of entries
    whose source and target ids both grow by one, as (source_start,
    target_start, length) in list order."""
    runs = []
    i, n = 0, len(source_block_ids)
    while i < n:
        j = i + 1
        while (j < n and source_block_ids[j] == source_block_ids[j - 1] + 1
               and target_block_ids[j] == target_block_ids[j - 1] + 1):
            j += 1
        runs.append((int(source_block_ids[i]), int(target_block_ids[i]), j - i))
        i = j
    return runs


def swap_blocks(source_block_ids, target_block_ids, is_swap_in, k_cache, v_cache, k_swap, v_swap):
    """swiftLLM/csrc/src/block_swapping.cpp:22-85: each run copies K then V
    (:51-82), swap space -> cache when ``is_swap_in`` else cache -> swap
    space.  Returns the runs.  In place."""
    runs = swap_runs(source_block_ids, target_block_ids)
    for s, t, n in runs:
        for cache, swap in ((k_cache, k_swap), (v_cache, v_swap)):
            if is_swap_in:
                cache[t:t + n] = swap[s:s + n]
            else:
                swap[t:t + n] = cache[s:s + n]
    return runs


def benchmark_pattern(plane, slot, iteration):
    """copy_benchmark.py:61-62: the payload byte of (plane, request slot,
    iteration)."""
    return 1 + (plane * 79 + slot * 7 + iteration) % 180


def fill_benchmark_buffers(k_cache, v_cache, host_k, host_v, batch, blocks, direction, iteration):
    """copy_benchmark.py:65-82: request slot i owns blocks [i*cap, (i+1)*cap)
    with cap = blocks + 2 on both sides; every block is first set to the
    guard byte, then the source side's payload blocks [i*cap + 1, i*cap +
    blocks + 1) to the pattern byte.  Returns the copy plan's regions."""
    cap = blocks + 2
    regions = []
    for slot in range(batch):
        begin = slot * cap
        for plane, (cache, host) in enumerate(((k_cache, host_k), (v_cache, host_v))):
            cache[begin:begin + cap] = DEVICE_GUARD
            host[begin:begin + cap] = HOST_GUARD
            value = benchmark_pattern(plane, slot, iteration)
            if direction == "D2H":
                cache[begin + 1:begin + blocks + 1] = value
            else:
                host[begin + 1:begin + blocks + 1] = value
        regions.append((begin + 1, begin + 1, blocks))
    return regions


def check_benchmark_buffers(k_cache, v_cache, host_k, host_v, batch, blocks, iteration):
    """copy_benchmark.py:85-98: after the copy both sides hold the pattern in
    the payload blocks and the guard blocks are untouched.  Raises
    AssertionError naming the first difference."""
    cap = blocks + 2
    for slot in range(batch):
        begin = slot * cap
        for plane, (cache, host) in enumerate(((k_cache, host_k), (v_cache, host_v))):
            value = benchmark_pattern(plane, slot, iteration)
            for side, arr, guard in (("GPU", cache, DEVICE_GUARD), ("HostKV", host, HOST_GUARD)):
                req = arr[begin:begin + cap]
                if not (req[1:-1] == value).all():
                    raise AssertionError(f"copy payload mismatch ({side}, slot {slot}, plane {plane})")
                if not ((req[0] == guard).all() and (req[-1] == guard).all()):
                    raise AssertionError(f"{side} guard overwritten (slot {slot}, plane {plane})")
