"""Pins for the HostKV copy oracle (CPU only): the reference's own copy
benchmark fixture and byte check, a block-by-block loop, hand-built swap
runs, round trips, planted mistakes the checks must reject; and the C ABI's
range checks, which return before any HIP call."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from nebulasd_amd import _lib
from nebulasd_amd.hostkv import CopyPlan, CopyRegion, HostKVExtent


def _planes(rng, blocks, block_bytes):
    return [rng.integers(0, 256, (blocks, block_bytes), dtype=np.uint8) for _ in range(4)]


@pytest.mark.parametrize("direction", ["D2H", "H2D"])
def test_reference_benchmark_fixture(direction):
    """copy_benchmark.py:61-98: guards each side of every request, payload
    pattern per (plane, slot, iteration); three iterations on one buffer set
    (a copy that left stale bytes would fail the next iteration's check)."""
    batch, blocks, bb = 5, 3, 64
    k, v, hk, hv = (np.zeros((batch * (blocks + 2), bb), np.uint8) for _ in range(4))
    for it in range(3):
        regions = oracle.fill_benchmark_buffers(k, v, hk, hv, batch, blocks, direction, it)
        oracle.copy_block_ranges(k, v, hk, hv, regions, direction)
        oracle.check_benchmark_buffers(k, v, hk, hv, batch, blocks, it)


def _planted(kind):
    """The oracle with one mistake planted."""
    def copy(k, v, hk, hv, regions, direction):
        for g, h, c in regions:
            if kind == "host_off_by_one":
                h += 1
            pairs = ((k, hk), (v, hv)) if kind != "kv_swapped" else ((k, hv), (v, hk))
            for cache, host in pairs:
                if direction == "D2H":
                    host[h:h + c] = cache[g:g + c]
                else:
                    cache[g:g + c] = host[h:h + c]
    return copy


@pytest.mark.parametrize("kind", ["host_off_by_one", "kv_swapped"])
@pytest.mark.parametrize("direction", ["D2H", "H2D"])
def test_benchmark_check_rejects_planted_mistakes(kind, direction):
    batch, blocks, bb = 3, 4, 32
    k, v, hk, hv = (np.zeros((batch * (blocks + 2), bb), np.uint8) for _ in range(4))
    regions = oracle.fill_benchmark_buffers(k, v, hk, hv, batch, blocks, direction, 0)
    _planted(kind)(k, v, hk, hv, regions, direction)
    with pytest.raises(AssertionError):
        oracle.check_benchmark_buffers(k, v, hk, hv, batch, blocks, 0)


def _block_loop(k, v, hk, hv, regions, direction):
    """One block at a time, regions in order."""
    for g, h, c in regions:
        for j in range(c):
            for cache, host in ((k, hk), (v, hv)):
                if direction == "D2H":
                    host[h + j] = cache[g + j]
                else:
                    cache[g + j] = host[h + j]


def random_plan(rng, gpu_blocks, host_blocks, n, overlap=True):
    regions = []
    for _ in range(n):
        c = int(rng.integers(0, 6))
        g = int(rng.integers(0, gpu_blocks - c + 1))
        h = int(rng.integers(0, host_blocks - c + 1))
        regions.append((g, h, c))
        if rng.random() < 0.3:  # a region that continues this one on both sides (merges into one run)
            c2 = int(rng.integers(1, 4))
            if g + c + c2 <= gpu_blocks and h + c + c2 <= host_blocks:
                regions.append((g + c, h + c, c2))
    if not overlap:
        return regions
    if regions:  # an overlapping destination: the later copy must win
        g, h, c = regions[0]
        regions.append((g, (h + 1) % max(1, host_blocks - c), c))
    return regions


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("direction", ["D2H", "H2D"])
def test_copy_matches_block_loop(seed, direction):
    rng = np.random.default_rng(seed)
    a = _planes(rng, 40, 24)
    b = [x.copy() for x in a]
    # host planes are a[2], a[3] with 40 blocks too
    regions = random_plan(rng, 40, 40, 12)
    oracle.copy_block_ranges(*a, regions, direction)
    _block_loop(*b, regions, direction)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_copy_range_errors():
    k, v, hk, hv = (np.zeros((8, 16), np.uint8) for _ in range(4))
    for regions, msg in (([(-1, 0, 1)], "negative copy range"), ([(6, 0, 3)], "exceeds GPU KV cache"),
                         ([(0, 7, 2)], "exceeds HostKV plane")):
        with pytest.raises(ValueError, match=msg):
            oracle.copy_block_ranges(k, v, hk, hv, regions, "H2D")
    with pytest.raises(ValueError):
        oracle.copy_block_ranges(k, v, hk, hv, [(0, 0, 1)], "D2D")


def test_swap_runs_known_answers():
    # consecutive on both sides -> one run; a break on either side splits
    assert oracle.swap_runs([3, 4, 5, 9, 10], [2, 3, 4, 7, 8]) == [(3, 2, 3), (9, 7, 2)]
    assert oracle.swap_runs([1, 2, 3], [5, 6, 8]) == [(1, 5, 2), (3, 8, 1)]
    assert oracle.swap_runs([1, 2, 4], [5, 6, 7]) == [(1, 5, 2), (4, 7, 1)]
    assert oracle.swap_runs([7, 7], [1, 2]) == [(7, 1, 1), (7, 2, 1)]
    assert oracle.swap_runs([], []) == []
    assert oracle.swap_runs([4, 3], [1, 0]) == [(4, 1, 1), (3, 0, 1)]


def test_swap_runs_rejects_planted_mistake():
    """Merging on the source side alone would join (1, 5) and (2, 7)."""
    def src_only(s, t):
        runs, i = [], 0
        while i < len(s):
            j = i + 1
            while j < len(s) and s[j] == s[j - 1] + 1:
                j += 1
            runs.append((s[i], t[i], j - i))
            i = j
        return runs
    s, t = [1, 2, 3], [5, 7, 8]
    assert src_only(s, t) != oracle.swap_runs(s, t)


@pytest.mark.parametrize("is_swap_in", [False, True])
def test_swap_blocks_matches_block_loop_and_round_trips(is_swap_in):
    rng = np.random.default_rng(11)
    k, v, ks, vs = _planes(rng, 50, 40)
    src = rng.permutation(50)[:20]
    src[5:9] = np.arange(30, 34)  # a run
    dst = rng.permutation(50)[:20]
    dst[5:9] = np.arange(10, 14)
    want = [x.copy() for x in (k, v, ks, vs)]
    for s, t in zip(src, dst):
        for cache, swap in ((want[0], want[2]), (want[1], want[3])):
            if is_swap_in:
                cache[t] = swap[s]
            else:
                swap[t] = cache[s]
    got = [x.copy() for x in (k, v, ks, vs)]
    oracle.swap_blocks(src, dst, is_swap_in, *got)
    for x, y in zip(got, want):
        np.testing.assert_array_equal(x, y)


def test_swap_out_then_in_restores_cache():
    rng = np.random.default_rng(12)
    k, v, ks, vs = _planes(rng, 30, 16)
    k0, v0 = k.copy(), v.copy()
    gpu_ids = rng.permutation(30)[:12]
    host_ids = rng.permutation(30)[:12]
    oracle.swap_blocks(gpu_ids, host_ids, False, k, v, ks, vs)
    k[gpu_ids] = 0
    v[gpu_ids] = 0
    oracle.swap_blocks(host_ids, gpu_ids, True, k, v, ks, vs)
    np.testing.assert_array_equal(k, k0)
    np.testing.assert_array_equal(v, v0)


def test_plan_types_validate_like_the_reference():
    ext = HostKVExtent(offset_blocks=4, capacity_blocks=6)
    with pytest.raises(ValueError, match="negative copy range"):
        CopyRegion(ext, -1, 0, 1)
    with pytest.raises(ValueError, match="copy exceeds HostKV extent"):
        CopyRegion(ext, 0, 3, 4)
    with pytest.raises(ValueError, match="non-empty batch"):
        CopyPlan("H2D", ())
    with pytest.raises(ValueError, match="non-empty batch"):
        CopyPlan("D2D", (CopyRegion(ext, 0, 0, 1),))
    with pytest.raises(ValueError, match="copy rounds must match"):
        CopyPlan("D2H", (CopyRegion(ext, 0, 0, 1),), round_ids=(1, 2))


def _call(lib, g, h, c, *, gpu_blocks=10, host_blocks=10, direction=_lib.COPY_H2D, engine=_lib.COPY_ENGINE_DMA,
          block_bytes=64, planes=(0x10000, 0x20000, 0x30000, 0x40000)):
    arr = [np.asarray(x, np.int64) for x in (g, h, c)]
    return lib.nsd_copy_block_ranges(planes[0], planes[1], gpu_blocks, planes[2], planes[3], host_blocks,
                                     block_bytes, *(a.ctypes.data for a in arr), len(arr[0]), direction, engine,
                                     None)


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from nebulasd_amd.build import build

        build()
    return _lib.load()


def test_capi_range_checks_without_gpu(lib):
    """Every range is checked before anything is enqueued (the planes here
    are never dereferenced: each call fails or has nothing to copy)."""
    cases = [
        (([-1], [0], [1]), {}, "negative copy range"),
        (([8], [0], [3]), {}, "copy exceeds GPU KV cache"),
        (([0], [9], [2]), {}, "copy exceeds HostKV plane"),
        (([0, 8], [0, 0], [1, 3]), {}, "region 1"),
        (([0], [0], [1]), {"engine": 7}, "unknown copy engine"),
        (([0], [0], [1]), {"direction": 5}, "direction"),
        (([0], [0], [1]), {"planes": (0x10000, 0x10020, 0x30000, 0x40000)}, "K and V caches overlap"),
        (([0], [0], [1]), {"planes": (0x10000, 0x20000, 0x30000, 0x30100)}, "K and V host planes overlap"),
        (([0], [0], [1]), {"block_bytes": 0}, "block geometry"),
    ]
    for (g, h, c), kw, msg in cases:
        rc = _call(lib, g, h, c, **kw)
        assert rc == _lib.NSD_OK + 1 and msg in _lib.last_error(), (msg, rc, _lib.last_error())
    # nothing to copy: no HIP call, success
    assert _call(lib, [], [], []) == 0
    assert _call(lib, [3, 9], [2, 10], [0, 0]) == 0
    ids = np.array([0, 12], np.int64)
    rc = lib.nsd_swap_blocks(ids.ctypes.data, ids.ctypes.data, 2, 1, 0x10000, 0x20000, 10, 0x30000, 0x40000, 20,
                             64, 0, None)
    assert rc == 1 and "copy exceeds GPU KV cache" in _lib.last_error()
    assert lib.nsd_swap_blocks(None, None, 0, 1, None, None, 0, None, None, 0, 64, 0, None) == 0
    assert isinstance(lib.nsd_swap_blocks, ctypes._CFuncPtr)
