"""GPU parity of the HostKV block-range copies and swap_blocks against the
numpy oracle: bit-exact, both engines, both directions.

Every case prints its name first (pytest -v) so a failing GPU step is named.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from nebulasd_amd import _lib
from nebulasd_amd.hostkv import (CopyPlan, CopyRegion, HostCompletedFence, HostKVArena, HostKVCopyBackend,
                                 copy_block_ranges, swap_blocks)
from test_oracle_hostkv import random_plan

pytestmark = pytest.mark.gpu

ENGINES = ["dma", "kernel"]


def _cache(gpu, blocks, shape, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    k = torch.randint(-30000, 30000, (blocks, *shape), generator=g, dtype=torch.int16).view(torch.float16)
    v = torch.randint(-30000, 30000, (blocks, *shape), generator=g, dtype=torch.int16).view(torch.float16)
    return k.to(gpu), v.to(gpu)


def _bytes(t):
    return t.detach().cpu().contiguous().view(torch.uint8).reshape(t.shape[0], -1).numpy().copy()


def _arena_random(arena, seed):
    rng = np.random.default_rng(seed)
    arena.k.copy_(torch.from_numpy(rng.integers(0, 256, tuple(arena.k.shape), dtype=np.uint8)))
    arena.v.copy_(torch.from_numpy(rng.integers(0, 256, tuple(arena.v.shape), dtype=np.uint8)))


@pytest.mark.parametrize("engine", ENGINES)
def test_reference_benchmark_fixture(gpu, engine):
    """copy_benchmark.py:61-98 on the device: guard blocks each side of every
    request, payload pattern per (plane, slot, iteration), D2H then H2D,
    three iterations on the same buffers (stale bytes in any cache level
    would fail a later iteration's check)."""
    shape = (4, 8, 16, 128)  # [L, Hkv, 16, d] fp16: 128 KB blocks
    batch, blocks = 4, 5
    cap = blocks + 2
    k, v = _cache(gpu, batch * cap, shape, 0)
    bb = k[0].numel() * 2
    arena = HostKVArena.create(total_blocks=batch * cap, block_bytes=bb, kv_block_shape=shape)
    backend = HostKVCopyBackend(arena=arena, k_cache=k, v_cache=v, engine=engine)
    extents = [arena.make_extent(offset_blocks=i * cap, capacity_blocks=cap) for i in range(batch)]
    for direction in ("D2H", "H2D"):
        plan = CopyPlan(direction, tuple(CopyRegion(e, i * cap + 1, 1, blocks) for i, e in enumerate(extents)))
        for it in range(3):
            kb, vb = _bytes(k), _bytes(v)
            hk, hv = arena.k.numpy(), arena.v.numpy()
            oracle.fill_benchmark_buffers(kb, vb, hk, hv, batch, blocks, direction, it)
            k.view(torch.uint8).view(kb.shape).copy_(torch.from_numpy(kb))
            v.view(torch.uint8).view(vb.shape).copy_(torch.from_numpy(vb))
            torch.cuda.synchronize()
            ticket = backend.launch(plan)
            ticket.synchronize()
            assert ticket.query() and ticket.duration_ms() >= 0
            oracle.check_benchmark_buffers(_bytes(k), _bytes(v), arena.k.numpy(), arena.v.numpy(), batch, blocks, it)
        print(f"benchmark fixture {engine} {direction}: ok", flush=True)
    backend.close()


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("direction", ["D2H", "H2D"])
@pytest.mark.parametrize("shape", [(3, 2, 16, 40), (36, 8, 16, 128)], ids=["7680B", "8b"])
def test_random_plans_match_oracle(gpu, engine, direction, shape):
    """Random regions (adjacent ones merge into runs, zero counts, >64 runs so
    the kernel engine needs several launches); block sizes that are and are
    not a multiple of the 64 KB chunk."""
    gblocks, hblocks = (300, 260) if shape[0] == 3 else (24, 20)
    rng = np.random.default_rng(100 * ENGINES.index(engine) + 10 * (direction == "D2H") + shape[0])
    k, v = _cache(gpu, gblocks, shape, 1)
    arena = HostKVArena.create(total_blocks=hblocks, block_bytes=k[0].numel() * 2)
    _arena_random(arena, 2)
    n = 90 if shape[0] == 3 else 6
    regions = random_plan(rng, gblocks, hblocks, n, overlap=False)
    # keep destinations disjoint (the kernel engine requires it)
    seen, plan = set(), []
    for g, h, c in regions:
        dst = range(h, h + c) if direction == "D2H" else range(g, g + c)
        if seen.isdisjoint(dst):
            seen.update(dst)
            plan.append((g, h, c))
    want = [_bytes(k), _bytes(v), arena.k.numpy().copy(), arena.v.numpy().copy()]
    oracle.copy_block_ranges(*want, plan, direction)
    g_, h_, c_ = zip(*plan)
    copy_block_ranges(k, v, arena.address(), arena.address() + arena.descriptor.plane_bytes, hblocks,
                      g_, h_, c_, direction, engine)
    torch.cuda.synchronize()
    got = [_bytes(k), _bytes(v), arena.k.numpy(), arena.v.numpy()]
    for name, x, y in zip("k v host_k host_v".split(), got, want):
        assert np.array_equal(x, y), f"{name} differs"
    print(f"random plan {engine} {direction} {shape}: {len(plan)} regions ok", flush=True)


def test_overlapping_destinations(gpu):
    """The DMA engine keeps plan order (the later region wins, as with the
    reference's stream of copies); the kernel engine refuses the plan."""
    shape = (2, 2, 16, 64)
    k, v = _cache(gpu, 16, shape, 3)
    arena = HostKVArena.create(total_blocks=16, block_bytes=k[0].numel() * 2)
    _arena_random(arena, 4)
    plan = [(2, 0, 4), (4, 8, 3), (0, 12, 2)]  # device blocks 4, 5 written twice
    want = [_bytes(k), _bytes(v), arena.k.numpy().copy(), arena.v.numpy().copy()]
    oracle.copy_block_ranges(*want, plan, "H2D")
    args = (k, v, arena.address(), arena.address() + arena.descriptor.plane_bytes, 16, *zip(*plan), "H2D")
    with pytest.raises(_lib.NativeLibraryError, match="disjoint destinations"):
        copy_block_ranges(*args, "kernel")
    copy_block_ranges(*args, "dma")
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(k), want[0]) and np.array_equal(_bytes(v), want[1])


@pytest.mark.parametrize("engine", ENGINES)
@pytest.mark.parametrize("is_swap_in", [False, True])
def test_swap_blocks_matches_oracle(gpu, engine, is_swap_in):
    shape = (28, 8, 16, 128)  # the 0.6B draft's 917,504-byte blocks
    k, v = _cache(gpu, 40, shape, 5)
    ks = torch.empty((48, *shape), dtype=torch.float16, pin_memory=True)
    vs = torch.empty_like(ks, pin_memory=True)
    rng = np.random.default_rng(6)
    ks.view(torch.int16).copy_(torch.from_numpy(rng.integers(-30000, 30000, ks.shape, dtype=np.int16)))
    vs.view(torch.int16).copy_(torch.from_numpy(rng.integers(-30000, 30000, vs.shape, dtype=np.int16)))
    n = 24
    n_src, n_dst = (48, 40) if is_swap_in else (40, 48)
    src = rng.permutation(n_src)[:n]
    dst = rng.permutation(np.setdiff1d(np.arange(n_dst), np.arange(30, 35)))[:n]  # targets distinct
    src[3:8], dst[3:8] = np.arange(20, 25), np.arange(30, 35)  # one run of five
    want = [_bytes(k), _bytes(v), _bytes(ks), _bytes(vs)]
    runs = oracle.swap_blocks(src, dst, is_swap_in, *want)
    swap_blocks(src.tolist(), dst.tolist(), is_swap_in, k, v, ks, vs, engine=engine)
    torch.cuda.synchronize()
    for name, x, y in zip("k v k_swap v_swap".split(), (_bytes(k), _bytes(v), _bytes(ks), _bytes(vs)), want):
        assert np.array_equal(x, y), f"{name} differs"
    print(f"swap_blocks {engine} in={is_swap_in}: {len(runs)} runs ok", flush=True)


@pytest.mark.parametrize("engine", ENGINES)
def test_swap_out_then_in_round_trip(gpu, engine):
    shape = (4, 8, 16, 128)
    k, v = _cache(gpu, 32, shape, 7)
    k0, v0 = k.clone(), v.clone()
    ks = torch.zeros((32, *shape), dtype=torch.float16, pin_memory=True)
    vs = torch.zeros_like(ks, pin_memory=True)
    rng = np.random.default_rng(8)
    gpu_ids, host_ids = rng.permutation(32)[:20].tolist(), rng.permutation(32)[:20].tolist()
    swap_blocks(gpu_ids, host_ids, False, k, v, ks, vs, engine=engine)
    k[gpu_ids] = 0
    v[gpu_ids] = 0
    swap_blocks(host_ids, gpu_ids, True, k, v, ks, vs, engine=engine)
    torch.cuda.synchronize()
    assert torch.equal(k.view(torch.int16), k0.view(torch.int16))
    assert torch.equal(v.view(torch.int16), v0.view(torch.int16))


def test_pageable_swap_space(gpu):
    """swiftLLM's swap space is an ordinary (pageable) CPU tensor
    (model.py:176-177): the DMA engine copies it; the kernel engine, which
    reads host memory from the device, refuses it."""
    shape = (2, 2, 16, 64)
    k, v = _cache(gpu, 8, shape, 9)
    ks = torch.zeros((8, *shape), dtype=torch.float16)
    vs = torch.zeros_like(ks)
    with pytest.raises(_lib.NativeLibraryError, match="pinned"):
        swap_blocks([1, 2], [3, 4], False, k, v, ks, vs, engine="kernel")
    swap_blocks([1, 2], [3, 4], False, k, v, ks, vs, engine="dma")
    torch.cuda.synchronize()
    assert torch.equal(ks[3:5].view(torch.int16), k[1:3].cpu().view(torch.int16))
    assert torch.equal(vs[3:5].view(torch.int16), v[1:3].cpu().view(torch.int16))


@pytest.mark.parametrize("engine", ENGINES)
def test_backend_waits_for_dependencies_and_full_size_round_trip(gpu, engine):
    """Qwen3-8B blocks (1,179,648 bytes): a producer kernel on another stream
    writes the cache, the plan waits on its event (cuda_transfer.py:90-92),
    D2H to the arena, H2D into other device blocks; the copies equal the
    source (a size-independent round-trip property)."""
    shape = (36, 8, 16, 128)
    k, v = _cache(gpu, 48, shape, 10)
    arena = HostKVArena.create(total_blocks=24, block_bytes=k[0].numel() * 2, kv_block_shape=shape)
    backend = HostKVCopyBackend(arena=arena, k_cache=k, v_cache=v, engine=engine)
    ext = arena.make_extent(offset_blocks=0, capacity_blocks=24)
    producer = torch.cuda.Stream()
    with torch.cuda.stream(producer):
        k[:20].add_(1)
        v[:20].mul_(2)
        ready = torch.cuda.Event()
        ready.record(producer)
    out = backend.launch(CopyPlan("D2H", (CopyRegion(ext, 0, 0, 12), CopyRegion(ext, 12, 12, 8)),
                                  dependencies=(ready, HostCompletedFence())))
    back = backend.fork()
    with torch.cuda.stream(back.stream):
        back.stream.wait_event(out.done)
    inn = back.launch(CopyPlan("H2D", (CopyRegion(ext, 24, 0, 20),)))
    inn.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(k[24:44].view(torch.int16), k[:20].view(torch.int16))
    assert torch.equal(v[24:44].view(torch.int16), v[:20].view(torch.int16))
    gb = 2 * 20 * arena.descriptor.block_bytes / 1e9
    print(f"round trip {engine}: D2H {gb / out.duration_ms() * 1e3:.1f} GB/s, "
          f"H2D {gb / inn.duration_ms() * 1e3:.1f} GB/s", flush=True)
    with pytest.raises(ValueError, match="copy exceeds GPU KV cache"):
        backend.launch(CopyPlan("H2D", (CopyRegion(ext, 40, 0, 9),)))
    backend.close()
    back.close()
    with pytest.raises(RuntimeError, match="closed"):
        backend.launch(CopyPlan("H2D", (CopyRegion(ext, 0, 0, 1),)))
