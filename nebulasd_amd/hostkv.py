"""HostKV block-range copies -- drop-ins for NebulaSD's HostKV DMA backend and
swiftLLM's ``swap_blocks``.

Reference: nebulasd/src/nebulasd/kv/transfer.py:15-46 (CopyRegion, CopyPlan,
HostCompletedFence), nebulasd/src/nebulasd/kv/cuda_transfer.py:31-133
(CudaCopyBackend: own stream, per-region cudaMemcpyAsync of the K and V
planes, start/done events), nebulasd/src/nebulasd/kv/arena.py:123-220 (the
host arena layout: K plane at offset 0, V plane at ``plane_bytes``, each
``total_blocks * block_bytes``) and swiftLLM/csrc/src/block_swapping.cpp:22-85.

A HostKV block is the byte image of one device cache block; copies are
bit-exact.  The native library (``nsd_copy_block_ranges``,
``nsd_swap_blocks``) validates every range before enqueuing anything and
merges regions that continue each other into one run.  Two engines:

* ``"dma"`` -- one ``hipMemcpyAsync`` per run on the system DMA engines (no
  compute unit is taken from kernels the copy overlaps with; plan order is
  kept, so a later region wins where destinations overlap).
* ``"kernel"`` -- one gfx950 copy launch over every run, reading or writing
  the pinned host planes directly; one launch however scattered the blocks.
  Needs pinned host memory, 16-byte alignment and disjoint destinations.

The arena here is process-local pinned memory (``hipHostMalloc`` through
torch's pinned allocator).  The reference's arena is a POSIX shared-memory
segment registered with ``cudaHostRegister`` so several processes can map
it; that storage layer is outside this library, which takes any pinned
buffer laid out as above.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

ENGINES = {"dma": _lib.COPY_ENGINE_DMA, "kernel": _lib.COPY_ENGINE_KERNEL}
DIRECTIONS = {"D2H": _lib.COPY_D2H, "H2D": _lib.COPY_H2D}


def _engine(engine: str) -> int:
    try:
        return ENGINES[engine]
    except KeyError:
        raise ValueError(f"unknown copy engine {engine!r} (expected one of {sorted(ENGINES)})") from None


@dataclass(frozen=True)
class HostKVDescriptor:
    """arena.py:123-157: K plane at 0, V plane right after it."""
    block_bytes: int
    total_blocks: int
    dtype: str
    kv_block_shape: tuple

    @property
    def plane_bytes(self) -> int:
        return self.total_blocks * self.block_bytes

    @property
    def k_plane_offset(self) -> int:
        return 0

    @property
    def v_plane_offset(self) -> int:
        return self.plane_bytes

    @property
    def total_bytes(self) -> int:
        return 2 * self.plane_bytes


@dataclass(frozen=True)
class HostKVExtent:
    """A request's span of arena blocks (arena.py:36-75, reduced to its offset
    and capacity)."""
    offset_blocks: int
    capacity_blocks: int

    def __post_init__(self) -> None:
        if self.offset_blocks < 0 or self.capacity_blocks <= 0:
            raise ValueError("extent needs a non-negative offset and a positive capacity")


class HostKVArena:
    """Pinned host memory holding the K plane then the V plane, each
    ``total_blocks`` blocks of ``block_bytes``."""

    def __init__(self, descriptor: HostKVDescriptor, storage: torch.Tensor) -> None:
        if storage.dtype != torch.uint8 or storage.numel() < descriptor.total_bytes or storage.is_cuda:
            raise ValueError("arena storage must be a host uint8 tensor of total_bytes")
        self.descriptor = descriptor
        self._storage = storage

    @classmethod
    def create(cls, *, total_blocks: int, block_bytes: int, dtype: str = "torch.float16",
               kv_block_shape: tuple = ()) -> "HostKVArena":
        if total_blocks <= 0 or block_bytes <= 0:
            raise ValueError("total_blocks and block_bytes must be positive")
        desc = HostKVDescriptor(int(block_bytes), int(total_blocks), dtype, tuple(kv_block_shape))
        return cls(desc, torch.empty(desc.total_bytes, dtype=torch.uint8, pin_memory=True))

    def address(self) -> int:
        return self._storage.data_ptr()

    @property
    def k(self) -> torch.Tensor:
        """K plane as uint8 [total_blocks, block_bytes] (a view)."""
        d = self.descriptor
        return self._storage[:d.plane_bytes].view(d.total_blocks, d.block_bytes)

    @property
    def v(self) -> torch.Tensor:
        d = self.descriptor
        return self._storage[d.plane_bytes:d.total_bytes].view(d.total_blocks, d.block_bytes)

    def make_extent(self, *, offset_blocks: int, capacity_blocks: int) -> HostKVExtent:
        extent = HostKVExtent(offset_blocks, capacity_blocks)
        self._validate_extent(extent)
        return extent

    def _validate_extent(self, extent: HostKVExtent) -> None:
        if extent.offset_blocks + extent.capacity_blocks > self.descriptor.total_blocks:
            raise ValueError("HostKV extent exceeds the arena")


@dataclass(frozen=True)
class CopyRegion:
    """transfer.py:15-26."""
    extent: HostKVExtent
    gpu_begin_block: int
    host_begin_block: int
    block_count: int

    def __post_init__(self) -> None:
        if min(self.gpu_begin_block, self.host_begin_block, self.block_count) < 0:
            raise ValueError("negative copy range")
        if self.host_begin_block + self.block_count > self.extent.capacity_blocks:
            raise ValueError("copy exceeds HostKV extent")


@dataclass(frozen=True)
class HostCompletedFence:
    """transfer.py:29-31: the producer synchronised this dependency already."""


@dataclass(frozen=True)
class CopyPlan:
    """transfer.py:34-45."""
    direction: str
    regions: tuple
    dependencies: tuple = ()
    round_ids: tuple = ()

    def __post_init__(self) -> None:
        if self.direction not in ("D2H", "H2D") or not self.regions:
            raise ValueError("copy plan requires a direction and non-empty batch")
        if self.round_ids and len(self.round_ids) != len(self.regions):
            raise ValueError("copy rounds must match regions")


class CopyTicket:
    """cuda_transfer.py:16-28: start/done events around one launch."""

    def __init__(self, start: torch.cuda.Event, done: torch.cuda.Event) -> None:
        self.start, self.done = start, done

    def query(self) -> bool:
        return bool(self.done.query())

    def synchronize(self) -> None:
        self.done.synchronize()

    def duration_ms(self) -> float:
        return float(self.start.elapsed_time(self.done))


def _host_i64(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64))


def _check_caches(k_cache: torch.Tensor, v_cache: torch.Tensor) -> int:
    if (not k_cache.is_cuda or not v_cache.is_cuda or k_cache.device != v_cache.device
            or k_cache.dtype != v_cache.dtype or k_cache.shape != v_cache.shape
            or not k_cache.is_contiguous() or not v_cache.is_contiguous()):
        raise ValueError("copy backend requires matching contiguous CUDA KV caches")
    return k_cache[0].numel() * k_cache.element_size()


def copy_block_ranges(k_cache: torch.Tensor, v_cache: torch.Tensor, host_k: int, host_v: int,
                      host_blocks: int, gpu_begin, host_begin, block_count, direction: str,
                      engine: str = "dma", stream: int | None = None) -> None:
    """One plan's copies on ``stream`` (default: the current stream of the
    caches' device).  ``host_k``/``host_v`` are the host planes' addresses,
    ``host_begin`` absolute block indices into them."""
    block_bytes = _check_caches(k_cache, v_cache)
    if direction not in DIRECTIONS:
        raise ValueError("copy plan requires a direction and non-empty batch")
    g, h, c = _host_i64(gpu_begin), _host_i64(host_begin), _host_i64(block_count)
    if not (g.shape == h.shape == c.shape) or g.ndim != 1:
        raise ValueError("region arrays must be 1-D and of one length")
    if stream is None:
        stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    _lib.call("nsd_copy_block_ranges", k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], host_k, host_v,
              int(host_blocks), block_bytes, g.ctypes.data, h.ctypes.data, c.ctypes.data, len(g),
              DIRECTIONS[direction], _engine(engine), stream)


class HostKVCopyBackend:
    """cuda_transfer.py:31-133: copies plans between ``arena`` and the device
    caches on a stream of its own (default priority); ``launch`` returns a
    ticket whose events bracket the plan's copies."""

    def __init__(self, *, arena: HostKVArena, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 engine: str = "dma") -> None:
        block_bytes = _check_caches(k_cache, v_cache)
        if arena.descriptor.block_bytes != block_bytes:
            raise ValueError("HostKV block byte size does not match GPU layout")
        if arena.descriptor.kv_block_shape and arena.descriptor.kv_block_shape != tuple(k_cache.shape[1:]):
            raise ValueError("HostKV dtype/block shape does not match GPU layout")
        _engine(engine)
        self.arena, self.k_cache, self.v_cache, self.engine = arena, k_cache, v_cache, engine
        self._device = k_cache.device
        self._stream = None
        self._closed = False

    def fork(self) -> "HostKVCopyBackend":
        """Another stream and its own events over the same caches and arena."""
        return type(self)(arena=self.arena, k_cache=self.k_cache, v_cache=self.v_cache, engine=self.engine)

    def initialize(self) -> None:
        if self._closed:
            raise RuntimeError("copy backend is closed")
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self._device)

    @property
    def stream(self) -> torch.cuda.Stream:
        self.initialize()
        return self._stream

    def launch(self, plan: CopyPlan) -> CopyTicket:
        self.initialize()
        d = self.arena.descriptor
        gpu, host, count = [], [], []
        for region in plan.regions:
            self.arena._validate_extent(region.extent)
            if region.gpu_begin_block + region.block_count > self.k_cache.shape[0]:
                raise ValueError("copy exceeds GPU KV cache")
            gpu.append(region.gpu_begin_block)
            host.append(region.extent.offset_blocks + region.host_begin_block)
            count.append(region.block_count)
        with torch.cuda.stream(self._stream):
            for dependency in plan.dependencies:
                if not isinstance(dependency, HostCompletedFence):
                    self._stream.wait_event(dependency)
            start = torch.cuda.Event(enable_timing=True)
            done = torch.cuda.Event(enable_timing=True, blocking=True)
            start.record(self._stream)
            base = self.arena.address()
            copy_block_ranges(self.k_cache, self.v_cache, base + d.k_plane_offset, base + d.v_plane_offset,
                              d.total_blocks, gpu, host, count, plan.direction, self.engine,
                              self._stream.cuda_stream)
            done.record(self._stream)
        return CopyTicket(start, done)

    def close(self) -> None:
        """Waits for the stream's copies; the arena must outlive them."""
        if self._closed:
            return
        self._closed = True
        if self._stream is not None:
            self._stream.synchronize()
        self._stream = None


def swap_blocks(source_block_ids, target_block_ids, is_swap_in: bool, k_cache: torch.Tensor,
                v_cache: torch.Tensor, k_swap: torch.Tensor, v_swap: torch.Tensor,
                engine: str = "dma") -> None:
    """block_swapping.cpp:22-85 on the current stream: ``source_block_ids[i]``
    goes to ``target_block_ids[i]``, swap space -> cache when ``is_swap_in``
    else cache -> swap space, K and V.  ``k_swap``/``v_swap`` are host
    tensors with the caches' block layout (pinned for the kernel engine)."""
    block_bytes = _check_caches(k_cache, v_cache)
    if (k_swap.is_cuda or v_swap.is_cuda or k_swap.shape[1:] != k_cache.shape[1:] or k_swap.shape != v_swap.shape
            or k_swap.dtype != k_cache.dtype or v_swap.dtype != k_cache.dtype
            or not k_swap.is_contiguous() or not v_swap.is_contiguous()):
        raise ValueError("swap space must be contiguous host tensors with the caches' block layout")
    s, t = _host_i64(source_block_ids), _host_i64(target_block_ids)
    if s.shape != t.shape or s.ndim != 1:
        raise ValueError("source and target block ids must be 1-D and of one length")
    _lib.call("nsd_swap_blocks", s.ctypes.data, t.ctypes.data, len(s), int(bool(is_swap_in)), k_cache.data_ptr(),
              v_cache.data_ptr(), k_cache.shape[0], k_swap.data_ptr(), v_swap.data_ptr(), k_swap.shape[0],
              block_bytes, _engine(engine), torch.cuda.current_stream(k_cache.device).cuda_stream)
