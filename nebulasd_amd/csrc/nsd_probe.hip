// HBM ceiling probes for the attention path (read-only, no arithmetic on the data).
//
// nsd_probe_stream_read[_unroll]: every byte of a contiguous buffer is read
//   once with 16-byte loads; the sequential-read rate of the device, over
//   grid sizes and loads in flight per thread.
// nsd_probe_tile_gather: the K and V tiles (one block, layer and kv head:
//   16 tokens x 128 dims fp16, 4 KB each) that a tile list names are split
//   across workgroups in contiguous ranges and streamed into an LDS ring by
//   global_load_lds_dwordx4, four waves per workgroup, two workgroups per
//   CU, as the attention kernel streams them, and only touched in LDS: the
//   rate at which the attention's K/V reads could complete for the same
//   tiles with its arithmetic, merges and imbalance taken away.
// nsd_probe_gather_pieces: the same tiles cut into pieces, one workgroup
//   per piece dispatched by the hardware as CU slots free up, with the ring
//   depth and the workgroups per CU as parameters.
// nsd_probe_gather_vgpr: the same pieces loaded into registers instead of
//   LDS, more waves per SIMD.
// nsd_probe_empty: a kernel that does nothing (the fixed cost of a launch).
//
// The kernels clamp every index and offset they read from device memory into
// the buffers' bounds, so any tile list or split reads in bounds.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nsd_common.h"
#include "nsd_probe.h"
#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kStreamThreads = 256;
constexpr int64_t kStreamQuantum = (int64_t)kStreamThreads * 16 * 16;  // bytes: one chunk at the largest unroll

// Workgroup c reads chunks c, c + grid, ... of U x 4 KB (one 16-byte load per
// thread and unroll step, all U issued before any is used).
template <int U>
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                                     int64_t n_chunks, uint32_t* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const u32x4* p = src + c * (kStreamThreads * U) + threadIdx.x;
    u32x4 r[U];
#pragma unroll
    for (int j = 0; j < U; ++j) r[j] = __builtin_nontemporal_load(p + j * kStreamThreads);
#pragma unroll
    for (int j = 0; j < U; ++j) acc ^= r[j];
  }
  // never true for the probe's data in practice; keeps the loads live
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[0] = acc[0];
}

__global__ void empty_kernel() {}

constexpr int kGatherThreads = 256;          // four waves
constexpr int kTileBytes = 16 * 128 * 2;     // one block's K (or V) of one head and layer
constexpr int kTileElems = kTileBytes / 2;
constexpr int kGatherRing = 8;               // items (K + V tile) in the LDS ring
constexpr int kGatherSlot = 2 * kTileBytes;
constexpr int kGatherMaxItems = 1536;        // tile offsets a workgroup holds in LDS
constexpr int kGatherLds = kGatherRing * kGatherSlot + kGatherMaxItems * 8;
static_assert(2 * kGatherLds <= 160 * 1024, "two workgroups per CU");

__device__ inline void dma16(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(lds_addr), "v"(src) : "memory", "m0");
}
template <int N>
__device__ inline void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}
// All but this wave's loads of the n most recent items done (two loads per item).
__device__ inline void wait_items(int n) {
  static_assert(kGatherRing == 8, "wait table");
  switch (n) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<2>(); break;
    case 2: wait_vm<4>(); break;
    case 3: wait_vm<6>(); break;
    case 4: wait_vm<8>(); break;
    case 5: wait_vm<10>(); break;
    default: wait_vm<12>(); break;
  }
}

__global__ __launch_bounds__(kGatherThreads) void tile_gather_kernel(
    const f16* __restrict__ k_cache, const f16* __restrict__ v_cache, int64_t cache_elems,
    const int64_t* __restrict__ tiles, int64_t n_tiles, const int64_t* __restrict__ wstart,
    uint32_t* sink) {
  extern __shared__ __align__(16) char smem[];
  int64_t* s_off = reinterpret_cast<int64_t*>(smem + kGatherRing * kGatherSlot);
  const int64_t w = blockIdx.x;
  int64_t s = wstart[w], e = wstart[w + 1];
  s = s < 0 ? 0 : (s > n_tiles ? n_tiles : s);
  e = e < s ? s : (e > n_tiles ? n_tiles : e);
  if (e - s > kGatherMaxItems) e = s + kGatherMaxItems;
  const int n = (int)(e - s);
  const int64_t last = cache_elems - kTileElems;
  for (int i = threadIdx.x; i < n; i += kGatherThreads) {
    int64_t off = tiles[s + i];
    s_off[i] = off < 0 ? 0 : (off > last ? last : off);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t lane_off = wave * 512 + lane * 8;  // rows 4w .. 4w+3 of the tile, 16 B a lane
  const uint32_t ring = (uint32_t)(uintptr_t)smem;
  int issued = 0;
  auto issue = [&]() {
    const int slot = issued % kGatherRing;
    const int64_t off = s_off[issued];
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)off);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)off >> 32));
    const int64_t base = (int64_t)(((uint64_t)hi << 32) | lo) + lane_off;
    dma16(ring + slot * kGatherSlot + wave * 1024, k_cache + base);
    dma16(ring + slot * kGatherSlot + kTileBytes + wave * 1024, v_cache + base);
    ++issued;
  };
  while (issued < n && issued < kGatherRing - 1) issue();
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int i = 0; i < n; ++i) {
    wait_items(issued - i - 1);  // item i landed (this wave's part) ...
    asm volatile("s_barrier" ::: "memory");  // ... and every wave's; slot of item i-1 is free
    if (issued < n) issue();
    const char* sl = smem + (i % kGatherRing) * kGatherSlot;
    acc ^= *reinterpret_cast<const u32x4*>(sl + threadIdx.x * 16);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[0] = acc[0];
}

// All but this wave's loads of the n most recent ring items done (two loads
// per item); n is clamped to [0, 15].
__device__ inline void wait_ring_items(int n) {
  switch (n <= 0 ? 0 : (n > 15 ? 15 : n)) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<2>(); break;
    case 2: wait_vm<4>(); break;
    case 3: wait_vm<6>(); break;
    case 4: wait_vm<8>(); break;
    case 5: wait_vm<10>(); break;
    case 6: wait_vm<12>(); break;
    case 7: wait_vm<14>(); break;
    case 8: wait_vm<16>(); break;
    case 9: wait_vm<18>(); break;
    case 10: wait_vm<20>(); break;
    case 11: wait_vm<22>(); break;
    case 12: wait_vm<24>(); break;
    case 13: wait_vm<26>(); break;
    case 14: wait_vm<28>(); break;
    default: wait_vm<30>(); break;
  }
}

constexpr int kPieceMaxTiles = 256;  // tiles one piece-workgroup streams (its LDS offset table)

// Loads piece blockIdx.x's tile offsets (clamped into the cache) into s_off;
// returns the piece's tile count (<= kPieceMaxTiles).
__device__ inline int load_piece_offsets(const int64_t* __restrict__ tiles, int64_t n_tiles,
                                         const int64_t* __restrict__ pstart, int64_t cache_elems,
                                         int64_t* s_off) {
  int64_t s = pstart[blockIdx.x], e = pstart[blockIdx.x + 1];
  s = s < 0 ? 0 : (s > n_tiles ? n_tiles : s);
  e = e < s ? s : (e > n_tiles ? n_tiles : e);
  if (e - s > kPieceMaxTiles) e = s + kPieceMaxTiles;
  const int n = (int)(e - s);
  const int64_t last = cache_elems - kTileElems;
  for (int i = threadIdx.x; i < n; i += kGatherThreads) {
    const int64_t off = tiles[s + i];
    s_off[i] = off < 0 ? 0 : (off > last ? last : off);
  }
  return n;
}

// One workgroup per piece (a contiguous range of the tile list), dispatched
// by the hardware as slots free up: the ring of RING items is filled by
// global_load_lds_dwordx4 as in tile_gather_kernel.  Occupancy follows from
// the LDS size (ring, offset table and an optional pad).
template <int RING>
__global__ __launch_bounds__(kGatherThreads) void gather_pieces_kernel(
    const f16* __restrict__ k_cache, const f16* __restrict__ v_cache, int64_t cache_elems,
    const int64_t* __restrict__ tiles, int64_t n_tiles, const int64_t* __restrict__ pstart,
    uint32_t* sink) {
  extern __shared__ __align__(16) char smem[];
  int64_t* s_off = reinterpret_cast<int64_t*>(smem + RING * kGatherSlot);
  const int n = load_piece_offsets(tiles, n_tiles, pstart, cache_elems, s_off);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t lane_off = wave * 512 + lane * 8;
  const uint32_t ring = (uint32_t)(uintptr_t)smem;
  int issued = 0;
  auto issue = [&]() {
    const int slot = issued % RING;
    const int64_t off = s_off[issued];
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)off);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)off >> 32));
    const int64_t base = (int64_t)(((uint64_t)hi << 32) | lo) + lane_off;
    dma16(ring + slot * kGatherSlot + wave * 1024, k_cache + base);
    dma16(ring + slot * kGatherSlot + kTileBytes + wave * 1024, v_cache + base);
    ++issued;
  };
  while (issued < n && issued < RING - 1) issue();
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int i = 0; i < n; ++i) {
    wait_ring_items(issued - i - 1);
    asm volatile("s_barrier" ::: "memory");
    if (issued < n) issue();
    const char* sl = smem + (i % RING) * kGatherSlot;
    acc ^= *reinterpret_cast<const u32x4*>(sl + threadIdx.x * 16);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[0] = acc[0];
}

// The same pieces read into registers: wave w of a workgroup loads tiles
// w, w + 4, ... of its piece, U tiles (K and V, 8 KB) per round with
// 16-byte loads, all issued before any is used; occupancy follows from the
// registers (no LDS ring).
template <int U>
__global__ __launch_bounds__(kGatherThreads) void gather_vgpr_kernel(
    const f16* __restrict__ k_cache, const f16* __restrict__ v_cache, int64_t cache_elems,
    const int64_t* __restrict__ tiles, int64_t n_tiles, const int64_t* __restrict__ pstart,
    uint32_t* sink) {
  __shared__ int64_t s_off[kPieceMaxTiles];
  const int n = load_piece_offsets(tiles, n_tiles, pstart, cache_elems, s_off);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int t0 = wave; t0 < n; t0 += 4 * U) {
    u32x4 r[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + 4 * u < n ? t0 + 4 * u : t0;
      const int64_t off = s_off[t];
      const u32x4* kp = reinterpret_cast<const u32x4*>(k_cache + off) + lane;
      const u32x4* vp = reinterpret_cast<const u32x4*>(v_cache + off) + lane;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r[u][j] = __builtin_nontemporal_load(kp + 64 * j);
        r[u][4 + j] = __builtin_nontemporal_load(vp + 64 * j);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc ^= r[u][j];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[0] = acc[0];
}

// Waves stream on their own (no barriers): wave w of a workgroup takes tiles
// w, w + 4, ... of its piece, R tiles per round with the next round's loads
// issued before the current round is used.  K is read into registers in the
// A-operand layout of v_mfma_f32_16x16x32_f16 (lane (i, g): token i, dims
// 32kk + 8g .. +7) when KMODE is 1, in 1 KB contiguous runs when 0; V goes
// into registers (VMODE 0) or by global_load_lds_dwordx4 into a slot of the
// wave's own LDS ring (VMODE 1).
template <int R, int KMODE, int VMODE>
__global__ __launch_bounds__(kGatherThreads) void gather_wave_kernel(
    const f16* __restrict__ k_cache, const f16* __restrict__ v_cache, int64_t cache_elems,
    const int64_t* __restrict__ tiles, int64_t n_tiles, const int64_t* __restrict__ pstart,
    uint32_t* sink) {
  extern __shared__ __align__(16) char smem[];
  int64_t* s_off = reinterpret_cast<int64_t*>(smem);
  const int n = load_piece_offsets(tiles, n_tiles, pstart, cache_elems, s_off);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // this wave's V slots: 2 rounds x R tiles x 4 KB
  const uint32_t vring = (uint32_t)(uintptr_t)smem + kPieceMaxTiles * 8 + wave * (2 * R * kTileBytes);
  const int64_t k_lane = KMODE ? (int64_t)(lane & 15) * 128 + 8 * (lane >> 4) : (int64_t)lane * 8;
  const int n_mine = n > wave ? (n - wave + 3) / 4 : 0;  // tiles of this wave
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 kr[2][R][4];
  u32x4 vr[2][R][4];
  auto issue = [&](int set, int round) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int j = round * R + u;
      const int t = wave + 4 * (j < n_mine ? j : 0);
      const int64_t off = s_off[t < n ? t : 0];
      const f16* kp = k_cache + off + k_lane;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kr[set][u][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + (KMODE ? 32 * c : 512 * c)));
      if (VMODE == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          vr[set][u][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(v_cache + off + lane * 8 + 512 * c));
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          dma16(vring + (set * R + u) * kTileBytes + c * 1024, v_cache + off + lane * 8 + 512 * c);
      }
    }
  };
  auto consume = [&](int set) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc ^= kr[set][u][c];
      if (VMODE == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc ^= vr[set][u][c];
      } else {
        acc ^= *reinterpret_cast<const u32x4*>(smem + kPieceMaxTiles * 8 + wave * (2 * R * kTileBytes) +
                                               (set * R + u) * kTileBytes + lane * 16);
      }
    }
  };
  const int rounds = (n_mine + R - 1) / R;
  if (rounds > 0) issue(0, 0);
  for (int r = 0; r < rounds; r += 2) {
    if (r + 1 < rounds) issue(1, r + 1);
    if (r + 1 < rounds) wait_vm<8 * R>(); else wait_vm<0>();
    consume(0);
    if (r + 1 >= rounds) break;
    if (r + 2 < rounds) issue(0, r + 2);
    if (r + 2 < rounds) wait_vm<8 * R>(); else wait_vm<0>();
    consume(1);
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) sink[0] = acc[0];
}

// Lane 0 of every workgroup adds 1 to a counter `per_wg` times in a row,
// each add waiting for the previous one's result: one counter for the whole
// grid (spread 0), one per XCD (spread 1, by blockIdx.x % 8), or one per
// workgroup (spread 2); counters sit 256 bytes apart.  Measures the round
// trip and the same-address throughput of device-scope atomics.
__global__ void atomics_kernel(int32_t* ctrs, int per_wg, int spread, uint32_t* sink) {
  if (threadIdx.x != 0) return;
  const int slot = spread == 0 ? 0 : spread == 1 ? (int)(blockIdx.x % 8) : (int)(blockIdx.x % 1024);
  int32_t* c = ctrs + 64 * slot;
  int v = 0;
  for (int i = 0; i < per_wg; ++i)
    v += __hip_atomic_fetch_add(c, 1 + (v & 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (v == 0x7fffffff) sink[0] = (uint32_t)v;
}

}  // namespace
}  // namespace nsd

using namespace nsd;

namespace {

template <int U>
void launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int grid, hipStream_t st) {
  hipLaunchKernelGGL(stream_read_kernel<U>, dim3(grid), dim3(kStreamThreads), 0, st,
                     static_cast<const u32x4*>(src), bytes / ((int64_t)kStreamThreads * U * 16), sink);
}

// Raises a kernel's dynamic-LDS limit to the whole CU; callers keep the
// result in a function-local static, so it runs once per process (C++
// static initialisation is thread-safe) and a failure stays reported.
hipError_t allow_full_lds(const void* fn) {
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

template <int RING>
int launch_gather_pieces(const void* k_cache, const void* v_cache, int64_t cache_elems, const int64_t* tiles,
                         int64_t n_tiles, const int64_t* piece_start, int n_pieces, int lds_extra,
                         uint32_t* sink, hipStream_t st) {
  static const hipError_t attr = allow_full_lds(reinterpret_cast<const void*>(&gather_pieces_kernel<RING>));
  if (attr != hipSuccess)
    return fail(NSD_ERR_HIP, "nsd_probe_gather_pieces: LDS attribute: %s", hipGetErrorString(attr));
  const int lds = RING * kGatherSlot + kPieceMaxTiles * 8 + lds_extra;
  if (lds > 160 * 1024) return fail(NSD_ERR_INVALID, "nsd_probe_gather_pieces: %d bytes of LDS", lds);
  hipLaunchKernelGGL(gather_pieces_kernel<RING>, dim3(n_pieces), dim3(kGatherThreads), lds, st,
                     static_cast<const f16*>(k_cache), static_cast<const f16*>(v_cache), cache_elems, tiles,
                     n_tiles, piece_start, sink);
  return launch_status("nsd_probe_gather_pieces");
}

template <int U>
int launch_gather_vgpr(const void* k_cache, const void* v_cache, int64_t cache_elems, const int64_t* tiles,
                       int64_t n_tiles, const int64_t* piece_start, int n_pieces, uint32_t* sink,
                       hipStream_t st) {
  hipLaunchKernelGGL(gather_vgpr_kernel<U>, dim3(n_pieces), dim3(kGatherThreads), 0, st,
                     static_cast<const f16*>(k_cache), static_cast<const f16*>(v_cache), cache_elems, tiles,
                     n_tiles, piece_start, sink);
  return launch_status("nsd_probe_gather_vgpr");
}

int check_gather_args(const char* what, const void* k_cache, const void* v_cache, int64_t cache_elems,
                      const int64_t* tiles, int64_t n_tiles, const int64_t* starts, int n, uint32_t* sink) {
  if (k_cache == nullptr || v_cache == nullptr || sink == nullptr || starts == nullptr ||
      (tiles == nullptr && n_tiles > 0))
    return fail(NSD_ERR_INVALID, "%s: null pointer", what);
  if (cache_elems < kTileElems || n_tiles < 0)
    return fail(NSD_ERR_INVALID, "%s: cache smaller than one tile or negative tile count", what);
  if (n <= 0 || n > (1 << 20)) return fail(NSD_ERR_INVALID, "%s: %d workgroups out of range", what, n);
  return NSD_OK;
}

template <int R, int KMODE, int VMODE>
int launch_gather_wave(const void* k_cache, const void* v_cache, int64_t cache_elems, const int64_t* tiles,
                       int64_t n_tiles, const int64_t* piece_start, int n_pieces, int lds_extra, uint32_t* sink,
                       hipStream_t st) {
  static const hipError_t attr = allow_full_lds(reinterpret_cast<const void*>(&gather_wave_kernel<R, KMODE, VMODE>));
  if (attr != hipSuccess)
    return fail(NSD_ERR_HIP, "nsd_probe_gather_wave: LDS attribute: %s", hipGetErrorString(attr));
  const int lds = kPieceMaxTiles * 8 + (VMODE ? 4 * 2 * R * kTileBytes : 0) + lds_extra;
  if (lds > 160 * 1024) return fail(NSD_ERR_INVALID, "nsd_probe_gather_wave: %d bytes of LDS", lds);
  hipLaunchKernelGGL((gather_wave_kernel<R, KMODE, VMODE>), dim3(n_pieces), dim3(kGatherThreads), lds, st,
                     static_cast<const f16*>(k_cache), static_cast<const f16*>(v_cache), cache_elems, tiles,
                     n_tiles, piece_start, sink);
  return launch_status("nsd_probe_gather_wave");
}

}  // namespace

extern "C" int nsd_probe_gather_wave(const void* k_cache, const void* v_cache, int64_t cache_elems,
                                     const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                                     int n_pieces, int round_tiles, int k_mode, int v_mode, int lds_extra,
                                     uint32_t* sink, void* stream) {
  int rc = check_gather_args("nsd_probe_gather_wave", k_cache, v_cache, cache_elems, tiles, n_tiles,
                             piece_start, n_pieces, sink);
  if (rc != NSD_OK) return rc;
  if (lds_extra < 0) return fail(NSD_ERR_INVALID, "nsd_probe_gather_wave: negative LDS pad");
  hipStream_t st = as_stream(stream);
  const int sel = round_tiles * 100 + k_mode * 10 + v_mode;
#define NSD_WAVE_CASE(R, K, V) \
  case R * 100 + K * 10 + V: \
    return launch_gather_wave<R, K, V>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, \
                                       lds_extra, sink, st);
  switch (sel) {
    NSD_WAVE_CASE(1, 0, 0) NSD_WAVE_CASE(1, 1, 0) NSD_WAVE_CASE(1, 0, 1) NSD_WAVE_CASE(1, 1, 1)
    NSD_WAVE_CASE(2, 0, 0) NSD_WAVE_CASE(2, 1, 0) NSD_WAVE_CASE(2, 0, 1) NSD_WAVE_CASE(2, 1, 1)
    default:
      return fail(NSD_ERR_INVALID, "nsd_probe_gather_wave: round %d, k mode %d, v mode %d not built",
                  round_tiles, k_mode, v_mode);
  }
#undef NSD_WAVE_CASE
}

namespace {

}  // namespace

extern "C" int nsd_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int grid, void* stream) {
  return nsd_probe_stream_read_unroll(src, bytes, sink, grid, 4, stream);
}

extern "C" int nsd_probe_stream_read_unroll(const void* src, int64_t bytes, uint32_t* sink, int grid, int unroll,
                                            void* stream) {
  if (src == nullptr || sink == nullptr) return fail(NSD_ERR_INVALID, "nsd_probe_stream_read: null pointer");
  if (bytes <= 0 || bytes % kStreamQuantum != 0)
    return fail(NSD_ERR_INVALID, "nsd_probe_stream_read: bytes must be a positive multiple of %lld",
                (long long)kStreamQuantum);
  if (grid <= 0 || grid > (1 << 20)) return fail(NSD_ERR_INVALID, "nsd_probe_stream_read: grid out of range");
  hipStream_t st = as_stream(stream);
  switch (unroll) {
    case 1: launch_stream_read<1>(src, bytes, sink, grid, st); break;
    case 2: launch_stream_read<2>(src, bytes, sink, grid, st); break;
    case 4: launch_stream_read<4>(src, bytes, sink, grid, st); break;
    case 8: launch_stream_read<8>(src, bytes, sink, grid, st); break;
    case 16: launch_stream_read<16>(src, bytes, sink, grid, st); break;
    default: return fail(NSD_ERR_INVALID, "nsd_probe_stream_read: unroll %d not in {1, 2, 4, 8, 16}", unroll);
  }
  return launch_status("nsd_probe_stream_read");
}

extern "C" int nsd_probe_atomics(int32_t* counters, int per_wg, int spread, int grid, uint32_t* sink,
                                 void* stream) {
  if (counters == nullptr || sink == nullptr) return fail(NSD_ERR_INVALID, "nsd_probe_atomics: null pointer");
  if (per_wg < 0 || per_wg > 4096 || spread < 0 || spread > 2 || grid <= 0 || grid > (1 << 20))
    return fail(NSD_ERR_INVALID, "nsd_probe_atomics: argument out of range");
  hipLaunchKernelGGL(atomics_kernel, dim3(grid), dim3(64), 0, as_stream(stream), counters, per_wg, spread, sink);
  return launch_status("nsd_probe_atomics");
}

extern "C" int nsd_probe_empty(int grid, void* stream) {
  if (grid <= 0 || grid > (1 << 20)) return fail(NSD_ERR_INVALID, "nsd_probe_empty: grid out of range");
  hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(64), 0, as_stream(stream));
  return launch_status("nsd_probe_empty");
}

extern "C" int nsd_probe_gather_pieces(const void* k_cache, const void* v_cache, int64_t cache_elems,
                                       const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                                       int n_pieces, int ring, int lds_extra, uint32_t* sink, void* stream) {
  int rc = check_gather_args("nsd_probe_gather_pieces", k_cache, v_cache, cache_elems, tiles, n_tiles,
                             piece_start, n_pieces, sink);
  if (rc != NSD_OK) return rc;
  if (lds_extra < 0) return fail(NSD_ERR_INVALID, "nsd_probe_gather_pieces: negative LDS pad");
  hipStream_t st = as_stream(stream);
  switch (ring) {
    case 3: return launch_gather_pieces<3>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    case 4: return launch_gather_pieces<4>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    case 6: return launch_gather_pieces<6>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    case 8: return launch_gather_pieces<8>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    case 12: return launch_gather_pieces<12>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    case 16: return launch_gather_pieces<16>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, lds_extra, sink, st);
    default: return fail(NSD_ERR_INVALID, "nsd_probe_gather_pieces: ring %d not in {3, 4, 6, 8, 12, 16}", ring);
  }
}

extern "C" int nsd_probe_gather_vgpr(const void* k_cache, const void* v_cache, int64_t cache_elems,
                                     const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                                     int n_pieces, int unroll, uint32_t* sink, void* stream) {
  int rc = check_gather_args("nsd_probe_gather_vgpr", k_cache, v_cache, cache_elems, tiles, n_tiles,
                             piece_start, n_pieces, sink);
  if (rc != NSD_OK) return rc;
  hipStream_t st = as_stream(stream);
  switch (unroll) {
    case 1: return launch_gather_vgpr<1>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, sink, st);
    case 2: return launch_gather_vgpr<2>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, sink, st);
    case 4: return launch_gather_vgpr<4>(k_cache, v_cache, cache_elems, tiles, n_tiles, piece_start, n_pieces, sink, st);
    default: return fail(NSD_ERR_INVALID, "nsd_probe_gather_vgpr: unroll %d not in {1, 2, 4}", unroll);
  }
}

extern "C" int nsd_probe_tile_gather(const void* k_cache, const void* v_cache, int64_t cache_elems,
                                     const int64_t* tiles, int64_t n_tiles, const int64_t* worker_start,
                                     int n_workers, uint32_t* sink, void* stream) {
  if (k_cache == nullptr || v_cache == nullptr || sink == nullptr || worker_start == nullptr ||
      (tiles == nullptr && n_tiles > 0))
    return fail(NSD_ERR_INVALID, "nsd_probe_tile_gather: null pointer");
  if (cache_elems < kTileElems || n_tiles < 0)
    return fail(NSD_ERR_INVALID, "nsd_probe_tile_gather: cache smaller than one tile or negative tile count");
  if (n_workers <= 0 || n_workers > (1 << 20))
    return fail(NSD_ERR_INVALID, "nsd_probe_tile_gather: n_workers out of range");
  static const hipError_t attr = allow_full_lds(reinterpret_cast<const void*>(&tile_gather_kernel));
  if (attr != hipSuccess)
    return fail(NSD_ERR_HIP, "nsd_probe_tile_gather: LDS attribute: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL(tile_gather_kernel, dim3(n_workers), dim3(kGatherThreads), kGatherLds, as_stream(stream),
                     static_cast<const f16*>(k_cache), static_cast<const f16*>(v_cache), cache_elems, tiles,
                     n_tiles, worker_start, sink);
  return launch_status("nsd_probe_tile_gather");
}
