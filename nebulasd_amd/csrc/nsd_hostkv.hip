// HostKV block-range copies for gfx950 (MI355X): byte images of KV-cache
// blocks moved between the device caches and pinned host planes.
//
//   nsd_copy_block_ranges -- one copy plan of the HostKV DMA backend
//     (nebulasd/src/nebulasd/kv/cuda_transfer.py:78-108): for every region,
//     block_count blocks of the K plane and of the V plane, device to host
//     (write-back) or host to device (restore).
//   nsd_swap_blocks -- swiftLLM/csrc/src/block_swapping.cpp:22-85: block-id
//     pairs between the device caches and a host swap space.
//
// A block is block_bytes contiguous bytes on both sides ([L, Hkv, 16, d]
// fp16 for the caches of this project), so a region is one contiguous range
// per plane.  Regions that continue where the previous region ended on both
// sides are merged into one run (the coalescing block_swapping.cpp:35-40 does
// for consecutive ids, applied to any plan).  Runs keep the plan's order,
// K before V within a region, as the reference issues its copies.
//
// Two engines carry the runs:
//   NSD_COPY_ENGINE_DMA    -- one hipMemcpyAsync per run: the system DMA
//     engines move the bytes and no compute unit is taken from the kernels
//     the copy overlaps with.  Runs execute in order, so a later run wins
//     where destinations overlap, as with the reference's stream of copies.
//   NSD_COPY_ENGINE_KERNEL -- one launch per kMaxRunsPerLaunch runs: 32
//     workgroups of 256 threads stride over the runs' 64 KB chunks with
//     16-byte vector loads and stores, reading or writing the pinned host
//     memory directly over the host link.  A plan of many scattered blocks
//     costs one launch instead of one DMA command (about 9 us each) per
//     run; the price is 32 compute units taken from kernels the copy
//     overlaps with.  Overlapping destinations are rejected (no order
//     between workgroups).  Host planes must be pinned (hipHostMalloc) and
//     everything 16-byte aligned.
#include <algorithm>
#include <vector>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kVec = 16;                                   // bytes per vector access
constexpr int kChunkBytes = 64 * 1024;                     // one workgroup's share of a run
constexpr int kVecPerThread = kChunkBytes / (kCopyThreads * kVec);  // 16
constexpr int kMaxRunsPerLaunch = 64;                      // runs carried in the kernel arguments
constexpr uint32_t kMaxChunksPerLaunch = 1u << 23;         // 2^31 work-items per launch at most
constexpr int64_t kMaxRunBytes = (int64_t)kMaxChunksPerLaunch * kChunkBytes;

static_assert(kVecPerThread * kCopyThreads * kVec == kChunkBytes, "chunk must tile the workgroup");

// Global address space, so the accesses compile to global_* rather than flat_*.
typedef __attribute__((address_space(1))) u32x4 gbl_u32x4;

// The runs of one launch, passed by value (1.8 KB of kernel arguments).
// Run r covers chunks [chunk_begin[r], chunk_begin[r+1]).
struct CopyRuns {
  uint64_t src[kMaxRunsPerLaunch];
  uint64_t dst[kMaxRunsPerLaunch];
  uint64_t bytes[kMaxRunsPerLaunch];
  uint32_t chunk_begin[kMaxRunsPerLaunch + 1];
  int32_t n;
};

// Workgroups per launch.  32 keep 32 x 64 KB of requests in flight, enough
// to fill the host link (about 57 GB/s each way, the same as the DMA
// engines, on plans of 1.2 MB blocks); more add nothing and take compute
// units from kernels the copy overlaps with.  Plain (temporal) accesses:
// non-temporal stores to host memory measured slower.
constexpr uint32_t kCopyWorkgroups = 32;

// Workgroup w copies chunks w, w + gridDim.x, ... of the launch's runs.
__global__ void __launch_bounds__(kCopyThreads) copy_runs_kernel(const CopyRuns runs) {
  const uint32_t total = runs.chunk_begin[runs.n];
  for (uint32_t c = blockIdx.x; c < total; c += gridDim.x) {
    // Binary search for the run holding chunk c: chunk_begin[lo] <= c < chunk_begin[hi].
    int lo = 0, hi = runs.n;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (runs.chunk_begin[mid] <= c) lo = mid; else hi = mid;
    }
    const uint64_t off = (uint64_t)(c - runs.chunk_begin[lo]) * kChunkBytes;
    const uint64_t left = runs.bytes[lo] - off;  // > 0, a multiple of kVec
    const gbl_u32x4* src = reinterpret_cast<const gbl_u32x4*>(runs.src[lo] + off);
    gbl_u32x4* dst = reinterpret_cast<gbl_u32x4*>(runs.dst[lo] + off);
    if (left >= (uint64_t)kChunkBytes) {
      // Every load of the chunk is issued before the first store, so a wave
      // keeps 16 requests in flight across the host link's latency.
      u32x4 v[kVecPerThread];
#pragma unroll
      for (int i = 0; i < kVecPerThread; ++i) v[i] = src[threadIdx.x + i * kCopyThreads];
#pragma unroll
      for (int i = 0; i < kVecPerThread; ++i) dst[threadIdx.x + i * kCopyThreads] = v[i];
    } else {
      const int nv = (int)(left / kVec);
      for (int i = threadIdx.x; i < nv; i += kCopyThreads) dst[i] = src[i];
    }
  }
}

struct Run {
  char* dst;
  const char* src;
  int64_t bytes;
};

struct Planes {
  char* gpu[2];   // K, V device caches
  char* host[2];  // K, V host planes
  int64_t gpu_blocks, host_blocks, block_bytes;
};

// Regions -> runs, merging a region into the previous one when both of its
// ranges continue where the previous region's ended.  Validates every range
// before anything is enqueued.
int build_runs(const Planes& p, const int64_t* gpu_begin, const int64_t* host_begin, const int64_t* count,
               int64_t n, bool d2h, const char* what, std::vector<Run>* runs) {
  int64_t cur_g = -1, cur_h = -1, cur_n = 0;
  auto flush = [&]() {
    if (cur_n == 0) return;
    const int64_t bytes = cur_n * p.block_bytes;
    for (int plane = 0; plane < 2; ++plane) {
      char* g = p.gpu[plane] + cur_g * p.block_bytes;
      char* h = p.host[plane] + cur_h * p.block_bytes;
      runs->push_back(d2h ? Run{h, g, bytes} : Run{g, h, bytes});
    }
    cur_n = 0;
  };
  for (int64_t i = 0; i < n; ++i) {
    const int64_t g = gpu_begin[i], h = host_begin[i], c = count[i];
    if (g < 0 || h < 0 || c < 0) return fail(NSD_ERR_INVALID, "%s: negative copy range (region %lld)", what, (long long)i);
    if (c > p.gpu_blocks - g) return fail(NSD_ERR_INVALID, "%s: copy exceeds GPU KV cache (region %lld)", what, (long long)i);
    if (c > p.host_blocks - h) return fail(NSD_ERR_INVALID, "%s: copy exceeds HostKV plane (region %lld)", what, (long long)i);
    if (c == 0) continue;
    if (cur_n > 0 && g == cur_g + cur_n && h == cur_h + cur_n) {
      cur_n += c;
    } else {
      flush();
      cur_g = g, cur_h = h, cur_n = c;
    }
  }
  flush();
  return NSD_OK;
}

bool destinations_overlap(const std::vector<Run>& runs) {
  std::vector<std::pair<uintptr_t, uintptr_t>> iv;
  iv.reserve(runs.size());
  for (const Run& r : runs) iv.emplace_back((uintptr_t)r.dst, (uintptr_t)r.dst + (uintptr_t)r.bytes);
  std::sort(iv.begin(), iv.end());
  for (size_t i = 1; i < iv.size(); ++i)
    if (iv[i].first < iv[i - 1].second) return true;
  return false;
}

bool ranges_overlap(const char* a, const char* b, int64_t bytes) {
  return (uintptr_t)a < (uintptr_t)b + (uintptr_t)bytes && (uintptr_t)b < (uintptr_t)a + (uintptr_t)bytes;
}

// True when [p, p + bytes) starts and ends in memory the device can reach
// as pinned host memory.
bool pinned_host(const char* p, int64_t bytes) {
  for (const char* q : {p, p + bytes - 1}) {
    hipPointerAttribute_t a{};
    const hipError_t err = hipPointerGetAttributes(&a, q);
    if (err != hipSuccess) {
      (void)hipGetLastError();  // an unregistered pointer is an answer, not a pending error
      return false;
    }
    if (a.type != hipMemoryTypeHost || a.devicePointer != (void*)q) return false;
  }
  return true;
}

int run_dma(const std::vector<Run>& runs, bool d2h, hipStream_t stream, const char* what) {
  const hipMemcpyKind kind = d2h ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
  for (const Run& r : runs) {
    const hipError_t err = hipMemcpyAsync(r.dst, r.src, (size_t)r.bytes, kind, stream);
    if (err != hipSuccess) return fail(NSD_ERR_HIP, "%s: hipMemcpyAsync failed: %s", what, hipGetErrorString(err));
  }
  return NSD_OK;
}

int run_kernel(const std::vector<Run>& runs, hipStream_t stream, const char* what) {
  CopyRuns batch{};
  uint32_t chunks = 0;
  auto launch = [&]() -> int {
    if (batch.n == 0) return NSD_OK;
    batch.chunk_begin[batch.n] = chunks;
    const uint32_t grid = std::min(chunks, kCopyWorkgroups);
    hipLaunchKernelGGL(copy_runs_kernel, dim3(grid), dim3(kCopyThreads), 0, stream, batch);
    const int rc = launch_status(what);
    batch.n = 0;
    chunks = 0;
    return rc;
  };
  for (const Run& r : runs) {
    const uint32_t rc = (uint32_t)((r.bytes + kChunkBytes - 1) / kChunkBytes);
    if (batch.n == kMaxRunsPerLaunch || (batch.n > 0 && chunks + rc > kMaxChunksPerLaunch)) {
      if (int e = launch()) return e;
    }
    batch.src[batch.n] = (uint64_t)(uintptr_t)r.src;
    batch.dst[batch.n] = (uint64_t)(uintptr_t)r.dst;
    batch.bytes[batch.n] = (uint64_t)r.bytes;
    batch.chunk_begin[batch.n] = chunks;
    ++batch.n;
    chunks += rc;
  }
  return launch();
}

int copy_plan(const Planes& p, const int64_t* gpu_begin, const int64_t* host_begin, const int64_t* count, int64_t n,
              bool d2h, int engine, void* stream, const char* what) {
  if (n < 0) return fail(NSD_ERR_INVALID, "%s: negative region count", what);
  if (n == 0) return NSD_OK;
  if (!gpu_begin || !host_begin || !count) return fail(NSD_ERR_INVALID, "%s: null region array", what);
  if (!p.gpu[0] || !p.gpu[1] || !p.host[0] || !p.host[1]) return fail(NSD_ERR_INVALID, "%s: null plane", what);
  if (p.block_bytes < 1 || p.gpu_blocks < 0 || p.host_blocks < 0)
    return fail(NSD_ERR_INVALID, "%s: bad block geometry", what);
  if (engine != NSD_COPY_ENGINE_DMA && engine != NSD_COPY_ENGINE_KERNEL)
    return fail(NSD_ERR_INVALID, "%s: unknown copy engine %d", what, engine);
  if (p.gpu_blocks > INT64_MAX / p.block_bytes || p.host_blocks > INT64_MAX / p.block_bytes)
    return fail(NSD_ERR_INVALID, "%s: plane size overflows", what);
  const int64_t gpu_plane = p.gpu_blocks * p.block_bytes, host_plane = p.host_blocks * p.block_bytes;
  if (ranges_overlap(p.gpu[0], p.gpu[1], gpu_plane)) return fail(NSD_ERR_INVALID, "%s: K and V caches overlap", what);
  if (ranges_overlap(p.host[0], p.host[1], host_plane)) return fail(NSD_ERR_INVALID, "%s: K and V host planes overlap", what);

  std::vector<Run> runs;
  runs.reserve((size_t)std::min<int64_t>(n, 4096) * 2);
  if (int e = build_runs(p, gpu_begin, host_begin, count, n, d2h, what, &runs)) return e;
  if (runs.empty()) return NSD_OK;
  if (engine == NSD_COPY_ENGINE_DMA) return run_dma(runs, d2h, as_stream(stream), what);

  if (p.block_bytes % kVec != 0)
    return fail(NSD_ERR_UNSUPPORTED, "%s: kernel engine needs block_bytes %% 16 == 0 (got %lld)", what,
                (long long)p.block_bytes);
  for (int plane = 0; plane < 2; ++plane)
    if ((uintptr_t)p.gpu[plane] % kVec != 0 || (uintptr_t)p.host[plane] % kVec != 0)
      return fail(NSD_ERR_UNSUPPORTED, "%s: kernel engine needs 16-byte aligned planes", what);
  for (const Run& r : runs)
    if (r.bytes > kMaxRunBytes) return fail(NSD_ERR_UNSUPPORTED, "%s: run of %lld bytes exceeds the kernel engine's limit", what, (long long)r.bytes);
  if (host_plane > 0 && (!pinned_host(p.host[0], host_plane) || !pinned_host(p.host[1], host_plane)))
    return fail(NSD_ERR_INVALID, "%s: kernel engine needs pinned host planes (hipHostMalloc)", what);
  if (destinations_overlap(runs))
    return fail(NSD_ERR_UNSUPPORTED, "%s: kernel engine needs disjoint destinations (use the DMA engine)", what);
  return run_kernel(runs, as_stream(stream), what);
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_copy_block_ranges(void* k_cache, void* v_cache, int64_t gpu_blocks, void* host_k, void* host_v,
                                     int64_t host_blocks, int64_t block_bytes, const int64_t* gpu_begin_block,
                                     const int64_t* host_begin_block, const int64_t* block_count, int64_t n_regions,
                                     int direction, int engine, void* stream) {
  if (direction != NSD_COPY_D2H && direction != NSD_COPY_H2D)
    return fail(NSD_ERR_INVALID, "copy_block_ranges: direction must be NSD_COPY_D2H or NSD_COPY_H2D");
  const Planes p{{(char*)k_cache, (char*)v_cache}, {(char*)host_k, (char*)host_v}, gpu_blocks, host_blocks, block_bytes};
  return copy_plan(p, gpu_begin_block, host_begin_block, block_count, n_regions, direction == NSD_COPY_D2H, engine,
                   stream, "copy_block_ranges");
}

extern "C" int nsd_swap_blocks(const int64_t* source_block_ids, const int64_t* target_block_ids, int64_t n,
                               int is_swap_in, void* k_cache, void* v_cache, int64_t gpu_blocks, void* k_swap,
                               void* v_swap, int64_t swap_blocks, int64_t block_bytes, int engine, void* stream) {
  if (n < 0) return fail(NSD_ERR_INVALID, "swap_blocks: negative block count");
  if (n == 0) return NSD_OK;
  if (!source_block_ids || !target_block_ids) return fail(NSD_ERR_INVALID, "swap_blocks: null id array");
  // Every pair is a one-block region; consecutive pairs merge into runs.
  std::vector<int64_t> ones((size_t)n, 1);
  const int64_t* gpu_ids = is_swap_in ? target_block_ids : source_block_ids;
  const int64_t* host_ids = is_swap_in ? source_block_ids : target_block_ids;
  const Planes p{{(char*)k_cache, (char*)v_cache}, {(char*)k_swap, (char*)v_swap}, gpu_blocks, swap_blocks, block_bytes};
  return copy_plan(p, gpu_ids, host_ids, ones.data(), n, !is_swap_in, engine, stream, "swap_blocks");
}
