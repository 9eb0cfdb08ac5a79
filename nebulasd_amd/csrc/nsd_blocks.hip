// Block-table metadata kernels for gfx950 (MI355X): the writes that produce
// the attention path's index input.
//
//   nsd_write_block_ranges  -- bank ranges: row r gets begin_r + 0..count_r-1
//     (the metadata writer of nebulasd/src/nebulasd/workers/dma_process.py:95-125,
//     which builds flat index/value arrays on the host, copies both to the
//     device and runs index_copy_; and the per-request fill of
//     swiftLLM/swiftllm/worker/block_manager.py:685-691).  Here the device
//     gets three ints per range and writes the values itself.
//   nsd_set_block_table      -- swiftLLM/swiftllm/worker/kernels/block_mgmt.py:5-45
//   nsd_unset_block_table    -- block_mgmt.py:48-80
//   nsd_gather_allocated_blocks_and_unset -- block_mgmt.py:83-127
//
// All are latency-bound integer kernels (a few KB per call); bit-exact by
// construction.  Indices outside the table or the block pool are skipped and
// flagged in the optional status word instead of faulting.
#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kThreads = 256;
constexpr int kGatherThreads = 1024;
constexpr int kMaxGatherBatch = 4096;  // sequences per gather call (one workgroup's LDS scan)

// One workgroup per range.
__global__ void __launch_bounds__(kThreads)
write_ranges_kernel(int32_t* bt, int64_t bt_rows, int64_t bt_stride, const int32_t* rows,
                    const int32_t* begins, const int32_t* counts, int32_t* num_alloc,
                    int32_t* status) {
  const int i = blockIdx.x;
  const int row = rows[i], begin = begins[i], count = counts[i];
  if (row < 0 || row >= bt_rows || count < 0 || count > bt_stride || begin < 0) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  int32_t* dst = bt + (int64_t)row * bt_stride;
  for (int j = threadIdx.x; j < count; j += kThreads) dst[j] = begin + j;
  if (num_alloc != nullptr && threadIdx.x == 0) num_alloc[row] = count;
}

// One workgroup per batch entry; its offset into candidate_blocks is the sum
// of the earlier entries' block_needed (read-only here, so no ordering issue).
__global__ void __launch_bounds__(kThreads)
set_table_kernel(int32_t* num_alloc, int32_t* bt, int64_t bt_rows, int64_t bt_stride,
                 const int32_t* candidates, int64_t n_candidates, const int32_t* seq_ids,
                 const int32_t* needed, int32_t* status) {
  __shared__ int32_t s_part[kThreads / kWave];
  const int i = blockIdx.x;
  int32_t part = 0;
  for (int j = threadIdx.x; j < i; j += kThreads) part += needed[j];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, kWave);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
  __syncthreads();
  int64_t off = 0;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) off += s_part[w];
  const int seq = seq_ids[i], need = needed[i];
  if (seq < 0 || seq >= bt_rows || need < 0) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int have = num_alloc[seq];
  if (have < 0 || (int64_t)have + need > bt_stride || off + need > n_candidates) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  int32_t* dst = bt + (int64_t)seq * bt_stride + have;
  for (int j = threadIdx.x; j < need; j += kThreads) dst[j] = candidates[off + j];
  __syncthreads();  // every thread has read num_alloc[seq] before it changes
  if (threadIdx.x == 0) num_alloc[seq] = have + need;
}

// One workgroup per batch entry: mark its blocks free, zero its count.
__global__ void __launch_bounds__(kThreads)
unset_table_kernel(int32_t* num_alloc, const int32_t* bt, int64_t bt_rows, int64_t bt_stride,
                   const int32_t* seq_ids, uint8_t* is_free, int64_t num_blocks, int32_t* status) {
  const int seq = seq_ids[blockIdx.x];
  if (seq < 0 || seq >= bt_rows) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int n = num_alloc[seq];
  if (n < 0 || n > bt_stride) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int32_t* row = bt + (int64_t)seq * bt_stride;
  bool bad = false;
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int b = row[j];
    if (b < 0 || b >= num_blocks) bad = true;
    else is_free[b] = 1;
  }
  if (bad) flag_status(status, NSD_STATUS_BAD_BLOCK);
  __syncthreads();  // every thread has read num_alloc[seq] before it changes
  if (threadIdx.x == 0) num_alloc[seq] = 0;
}

// One workgroup: the counts of every batch entry are read into LDS and
// prefix-summed before any of them is reset, so an entry's offset never sees
// a count another entry already cleared.
__global__ void __launch_bounds__(kGatherThreads)
gather_unset_kernel(int32_t* num_alloc, const int32_t* bt, int64_t bt_rows, int64_t bt_stride,
                    const int32_t* seq_ids, int batch, uint8_t* is_free, int64_t num_blocks,
                    int32_t* gathered, int64_t capacity, int32_t* status) {
  __shared__ int32_t s_cnt[kMaxGatherBatch];
  __shared__ int32_t s_off[kMaxGatherBatch];  // <= batch * bt_stride, checked on the host
  __shared__ int32_t s_chunk[kGatherThreads];
  for (int i = threadIdx.x; i < batch; i += kGatherThreads) {
    const int seq = seq_ids[i];
    int n = (seq >= 0 && seq < bt_rows) ? num_alloc[seq] : -1;
    if (n < 0 || n > bt_stride) {
      flag_status(status, NSD_STATUS_BAD_SEQ);
      n = 0;
    }
    s_cnt[i] = n;
  }
  __syncthreads();
  // exclusive prefix: each thread sums a contiguous chunk, then a serial pass
  // over the chunk totals (batch <= 4096, so both steps are short)
  const int per = (batch + kGatherThreads - 1) / kGatherThreads;
  const int c0 = threadIdx.x * per, c1 = min(c0 + per, batch);
  int32_t t = 0;
  for (int i = c0; i < c1; ++i) t += s_cnt[i];
  s_chunk[threadIdx.x] = t;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t run = 0;
    for (int k = 0; k < kGatherThreads; ++k) {
      const int32_t v = s_chunk[k];
      s_chunk[k] = run;
      run += v;
    }
  }
  __syncthreads();
  int32_t run = s_chunk[threadIdx.x];
  for (int i = c0; i < c1; ++i) {
    s_off[i] = run;
    run += s_cnt[i];
  }
  __syncthreads();
  // copy out and free, one wave per entry
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  bool bad = false;
  for (int i = wave; i < batch; i += kGatherThreads / kWave) {
    const int n = s_cnt[i];
    if (n == 0) continue;
    const int32_t* row = bt + (int64_t)seq_ids[i] * bt_stride;
    const int64_t off = s_off[i];
    for (int j = lane; j < n; j += kWave) {
      const int b = row[j];
      if (off + j < capacity) gathered[off + j] = b;
      else bad = true;
      if (b < 0 || b >= num_blocks) bad = true;
      else is_free[b] = 1;
    }
  }
  if (bad) flag_status(status, NSD_STATUS_BAD_BLOCK);
  __syncthreads();  // all counts read (into LDS) and all rows copied before the resets
  for (int i = threadIdx.x; i < batch; i += kGatherThreads) {
    const int seq = seq_ids[i];
    if (seq >= 0 && seq < bt_rows) num_alloc[seq] = 0;
  }
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_write_block_ranges(int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                                      const int32_t* rows, const int32_t* begins,
                                      const int32_t* counts, int64_t n_ranges, int32_t* num_alloc,
                                      int32_t* status, void* stream) {
  if (n_ranges < 0) return fail(NSD_ERR_INVALID, "write_block_ranges: negative range count");
  if (n_ranges == 0) return NSD_OK;
  if (!block_table || !rows || !begins || !counts)
    return fail(NSD_ERR_INVALID, "write_block_ranges: null pointer");
  if (bt_rows < 1 || bt_stride < 1) return fail(NSD_ERR_INVALID, "write_block_ranges: empty block table");
  if (n_ranges > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "write_block_ranges: too many ranges");
  hipLaunchKernelGGL(write_ranges_kernel, dim3((unsigned)n_ranges), dim3(kThreads), 0, as_stream(stream),
                     block_table, bt_rows, bt_stride, rows, begins, counts, num_alloc, status);
  return launch_status("write_block_ranges");
}

extern "C" int nsd_set_block_table(int32_t* num_alloc, int32_t* block_table, int64_t bt_rows,
                                   int64_t bt_stride, const int32_t* candidate_blocks,
                                   int64_t n_candidates, const int32_t* seq_ids,
                                   const int32_t* block_needed, int64_t batch, int32_t* status,
                                   void* stream) {
  if (batch < 0 || n_candidates < 0) return fail(NSD_ERR_INVALID, "set_block_table: negative size");
  if (batch == 0) return NSD_OK;
  if (!num_alloc || !block_table || !seq_ids || !block_needed || (n_candidates > 0 && !candidate_blocks))
    return fail(NSD_ERR_INVALID, "set_block_table: null pointer");
  if (batch > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "set_block_table: batch too large");
  hipLaunchKernelGGL(set_table_kernel, dim3((unsigned)batch), dim3(kThreads), 0, as_stream(stream), num_alloc,
                     block_table, bt_rows, bt_stride, candidate_blocks, n_candidates, seq_ids, block_needed,
                     status);
  return launch_status("set_block_table");
}

extern "C" int nsd_unset_block_table(int32_t* num_alloc, const int32_t* block_table, int64_t bt_rows,
                                     int64_t bt_stride, const int32_t* seq_ids, int64_t batch,
                                     uint8_t* is_block_free, int64_t num_blocks, int32_t* status,
                                     void* stream) {
  if (batch < 0) return fail(NSD_ERR_INVALID, "unset_block_table: negative batch");
  if (batch == 0) return NSD_OK;
  if (!num_alloc || !block_table || !seq_ids || !is_block_free)
    return fail(NSD_ERR_INVALID, "unset_block_table: null pointer");
  if (batch > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "unset_block_table: batch too large");
  hipLaunchKernelGGL(unset_table_kernel, dim3((unsigned)batch), dim3(kThreads), 0, as_stream(stream), num_alloc,
                     block_table, bt_rows, bt_stride, seq_ids, is_block_free, num_blocks, status);
  return launch_status("unset_block_table");
}

extern "C" int nsd_gather_allocated_blocks_and_unset(int32_t* num_alloc, const int32_t* block_table,
                                                     int64_t bt_rows, int64_t bt_stride,
                                                     const int32_t* seq_ids, int64_t batch,
                                                     uint8_t* is_block_free, int64_t num_blocks,
                                                     int32_t* gathered, int64_t gathered_capacity,
                                                     int32_t* status, void* stream) {
  if (batch < 0 || gathered_capacity < 0) return fail(NSD_ERR_INVALID, "gather_allocated_blocks: negative size");
  if (batch == 0) return NSD_OK;
  if (batch > kMaxGatherBatch)
    return fail(NSD_ERR_UNSUPPORTED, "gather_allocated_blocks: batch %lld > %d", (long long)batch, kMaxGatherBatch);
  if (!num_alloc || !block_table || !seq_ids || !is_block_free || (gathered_capacity > 0 && !gathered))
    return fail(NSD_ERR_INVALID, "gather_allocated_blocks: null pointer");
  if (batch * bt_stride > INT32_MAX)
    return fail(NSD_ERR_UNSUPPORTED, "gather_allocated_blocks: batch x row capacity exceeds int32");
  hipLaunchKernelGGL(gather_unset_kernel, dim3(1), dim3(kGatherThreads), 0, as_stream(stream), num_alloc,
                     block_table, bt_rows, bt_stride, seq_ids, (int)batch, is_block_free, num_blocks, gathered,
                     gathered_capacity, status);
  return launch_status("gather_allocated_blocks");
}
