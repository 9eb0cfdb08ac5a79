/*
 * Measurement probes beside the attention path: the HBM read rates that bound
 * the paged attention on this device.  They have no counterpart in the
 * reference (whose path is Triton kernels with no ceiling measurement); the
 * benchmark reports them next to the attention's achieved rate.  Both read
 * device memory only and write one word of `sink` only in a case the data
 * practically never meets (it keeps the loads from being optimised away).
 * Return codes as in nsd_attn.h.
 */
#ifndef NSD_PROBE_H
#define NSD_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * nsd_probe_stream_read: read `bytes` (a positive multiple of 16 KiB) of the
 * device buffer `src` once, in 16 KiB chunks strided over `grid` workgroups
 * of 256 threads with 16-byte loads.
 */
int nsd_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int grid, void* stream);

/*
 * nsd_probe_tile_gather: stream the K and V tiles named by `tiles` into LDS
 * without using them.  tiles: device int64 [n_tiles], element offsets of a
 * 16 x 128 fp16 tile in k_cache (the V tile is at the same offset in v_cache;
 * in the [blocks, layers, kv_heads, 16, 128] cache layout the offset of block
 * b, layer l, head h is ((b * layers + l) * kv_heads + h) * 2048).
 * worker_start: device int64 [n_workers + 1]; workgroup w reads tiles
 * [worker_start[w], worker_start[w + 1]) (at most 1536) in order.  Offsets and
 * ranges are clamped into [0, cache_elems - 2048] and [0, n_tiles].
 */
int nsd_probe_tile_gather(const void* k_cache, const void* v_cache, int64_t cache_elems,
                          const int64_t* tiles, int64_t n_tiles, const int64_t* worker_start,
                          int n_workers, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSD_PROBE_H */
