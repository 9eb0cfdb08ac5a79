/*
 * Measurement probes beside the attention path: the HBM read rates that bound
 * the paged attention on this device.  They have no counterpart in the
 * reference (whose path is Triton kernels with no ceiling measurement); the
 * benchmark reports them next to the attention's achieved rate.  The read
 * probes read device memory only and write one word of `sink` only in a case
 * the data practically never meets (it keeps the loads from being optimised
 * away).
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

/*
 * nsd_probe_stream_read_unroll: as nsd_probe_stream_read (which uses unroll
 * 4), with `unroll` (1, 2, 4, 8 or 16) 16-byte loads in flight per thread
 * and chunk; `bytes` a positive multiple of 64 KiB.
 */
int nsd_probe_stream_read_unroll(const void* src, int64_t bytes, uint32_t* sink, int grid, int unroll,
                                 void* stream);

/*
 * nsd_probe_gather_pieces: the tiles of nsd_probe_tile_gather cut into
 * `n_pieces` pieces; workgroup p streams tiles [piece_start[p],
 * piece_start[p + 1]) (at most 256) through an LDS ring of `ring` (3, 4, 6,
 * 8, 12 or 16) K+V items, as the hardware dispatches it.  Each workgroup
 * takes ring * 8 KiB + 2 KiB + lds_extra bytes of LDS (at most 160 KiB), which
 * sets how many share a CU.
 */
int nsd_probe_gather_pieces(const void* k_cache, const void* v_cache, int64_t cache_elems,
                            const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                            int n_pieces, int ring, int lds_extra, uint32_t* sink, void* stream);

/*
 * nsd_probe_gather_vgpr: the pieces of nsd_probe_gather_pieces read into
 * registers, `unroll` (1, 2 or 4) K+V tiles per wave and round.
 */
int nsd_probe_gather_vgpr(const void* k_cache, const void* v_cache, int64_t cache_elems,
                          const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                          int n_pieces, int unroll, uint32_t* sink, void* stream);

/*
 * nsd_probe_gather_wave: the pieces of nsd_probe_gather_pieces streamed by
 * each wave on its own (wave w takes tiles w, w + 4, ... of its workgroup's
 * piece; no barriers), `round_tiles` (1 or 2) tiles per round with the next
 * round in flight.  k_mode 1 reads K in the A-operand layout of
 * v_mfma_f32_16x16x32_f16 (16 rows x 64 B per load), 0 in contiguous 1 KB
 * runs; v_mode 0 reads V into registers, 1 into the wave's own LDS slots by
 * global_load_lds_dwordx4.  LDS: 2 KiB + (v_mode ? 32 KiB * round_tiles : 0)
 * + lds_extra bytes per workgroup (at most 160 KiB).
 */
int nsd_probe_gather_wave(const void* k_cache, const void* v_cache, int64_t cache_elems,
                          const int64_t* tiles, int64_t n_tiles, const int64_t* piece_start,
                          int n_pieces, int round_tiles, int k_mode, int v_mode, int lds_extra,
                          uint32_t* sink, void* stream);

/*
 * nsd_probe_atomics: lane 0 of each of `grid` workgroups adds 1 to a device
 * int32 counter `per_wg` (<= 4096) times, each add waiting for the previous
 * result; one counter for the grid (spread 0), one per XCD (1) or one per
 * workgroup (2, up to 1024 counters).  counters: device int32 [1024 * 64].
 */
int nsd_probe_atomics(int32_t* counters, int per_wg, int spread, int grid, uint32_t* sink, void* stream);

/* nsd_probe_empty: launch a kernel of `grid` one-wave workgroups that does nothing. */
int nsd_probe_empty(int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSD_PROBE_H */
