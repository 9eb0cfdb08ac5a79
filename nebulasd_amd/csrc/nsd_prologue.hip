// Attention prologue kernels for gfx950: QK-RMSNorm, RoPE, KV-cache store
// (decode/verify rows and prefill), and the fused one-launch prologue.
//
// All of these move at most a few MB per layer call, so they are
// launch-latency bound; the design goal is one launch, coalesced 16-byte
// copies for the cache writes, and wave64 shuffles for the norm reduction.
#include "nsd_device.h"

// fp32 results are rounded to fp32 and then to fp16, as the reference's
// `.to(tl.float16)` does; forbid contracting a multiply into a mixed fma
// that rounds straight to fp16.
#pragma clang fp contract(off)

namespace nsd {
namespace {

constexpr int D = kHeadDim;      // 128
constexpr int BS = kBlockTokens;  // 16
constexpr int kUnits = D / 8;     // 16-byte units per head row

// One workgroup per decode/verify row: K and V rows [Hkv, D] -> cache slot.
// Mirrors _fwd_kvcache_mgmt_decoding_kernel (kvcache_mgmt.py:50-79).
__global__ __launch_bounds__(256) void store_kv_decode_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, u32x4* __restrict__ kc,
    u32x4* __restrict__ vc, const int32_t* __restrict__ bt, int64_t bt_rows, int64_t bt_stride,
    const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ seq_lens, int64_t num_blocks,
    int num_layers, int layer, int hkv, int32_t* status) {
  const int64_t r = blockIdx.x;
  const int64_t sid = seq_ids[r];
  const int64_t pos = (int64_t)seq_lens[r] - 1;
  if (sid < 0 || sid >= bt_rows || pos < 0 || pos >= bt_stride * BS) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int64_t blk = bt[sid * bt_stride + pos / BS];
  if (blk < 0 || blk >= num_blocks) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_BLOCK);
    return;
  }
  // units of 16 B: slot base of head 0, then head stride BS*D halfs.
  const int64_t base = (((blk * num_layers + layer) * hkv) * BS + pos % BS) * kUnits;
  const int units = hkv * kUnits;
  for (int i = threadIdx.x; i < 2 * units; i += blockDim.x) {
    const bool isv = i >= units;
    const int u = isv ? i - units : i;
    const int h = u / kUnits, c = u % kUnits;
    const u32x4 val = (isv ? v : k)[r * units + u];
    (isv ? vc : kc)[base + (int64_t)h * BS * kUnits + c] = val;
  }
}

// grid (n_seqs, ceil(max_len/16)): one 16-token block of one prefill
// sequence.  Mirrors _fwd_kvcache_mgmt_prefill_kernel (kvcache_mgmt.py:10-48).
__global__ __launch_bounds__(256) void store_kv_prefill_kernel(
    const u32x4* __restrict__ k, const u32x4* __restrict__ v, u32x4* __restrict__ kc,
    u32x4* __restrict__ vc, const int32_t* __restrict__ bt, int64_t bt_rows, int64_t bt_stride,
    const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ start_locs,
    const int32_t* __restrict__ lens, int64_t num_blocks, int num_layers, int layer, int hkv,
    int32_t* status) {
  const int64_t s = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t len = lens[s];
  if (b * BS >= len) return;
  const int64_t sid = seq_ids[s];
  if (sid < 0 || sid >= bt_rows || len > bt_stride * BS) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int64_t blk = bt[sid * bt_stride + b];
  if (blk < 0 || blk >= num_blocks) {
    if (threadIdx.x == 0) flag_status(status, NSD_STATUS_BAD_BLOCK);
    return;
  }
  const int64_t tok0 = (int64_t)start_locs[s] + b * BS;
  const int ntok = (int)min<int64_t>(BS, len - b * BS);
  const int units = hkv * kUnits;  // per token
  const int64_t cbase = ((blk * num_layers + layer) * hkv) * BS * kUnits;
  for (int i = threadIdx.x; i < 2 * ntok * units; i += blockDim.x) {
    const bool isv = i >= ntok * units;
    const int u = isv ? i - ntok * units : i;
    const int t = u / units, hu = u % units;
    const int h = hu / kUnits, c = hu % kUnits;
    const u32x4 val = (isv ? v : k)[(tok0 + t) * units + hu];
    (isv ? vc : kc)[cbase + ((int64_t)h * BS + t) * kUnits + c] = val;
  }
}

// One wave per row of `hidden` values.  Mirrors _fwd_rmsnorm (rmsnorm.py:5-24).
__global__ __launch_bounds__(256) void rmsnorm_kernel(f16* __restrict__ x, const f16* __restrict__ w,
                                                      int64_t n_rows, int64_t hidden, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  f16* xr = x + row * hidden;
  float ss = 0.f;
  for (int64_t i = lane; i < hidden; i += kWave) {
    const float xv = (float)xr[i];
    ss += xv * xv;
  }
  ss = wave_sum(ss);
  const float rstd = 1.f / sqrtf(ss / (float)hidden + eps);
  for (int64_t i = lane; i < hidden; i += kWave) xr[i] = (f16)((float)xr[i] * rstd * (float)w[i]);
}

// One wave per (token, head); heads [0, Hq) rotate q, [Hq, Hq+Hkv) rotate k.
// Mirrors _fwd_rotary_embedding (rotary_emb.py:7-42) with fp32 arithmetic.
__global__ __launch_bounds__(256) void rope_kernel(f16* __restrict__ q, f16* __restrict__ k,
                                                   const f16* __restrict__ cos_t,
                                                   const f16* __restrict__ sin_t, int64_t n_tokens,
                                                   int hq, int hkv, int head_dim) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = hq + hkv;
  if (wid >= n_tokens * heads) return;
  const int64_t t = wid / heads;
  const int hd = (int)(wid % heads);
  f16* x = hd < hq ? q + (t * hq + hd) * head_dim : k + (t * hkv + (hd - hq)) * head_dim;
  const int half = head_dim / 2;
  for (int j = lane; j < half; j += kWave) {
    const float c = (float)cos_t[t * half + j], s = (float)sin_t[t * half + j];
    const float x0 = (float)x[j], x1 = (float)x[j + half];
    x[j] = (f16)(x0 * c - x1 * s);
    x[j + half] = (f16)(x0 * s + x1 * c);
  }
}

// Fused prologue: one wave per (row, head) over heads [q heads | k heads | v heads].
// q/k heads: rmsnorm (fp32, fp16 store) -> RoPE at seq_len-1; k in place, q
// into q_out (q itself, or a contiguous buffer when q is a strided slice of a
// fused q/k/v projection); k heads also write the rotated row to the cache
// slot; v heads copy to it.  Rows of q, k and v are q_stride, k_stride and
// v_stride elements apart.  Order and math of transformer_layer.py:114-145
// in one launch.  With `part` set, the fused q/k/v projection is given as
// fp32 split partials [splits][rows][q_stride] (q_stride = (hq + 2 hkv) D):
// each element is summed in split order and rounded to fp16 (the GEMM's
// output rounding) where it would be read, and k is written to the cache
// only.
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(
    const f16* q, int64_t q_stride, f16* q_out, f16* k, int64_t k_stride, const f16* __restrict__ v,
    int64_t v_stride,
    const f16* __restrict__ qw, const f16* __restrict__ kw, float eps,
    const f16* __restrict__ cos_c, const f16* __restrict__ sin_c, int64_t n_pos,
    f16* __restrict__ kc, f16* __restrict__ vc, const int32_t* __restrict__ bt, int64_t bt_rows,
    int64_t bt_stride, const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ seq_lens,
    int64_t n_rows, int64_t num_blocks, int num_layers, int layer, int hq, int hkv,
    int32_t* status, const float* __restrict__ part, int splits) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = hq + 2 * hkv;
  if (wid >= n_rows * heads) return;
  const int64_t r = wid / heads;
  const int hd = (int)(wid % heads);
  const int64_t pos = (int64_t)seq_lens[r] - 1;
  // element c of head hd of this row from the partials, as the GEMM's fp16 output
  const int64_t split_stride = n_rows * q_stride;
  auto from_part = [&](int c) {
    const float* p = part + r * q_stride + (int64_t)hd * D + c;
    float acc = p[0];
    for (int q2 = 1; q2 < splits; ++q2) acc += p[q2 * split_stride];
    return f16_of(acc);
  };

  int64_t slot = -1;  // element offset of (block, layer, head 0, pos % BS, 0)
  if (hd >= hq) {
    const int64_t sid = seq_ids[r];
    if (sid < 0 || sid >= bt_rows || pos < 0 || pos >= bt_stride * BS) {
      if (lane == 0) flag_status(status, NSD_STATUS_BAD_SEQ);
    } else {
      const int64_t blk = bt[sid * bt_stride + pos / BS];
      if (blk < 0 || blk >= num_blocks) {
        if (lane == 0) flag_status(status, NSD_STATUS_BAD_BLOCK);
      } else {
        slot = (((blk * num_layers + layer) * hkv) * BS + pos % BS) * D;
      }
    }
  }
  if (hd >= hq + hkv) {  // v head: bit-exact copy of 256 bytes
    const int h = hd - hq - hkv;
    if (slot >= 0) {
      if (part != nullptr) {
        f16* dst = vc + slot + (int64_t)h * BS * D;
        dst[lane] = from_part(lane);
        dst[lane + 64] = from_part(lane + 64);
      } else {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(v + r * v_stride + (int64_t)h * D);
        uint32_t* dst = reinterpret_cast<uint32_t*>(vc + slot + (int64_t)h * BS * D);
        dst[lane] = src[lane];
      }
    }
    return;
  }
  if (pos < 0 || pos >= n_pos) {
    if (lane == 0) flag_status(status, NSD_STATUS_BAD_POSITION);
    return;
  }
  const bool isk = hd >= hq;
  const int h = isk ? hd - hq : hd;
  f16* x = isk ? (part != nullptr ? nullptr : k + r * k_stride + (int64_t)h * D) : q_out + (r * hq + h) * D;
  const f16* w = isk ? kw : qw;
  float x0, x1;
  if (part != nullptr) {
    x0 = (float)from_part(lane);
    x1 = (float)from_part(lane + 64);
  } else {
    const f16* xin = isk ? k + r * k_stride + (int64_t)h * D : q + r * q_stride + (int64_t)h * D;
    x0 = (float)xin[lane];
    x1 = (float)xin[lane + 64];
  }
  if (w != nullptr) {
    const float ss = wave_sum(sq_pair(x0, x1));
    const float rstd = 1.f / sqrtf(ss / (float)D + eps);
    x0 = (float)f16_of(x0 * rstd * (float)w[lane]);
    x1 = (float)f16_of(x1 * rstd * (float)w[lane + 64]);
  }
  const float c = (float)cos_c[pos * (D / 2) + lane], s = (float)sin_c[pos * (D / 2) + lane];
  const f16 y0 = f16_of(rope_lo(x0, x1, c, s));
  const f16 y1 = f16_of(rope_hi(x0, x1, c, s));
  if (x != nullptr) {
    x[lane] = y0;
    x[lane + 64] = y1;
  }
  if (isk && slot >= 0) {
    f16* dst = kc + slot + (int64_t)h * BS * D;
    dst[lane] = y0;
    dst[lane + 64] = y1;
  }
}

int check_cache_shape(int num_layers, int layer, int num_kv_heads, int head_dim, int block_size,
                      int64_t num_blocks, const char* who) {
  if (head_dim != D) return fail(NSD_ERR_UNSUPPORTED, "%s: head_dim=%d (only 128)", who, head_dim);
  if (block_size != BS)
    return fail(NSD_ERR_UNSUPPORTED, "%s: block_size=%d (only 16)", who, block_size);
  if (num_kv_heads <= 0 || num_layers <= 0 || num_blocks <= 0)
    return fail(NSD_ERR_INVALID, "%s: bad cache shape (layers=%d, kv_heads=%d, blocks=%lld)", who,
                num_layers, num_kv_heads, (long long)num_blocks);
  if (layer < 0 || layer >= num_layers)
    return fail(NSD_ERR_INVALID, "%s: layer=%d outside [0, %d)", who, layer, num_layers);
  return NSD_OK;
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_rmsnorm_inplace(void* x, const void* w, int64_t n_rows, int64_t hidden,
                                   float eps, void* stream) {
  if (n_rows < 0 || hidden <= 0) return fail(NSD_ERR_INVALID, "rmsnorm: rows=%lld hidden=%lld",
                                             (long long)n_rows, (long long)hidden);
  if (n_rows == 0) return NSD_OK;
  if (x == nullptr || w == nullptr) return fail(NSD_ERR_INVALID, "rmsnorm: null pointer");
  const unsigned grid = (unsigned)((n_rows + 3) / 4);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                     static_cast<f16*>(x), static_cast<const f16*>(w), n_rows, hidden, eps);
  return launch_status("rmsnorm");
}

extern "C" int nsd_rotary_embedding_inplace(void* q, void* k, const void* cos_table,
                                            const void* sin_table, int64_t n_tokens,
                                            int num_q_heads, int num_kv_heads, int head_dim,
                                            void* stream) {
  if (n_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 2)
    return fail(NSD_ERR_INVALID, "rope: bad shape");
  if (n_tokens == 0) return NSD_OK;
  if (!q || !k || !cos_table || !sin_table) return fail(NSD_ERR_INVALID, "rope: null pointer");
  const int64_t waves = n_tokens * (num_q_heads + num_kv_heads);
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     as_stream(stream), static_cast<f16*>(q), static_cast<f16*>(k),
                     static_cast<const f16*>(cos_table), static_cast<const f16*>(sin_table),
                     n_tokens, num_q_heads, num_kv_heads, head_dim);
  return launch_status("rope");
}

extern "C" int nsd_store_kvcache(const void* k, const void* v, void* k_cache, void* v_cache,
                                 const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                                 const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                 int64_t num_blocks, int num_layers, int layer, int num_kv_heads,
                                 int head_dim, int block_size, int32_t* status, void* stream) {
  int rc = check_cache_shape(num_layers, layer, num_kv_heads, head_dim, block_size, num_blocks,
                             "store_kvcache");
  if (rc) return rc;
  if (n_rows < 0 || bt_rows <= 0 || bt_stride <= 0)
    return fail(NSD_ERR_INVALID, "store_kvcache: bad sizes");
  if (n_rows == 0) return NSD_OK;
  if (!k || !v || !k_cache || !v_cache || !block_table || !seq_ids || !seq_lens)
    return fail(NSD_ERR_INVALID, "store_kvcache: null pointer");
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(NSD_ERR_INVALID, "store_kvcache: k/v/cache must be 16-byte aligned");
  hipLaunchKernelGGL(store_kv_decode_kernel, dim3((unsigned)n_rows), dim3(256), 0,
                     as_stream(stream), static_cast<const u32x4*>(k),
                     static_cast<const u32x4*>(v), static_cast<u32x4*>(k_cache),
                     static_cast<u32x4*>(v_cache), block_table, bt_rows, bt_stride, seq_ids,
                     seq_lens, num_blocks, num_layers, layer, num_kv_heads, status);
  return launch_status("store_kvcache");
}

extern "C" int nsd_store_kvcache_prefill(const void* k, const void* v, void* k_cache,
                                         void* v_cache, const int32_t* block_table,
                                         int64_t bt_rows, int64_t bt_stride,
                                         const int32_t* seq_ids, const int32_t* start_locs,
                                         const int32_t* prefill_lens, int64_t n_seqs,
                                         int64_t max_prefill_len, int64_t num_blocks,
                                         int num_layers, int layer, int num_kv_heads, int head_dim,
                                         int block_size, int32_t* status, void* stream) {
  int rc = check_cache_shape(num_layers, layer, num_kv_heads, head_dim, block_size, num_blocks,
                             "store_kvcache_prefill");
  if (rc) return rc;
  if (n_seqs < 0 || max_prefill_len < 0 || bt_rows <= 0 || bt_stride <= 0)
    return fail(NSD_ERR_INVALID, "store_kvcache_prefill: bad sizes");
  if (n_seqs == 0 || max_prefill_len == 0) return NSD_OK;
  if (!k || !v || !k_cache || !v_cache || !block_table || !seq_ids || !start_locs || !prefill_lens)
    return fail(NSD_ERR_INVALID, "store_kvcache_prefill: null pointer");
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(NSD_ERR_INVALID, "store_kvcache_prefill: k/v/cache must be 16-byte aligned");
  const int64_t nb = (max_prefill_len + BS - 1) / BS;
  if (nb > 65535 || n_seqs > INT32_MAX)
    return fail(NSD_ERR_INVALID, "store_kvcache_prefill: grid too large");
  hipLaunchKernelGGL(store_kv_prefill_kernel, dim3((unsigned)n_seqs, (unsigned)nb), dim3(256), 0,
                     as_stream(stream), static_cast<const u32x4*>(k),
                     static_cast<const u32x4*>(v), static_cast<u32x4*>(k_cache),
                     static_cast<u32x4*>(v_cache), block_table, bt_rows, bt_stride, seq_ids,
                     start_locs, prefill_lens, num_blocks, num_layers, layer, num_kv_heads, status);
  return launch_status("store_kvcache_prefill");
}

static int qk_norm_rope_store_impl(const void* q, int64_t q_stride, void* q_out, void* k, int64_t k_stride,
                                   const void* v, int64_t v_stride, const void* q_norm_w, const void* k_norm_w,
                                   float eps, const void* cos_cache, const void* sin_cache, int64_t n_positions,
                                   void* k_cache, void* v_cache, const int32_t* block_table, int64_t bt_rows,
                                   int64_t bt_stride, const int32_t* seq_ids, const int32_t* seq_lens,
                                   int64_t n_rows, int64_t num_blocks, int num_layers, int layer,
                                   int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                   int32_t* status, void* stream, const float* part = nullptr, int splits = 1) {
  int rc = check_cache_shape(num_layers, layer, num_kv_heads, head_dim, block_size, num_blocks,
                             "qk_norm_rope_store");
  if (rc) return rc;
  if (num_q_heads <= 0 || n_rows < 0 || n_positions <= 0 || bt_rows <= 0 || bt_stride <= 0)
    return fail(NSD_ERR_INVALID, "qk_norm_rope_store: bad sizes");
  if (n_rows == 0) return NSD_OK;
  if ((part == nullptr && (!q || !k || !v)) || !q_out || !cos_cache || !sin_cache || !k_cache || !v_cache ||
      !block_table || !seq_ids || !seq_lens)
    return fail(NSD_ERR_INVALID, "qk_norm_rope_store: null pointer");
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(NSD_ERR_INVALID, "qk_norm_rope_store: pass both norm weights or neither");
  if (q_stride < (int64_t)num_q_heads * D || k_stride < (int64_t)num_kv_heads * D ||
      v_stride < (int64_t)num_kv_heads * D || (q_stride | k_stride | v_stride) & 1)
    return fail(NSD_ERR_INVALID, "qk_norm_rope_store: row strides must be even and cover the heads");
  const int64_t waves = n_rows * (num_q_heads + 2 * num_kv_heads);
  hipLaunchKernelGGL(qk_norm_rope_store_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     as_stream(stream), static_cast<const f16*>(q), q_stride, static_cast<f16*>(q_out),
                     static_cast<f16*>(k), k_stride, static_cast<const f16*>(v), v_stride,
                     static_cast<const f16*>(q_norm_w), static_cast<const f16*>(k_norm_w), eps,
                     static_cast<const f16*>(cos_cache), static_cast<const f16*>(sin_cache), n_positions,
                     static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), block_table, bt_rows, bt_stride,
                     seq_ids, seq_lens, n_rows, num_blocks, num_layers, layer, num_q_heads, num_kv_heads,
                     status, part, splits);
  return launch_status("qk_norm_rope_store");
}

extern "C" int nsd_qk_norm_rope_store(void* q, void* k, const void* v, const void* q_norm_w,
                                      const void* k_norm_w, float eps, const void* cos_cache,
                                      const void* sin_cache, int64_t n_positions, void* k_cache,
                                      void* v_cache, const int32_t* block_table, int64_t bt_rows,
                                      int64_t bt_stride, const int32_t* seq_ids,
                                      const int32_t* seq_lens, int64_t n_rows, int64_t num_blocks,
                                      int num_layers, int layer, int num_q_heads, int num_kv_heads,
                                      int head_dim, int block_size, int32_t* status,
                                      void* stream) {
  return qk_norm_rope_store_impl(q, (int64_t)num_q_heads * D, q, k, (int64_t)num_kv_heads * D, v,
                                 (int64_t)num_kv_heads * D, q_norm_w, k_norm_w, eps, cos_cache, sin_cache,
                                 n_positions, k_cache, v_cache, block_table, bt_rows, bt_stride, seq_ids, seq_lens,
                                 n_rows, num_blocks, num_layers, layer, num_q_heads, num_kv_heads, head_dim,
                                 block_size, status, stream);
}

extern "C" int nsd_qk_norm_rope_store_strided(const void* q, int64_t q_row_stride, void* q_out, void* k,
                                              int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                              const void* q_norm_w, const void* k_norm_w, float eps,
                                              const void* cos_cache, const void* sin_cache,
                                              int64_t n_positions, void* k_cache, void* v_cache,
                                              const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                                              const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                              int64_t num_blocks, int num_layers, int layer, int num_q_heads,
                                              int num_kv_heads, int head_dim, int block_size, int32_t* status,
                                              void* stream) {
  return qk_norm_rope_store_impl(q, q_row_stride, q_out, k, k_row_stride, v, v_row_stride, q_norm_w, k_norm_w, eps,
                                 cos_cache, sin_cache, n_positions, k_cache, v_cache, block_table, bt_rows,
                                 bt_stride, seq_ids, seq_lens, n_rows, num_blocks, num_layers, layer, num_q_heads,
                                 num_kv_heads, head_dim, block_size, status, stream);
}

extern "C" int nsd_qk_norm_rope_store_partials(const float* partials, int splits, void* q_out, const void* q_norm_w,
                                               const void* k_norm_w, float eps, const void* cos_cache,
                                               const void* sin_cache, int64_t n_positions, void* k_cache,
                                               void* v_cache, const int32_t* block_table, int64_t bt_rows,
                                               int64_t bt_stride, const int32_t* seq_ids, const int32_t* seq_lens,
                                               int64_t n_rows, int64_t num_blocks, int num_layers, int layer,
                                               int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                               int32_t* status, void* stream) {
  if (partials == nullptr || splits < 1 || splits > 8)
    return fail(NSD_ERR_INVALID, "qk_norm_rope_store_partials: %d splits (1..8) of partials", splits);
  const int64_t row_w = (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim;
  return qk_norm_rope_store_impl(nullptr, row_w, q_out, nullptr, row_w, nullptr, row_w, q_norm_w, k_norm_w, eps,
                                 cos_cache, sin_cache, n_positions, k_cache, v_cache, block_table, bt_rows,
                                 bt_stride, seq_ids, seq_lens, n_rows, num_blocks, num_layers, layer, num_q_heads,
                                 num_kv_heads, head_dim, block_size, status, stream, partials, splits);
}
