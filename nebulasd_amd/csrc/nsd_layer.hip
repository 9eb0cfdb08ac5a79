// The rest of the transformer layer around the attention path, for gfx950
// (MI355X): the element-wise kernels between the GEMMs, and the post-layer
// lm_head + argmax.
//
//   nsd_fused_add_rmsnorm_inplace -- swiftLLM/swiftllm/worker/kernels/rmsnorm.py:39-89:
//     r = x + r (fp16), x = fp16(fp32(r) * rstd * w), rstd over the row.
//   nsd_silu_and_mul_inplace -- swiftLLM/swiftllm/worker/kernels/silu_and_mul.py:5-34:
//     x[:, :I] = x[:, :I] * fp16(silu(fp32(x[:, I:2I]))) (first half "up",
//     second half "gate", the order of the stacked up_gate_proj weight).
//   nsd_lm_head_argmax -- swiftLLM/swiftllm/worker/layers/post_layer.py:70-71:
//     token[r] = argmax_v fp16(x[r] . W[v]) (torch.argmax: first maximum; NaN
//     counts as the maximum), without writing the [rows, vocab] logits.
//   nsd_argmax_rows -- the argmax alone over fp16 logits [rows, vocab].
//
// The element-wise kernels are HBM-bound (one read and one write of every
// element) and latency-bound at decode sizes.  lm_head + argmax is a skinny
// GEMM: the [vocab, hidden] weight (1.24 GB for Qwen3-8B) is streamed once per
// call at HBM rate by 16x16x32 MFMAs whose other operand (at most 128 rows of
// x) is staged through LDS; each workgroup folds its logits into one 64-bit
// key per row, (ordered fp16 value << 32) | ~index, merged with atomicMax so
// the largest value and then the smallest index win.
#include <algorithm>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxNormVecs = 4;  // 16-byte vectors per thread: hidden <= 8192

typedef __attribute__((address_space(1))) u32x4 gbl_u32x4;

__device__ inline f16x8 as_h8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ inline u32x4 as_u4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

template <int VPT>
__global__ void __launch_bounds__(kNormThreads)
fused_add_rmsnorm_kernel(f16* __restrict__ x, f16* __restrict__ res, const f16* __restrict__ w, int nvec,
                         int hidden, float eps) {
  __shared__ float s_part[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  u32x4* xr = reinterpret_cast<u32x4*>(x + row * hidden);
  u32x4* rr = reinterpret_cast<u32x4*>(res + row * hidden);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  f16x8 s[VPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    if (i < nvec) {
      const f16x8 a = as_h8(xr[i]), b = as_h8(rr[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[j][e] = (f16)((float)a[e] + (float)b[e]);  // one fp16 rounding, as an fp16 add
        const float f = (float)s[j][e];
        ss += f * f;
      }
      rr[i] = as_u4(s[j]);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < kNormThreads / kWave; ++q) tot += s_part[q];
  const float rstd = 1.f / sqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    if (i < nvec) {
      const f16x8 wv = as_h8(wr[i]);
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f16)((float)s[j][e] * rstd * (float)wv[e]);
      xr[i] = as_u4(o);
    }
  }
}

// One thread per 8 outputs.
__global__ void __launch_bounds__(256)
silu_and_mul_kernel(f16* __restrict__ x, int64_t n_tokens, int inter, int64_t total_vecs) {
  const int vpr = inter / 8;
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < total_vecs; v += (int64_t)gridDim.x * 256) {
    const int64_t t = v / vpr;
    const int j = (int)(v - t * vpr);
    u32x4* up_p = reinterpret_cast<u32x4*>(x + t * 2 * inter) + j;
    const u32x4* gate_p = reinterpret_cast<const u32x4*>(x + t * 2 * inter + inter) + j;
    const f16x8 up = as_h8(*up_p), gate = as_h8(*gate_p);
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = (float)gate[e];
      const f16 sg = (f16)(g / (1.f + expf(-g)));
      o[e] = (f16)((float)up[e] * (float)sg);  // exact product, one fp16 rounding
    }
    *up_p = as_u4(o);
  }
}

// ---- argmax keys ----------------------------------------------------------

// Order-preserving 16-bit code of an fp16 value; NaN above everything, -0 as +0.
__device__ inline uint32_t order16(f16 v) {
  uint32_t b = __builtin_bit_cast(uint16_t, v);
  if ((b & 0x7c00u) == 0x7c00u && (b & 0x03ffu)) return 0xffffu;  // NaN
  if (b == 0x8000u) b = 0;                                          // -0 == +0
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
// Larger key = larger value, then smaller index.  Never 0 for a real entry.
__device__ inline uint64_t argmax_key(f16 v, uint32_t index) {
  return ((uint64_t)(order16(v) + 1) << 32) | (uint64_t)(0xffffffffu - index);
}
__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ inline uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, kWave), hi = __shfl_xor((uint32_t)(v >> 32), m, kWave);
  return ((uint64_t)hi << 32) | lo;
}

// tokens[r] = index of the key; keys[r] back to 0 for the next call.
__global__ void __launch_bounds__(256) argmax_finalize_kernel(uint64_t* keys, int64_t* tokens, int rows) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const uint64_t k = keys[r];
  tokens[r] = k ? (int64_t)(0xffffffffu - (uint32_t)k) : -1;
  keys[r] = 0;
}

// One workgroup per row: argmax over fp16 logits.
__global__ void __launch_bounds__(256)
argmax_rows_kernel(const f16* __restrict__ logits, int64_t vocab, int64_t* tokens) {
  __shared__ uint64_t s_best[256 / kWave];
  const f16* lr = logits + (int64_t)blockIdx.x * vocab;
  uint64_t best = 0;
  for (int64_t v = threadIdx.x; v < vocab; v += 256) best = umax64(best, argmax_key(lr[v], (uint32_t)v));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) best = umax64(best, shfl_xor64(best, m));
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < 256 / kWave; ++q) best = umax64(best, s_best[q]);
    best = umax64(best, s_best[0]);
    tokens[blockIdx.x] = (int64_t)(0xffffffffu - (uint32_t)best);
  }
}

// ---- lm_head GEMV + argmax -----------------------------------------------

constexpr int kLmWaves = 8;
constexpr int kLmThreads = kLmWaves * kWave;
constexpr int kLmTilesPerWave = 2;                         // 16-row vocab tiles per wave
constexpr int kLmVocabPerWg = kLmWaves * kLmTilesPerWave * 16;  // 256
constexpr int kLmK = 128;                                  // k-chunk staged per step
constexpr int kLmRowBytes = kLmK * 2 + 16;                 // 272: rows 4 banks apart

template <int NRT>
constexpr int lm_lds_bytes() { return 2 * NRT * 16 * kLmRowBytes; }

// x chunk [NRT*16 rows][kLmK] -> LDS; rows >= n_rows are not written (their
// columns are never read back).  16 bytes per thread per pass.
template <int NRT>
__device__ inline void stage_x(lds_char* dst, const f16* x, int n_rows, int hidden, int k0) {
  constexpr int kVecs = NRT * 16 * (kLmK / 8);
  for (int i = threadIdx.x; i < kVecs; i += kLmThreads) {
    const int r = i / (kLmK / 8), c = i % (kLmK / 8);
    if (r < n_rows) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(x + (int64_t)r * hidden + k0 + c * 8);
      *reinterpret_cast<lds_u32x4*>(dst + r * kLmRowBytes + c * 16) = v;
    }
  }
}

// Workgroup: 256 vocab rows (8 waves x 2 tiles of 16) against NRT*16 rows of
// x.  Lane (i, g) of a wave loads 64 contiguous bytes of W row (tile row i),
// k = k0 + 32g .. 32g+31, and feeds them to the 4 MFMA steps s as elements
// 32g + 8s .. +7; the x fragment of row (rt*16 + i) uses the same k order,
// so every step's dot products cover the chunk exactly once.
template <int NRT>
__global__ void __launch_bounds__(kLmThreads)
lm_head_argmax_kernel(const f16* __restrict__ x, const f16* __restrict__ w, int n_rows, int hidden,
                      int64_t vocab, uint64_t* __restrict__ keys) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_char* lds = (lds_char*)lds_raw;
  __shared__ uint64_t s_best[kLmWaves][NRT * 16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t vbase = (int64_t)blockIdx.x * kLmVocabPerWg + wv * (kLmTilesPerWave * 16);
  const gbl_u32x4* wp[kLmTilesPerWave];
  bool wok[kLmTilesPerWave];
#pragma unroll
  for (int a = 0; a < kLmTilesPerWave; ++a) {
    const int64_t v = vbase + a * 16 + li;
    wok[a] = v < vocab;
    wp[a] = (const gbl_u32x4*)(uintptr_t)(w + (wok[a] ? v : 0) * (int64_t)hidden + lg * 32);
  }
  f32x4 acc[kLmTilesPerWave][NRT];
#pragma unroll
  for (int a = 0; a < kLmTilesPerWave; ++a)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) acc[a][rt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int chunks = hidden / kLmK;
  u32x4 wcur[kLmTilesPerWave][4], wnext[kLmTilesPerWave][4];
#pragma unroll
  for (int a = 0; a < kLmTilesPerWave; ++a)
#pragma unroll
    for (int s = 0; s < 4; ++s) wcur[a][s] = wok[a] ? __builtin_nontemporal_load(wp[a] + s) : u32x4{0, 0, 0, 0};
  stage_x<NRT>(lds, x, n_rows, hidden, 0);
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    lds_char* cur = lds + (c & 1) * (NRT * 16 * kLmRowBytes);
    lds_char* nxt = lds + ((c + 1) & 1) * (NRT * 16 * kLmRowBytes);
    if (c + 1 < chunks) {
#pragma unroll
      for (int a = 0; a < kLmTilesPerWave; ++a)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          wnext[a][s] = wok[a] ? __builtin_nontemporal_load(wp[a] + (c + 1) * (kLmK / 8) + s) : u32x4{0, 0, 0, 0};
      stage_x<NRT>(nxt, x, n_rows, hidden, (c + 1) * kLmK);
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const lds_char* xb = cur + (rt * 16 + li) * kLmRowBytes + lg * 64;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f16x8 bx = as_h8(*reinterpret_cast<const lds_u32x4*>(xb + s * 16));
#pragma unroll
        for (int a = 0; a < kLmTilesPerWave; ++a) acc[a][rt] = mfma_k32(as_h8(wcur[a][s]), bx, acc[a][rt]);
      }
    }
    __syncthreads();  // every wave is done with `cur` before it is refilled
    if (c + 1 < chunks) {
#pragma unroll
      for (int a = 0; a < kLmTilesPerWave; ++a)
#pragma unroll
        for (int s = 0; s < 4; ++s) wcur[a][s] = wnext[a][s];
    }
  }
  // acc[a][rt][e]: logit of vocab row vbase + a*16 + 4*lg + e, x row rt*16 + li.
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    uint64_t best = 0;
#pragma unroll
    for (int a = 0; a < kLmTilesPerWave; ++a)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t v = vbase + a * 16 + 4 * lg + e;
        if (v < vocab) best = umax64(best, argmax_key((f16)acc[a][rt][e], (uint32_t)v));
      }
    best = umax64(best, shfl_xor64(best, 16));
    best = umax64(best, shfl_xor64(best, 32));
    if (lg == 0) s_best[wv][rt * 16 + li] = best;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < n_rows; r += kLmThreads) {
    uint64_t best = 0;
#pragma unroll
    for (int q = 0; q < kLmWaves; ++q) best = umax64(best, s_best[q][r]);
    if (best) atomicMax(reinterpret_cast<unsigned long long*>(keys + r), (unsigned long long)best);
  }
}

template <int NRT>
void launch_lm(const f16* x, const f16* w, int rows, int hidden, int64_t vocab, uint64_t* keys, hipStream_t s) {
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_head_argmax_kernel<NRT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, lm_lds_bytes<NRT>()) == hipSuccess;
  }();
  (void)attr;
  const unsigned grid = (unsigned)((vocab + kLmVocabPerWg - 1) / kLmVocabPerWg);
  hipLaunchKernelGGL(lm_head_argmax_kernel<NRT>, dim3(grid), dim3(kLmThreads), lm_lds_bytes<NRT>(), s, x, w, rows,
                     hidden, vocab, keys);
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_fused_add_rmsnorm_inplace(void* x, void* residual, const void* weight, int64_t n_rows,
                                             int64_t hidden, float eps, void* stream) {
  if (n_rows < 0 || hidden <= 0) return fail(NSD_ERR_INVALID, "fused_add_rmsnorm: bad shape");
  if (n_rows == 0) return NSD_OK;
  if (!x || !residual || !weight) return fail(NSD_ERR_INVALID, "fused_add_rmsnorm: null pointer");
  if (hidden % 8 || hidden > 8 * kNormThreads * kMaxNormVecs)
    return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: hidden=%lld (need a multiple of 8, <= %d)",
                (long long)hidden, 8 * kNormThreads * kMaxNormVecs);
  if (!aligned16(x) || !aligned16(residual) || !aligned16(weight))
    return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: pointers must be 16-byte aligned");
  if (n_rows > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: too many rows");
  const int nvec = (int)(hidden / 8);
  const int vpt = (nvec + kNormThreads - 1) / kNormThreads;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)n_rows), dim3(kNormThreads), 0, as_stream(stream),
                       static_cast<f16*>(x), static_cast<f16*>(residual), static_cast<const f16*>(weight), nvec,
                       (int)hidden, eps);
  };
  switch (vpt) {
    case 1: go(fused_add_rmsnorm_kernel<1>); break;
    case 2: go(fused_add_rmsnorm_kernel<2>); break;
    case 3: go(fused_add_rmsnorm_kernel<3>); break;
    default: go(fused_add_rmsnorm_kernel<4>); break;
  }
  return launch_status("fused_add_rmsnorm");
}

extern "C" int nsd_silu_and_mul_inplace(void* x, int64_t n_tokens, int64_t inter_dim, void* stream) {
  if (n_tokens < 0 || inter_dim <= 0) return fail(NSD_ERR_INVALID, "silu_and_mul: bad shape");
  if (n_tokens == 0) return NSD_OK;
  if (!x) return fail(NSD_ERR_INVALID, "silu_and_mul: null pointer");
  if (inter_dim % 8 || inter_dim > INT32_MAX / 2)
    return fail(NSD_ERR_UNSUPPORTED, "silu_and_mul: inter_dim=%lld (need a multiple of 8)", (long long)inter_dim);
  if (!aligned16(x)) return fail(NSD_ERR_UNSUPPORTED, "silu_and_mul: x must be 16-byte aligned");
  const int64_t total = n_tokens * (inter_dim / 8);
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 256 * 16);
  hipLaunchKernelGGL(silu_and_mul_kernel, dim3(grid), dim3(256), 0, as_stream(stream), static_cast<f16*>(x), n_tokens,
                     (int)inter_dim, total);
  return launch_status("silu_and_mul");
}

extern "C" int nsd_lm_head_argmax(const void* x, const void* lm_head, int64_t n_rows, int64_t hidden,
                                  int64_t vocab, uint64_t* keys, int64_t* tokens, void* stream) {
  if (n_rows < 0 || hidden <= 0 || vocab <= 0) return fail(NSD_ERR_INVALID, "lm_head_argmax: bad shape");
  if (n_rows == 0) return NSD_OK;
  if (!x || !lm_head || !keys || !tokens) return fail(NSD_ERR_INVALID, "lm_head_argmax: null pointer");
  if (hidden % kLmK || hidden > INT32_MAX)
    return fail(NSD_ERR_UNSUPPORTED, "lm_head_argmax: hidden=%lld (need a multiple of %d)", (long long)hidden, kLmK);
  if (vocab > (int64_t)UINT32_MAX - 1) return fail(NSD_ERR_UNSUPPORTED, "lm_head_argmax: vocab too large");
  if (!aligned16(x) || !aligned16(lm_head)) return fail(NSD_ERR_UNSUPPORTED, "lm_head_argmax: pointers must be 16-byte aligned");
  const hipStream_t s = as_stream(stream);
  const f16* xp = static_cast<const f16*>(x);
  const f16* wp = static_cast<const f16*>(lm_head);
  // Rows in passes of at most 128 (each pass streams the weight once).
  for (int64_t r0 = 0; r0 < n_rows; r0 += 128) {
    const int rows = (int)std::min<int64_t>(128, n_rows - r0);
    const f16* xr = xp + r0 * hidden;
    uint64_t* kr = keys + r0;
    if (rows <= 16) launch_lm<1>(xr, wp, rows, (int)hidden, vocab, kr, s);
    else if (rows <= 32) launch_lm<2>(xr, wp, rows, (int)hidden, vocab, kr, s);
    else if (rows <= 64) launch_lm<4>(xr, wp, rows, (int)hidden, vocab, kr, s);
    else launch_lm<8>(xr, wp, rows, (int)hidden, vocab, kr, s);
    if (int e = launch_status("lm_head_argmax")) return e;
  }
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)((n_rows + 255) / 256)), dim3(256), 0, s, keys, tokens,
                     (int)n_rows);
  return launch_status("lm_head_argmax finalize");
}

extern "C" int nsd_argmax_rows(const void* logits, int64_t n_rows, int64_t vocab, int64_t* tokens, void* stream) {
  if (n_rows < 0 || vocab <= 0) return fail(NSD_ERR_INVALID, "argmax_rows: bad shape");
  if (n_rows == 0) return NSD_OK;
  if (!logits || !tokens) return fail(NSD_ERR_INVALID, "argmax_rows: null pointer");
  if (n_rows > INT32_MAX || vocab > (int64_t)UINT32_MAX - 1) return fail(NSD_ERR_UNSUPPORTED, "argmax_rows: too large");
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)n_rows), dim3(256), 0, as_stream(stream),
                     static_cast<const f16*>(logits), vocab, tokens);
  return launch_status("argmax_rows");
}
