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

constexpr int kLmK = 128;                                       // k-chunk per step
constexpr int kLmRowBytes = kLmK * 2 + 16;                      // 272: rows 4 banks apart
constexpr int kLmMaxRowTiles = 8;                               // <= 128 rows of x per pass

template <int NRT>
constexpr int lm_lds_bytes() { return 2 * NRT * 16 * kLmRowBytes; }

// Workgroup: NW*TPW*16 vocab rows (NW waves x TPW tiles of 16) against
// NRT*16 rows of x.  MFMA step s of chunk k0 covers k = k0 + 32s .. +31: lane (i, g) loads
// W row (tile row i) elements 32s + 8g .. +7, so the 4 lanes of a row read
// 64 contiguous bytes per load instruction (whole 64-byte segments), and the
// x fragment of row (rt*16 + i) is the same 8 elements from LDS.
//
// Pipeline per chunk c: x of chunk c+1 is loaded into registers first, then
// W of chunk c+1, then chunk c's MFMAs run (x from LDS, W from registers),
// then the x registers go to the other LDS buffer.  Loads complete in
// order, so that LDS store waits for the x loads only and the weight loads
// stay in flight across the MFMAs and the barrier.
//
// skinny_mainloop: the wave's weight rows [vbase, vbase + TPW*16) (rows past
// n_out read as zero) against x rows [0, n_rows) (row stride x_stride) over
// the k chunks [kc0, kc0 + chunks) of 128; sums accumulate into acc.  Every
// thread of the workgroup calls it with the same chunk range (it holds
// barriers).
template <int NRT, int TPW, int NW, int PD>
__device__ __forceinline__ void skinny_mainloop(const f16* __restrict__ x, int64_t x_stride,
                                                const f16* __restrict__ w, int n_rows, int hidden,
                                                int64_t vbase, int64_t n_out, int kc0, int chunks,
                                                lds_char* lds, f32x4 (&acc)[TPW][NRT]) {
  constexpr int kLmThreads = NW * kWave;
  constexpr int kBuf = NRT * 16 * kLmRowBytes;
  constexpr int kXRowStep = kLmThreads / (kLmK / 8);      // x rows one pass of the workgroup covers
  constexpr int kXv = (NRT * 16 + kXRowStep - 1) / kXRowStep;  // 16-byte x vectors per thread per chunk
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const gbl_u32x4* wp[TPW];
  bool wok[TPW];
#pragma unroll
  for (int a = 0; a < TPW; ++a) {
    const int64_t v = vbase + a * 16 + li;
    wok[a] = v < n_out;
    wp[a] = (const gbl_u32x4*)(uintptr_t)(w + (wok[a] ? v : 0) * (int64_t)hidden + (int64_t)kc0 * kLmK + lg * 8);
  }
  // x vector j of this thread: row xr0 + j*kXRowStep of the chunk, 16-byte
  // column threadIdx.x % 16.
  const int xc = threadIdx.x % (kLmK / 8), xr0 = threadIdx.x / (kLmK / 8);
  const f16* xk = x + (int64_t)kc0 * kLmK;
  auto load_x = [&](u32x4 (&xv)[kXv], int k0) {
#pragma unroll
    for (int j = 0; j < kXv; ++j)
      if (xr0 + j * kXRowStep < n_rows)
        xv[j] = *reinterpret_cast<const u32x4*>(xk + (int64_t)(xr0 + j * kXRowStep) * x_stride + k0 + xc * 8);
  };
  auto store_x = [&](lds_char* dst, const u32x4 (&xv)[kXv]) {
#pragma unroll
    for (int j = 0; j < kXv; ++j)
      if (xr0 + j * kXRowStep < n_rows)
        *reinterpret_cast<lds_u32x4*>(dst + (xr0 + j * kXRowStep) * kLmRowBytes + xc * 16) = xv[j];
  };
  auto load_w = [&](u32x4 (&wr)[TPW][4], int c) {
#pragma unroll
    for (int a = 0; a < TPW; ++a)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        wr[a][s] = wok[a] ? __builtin_nontemporal_load(wp[a] + c * (kLmK / 8) + s * 4) : u32x4{0, 0, 0, 0};
  };

  u32x4 xv[kXv];
  // Register ring of weight chunks: chunk c computes from wr[c % R] while
  // chunks c+1 .. c+PD load into the others (static indices: the loop is
  // unrolled by R, so no register moves wait on loads in flight).
  constexpr int R = PD + 1;
  u32x4 wr[R][TPW][4];
  load_x(xv, 0);
  static_for<PD>([&](auto u) {
    constexpr int k = decltype(u)::value;
    if (k < chunks) load_w(wr[k], k);
  });
  store_x(lds, xv);
  __syncthreads();
  for (int c0 = 0; c0 < chunks; c0 += R) {
    static_for<R>([&](auto u) {
      constexpr int k = decltype(u)::value;
      const int c = c0 + k;
      if (c < chunks) {
        const lds_char* cur = lds + (c & 1) * kBuf;
        lds_char* nxt = lds + ((c + 1) & 1) * kBuf;
        const bool more = c + 1 < chunks;
        if (more) load_x(xv, (c + 1) * kLmK);
        if (c + PD < chunks) load_w(wr[(k + PD) % R], c + PD);
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          const lds_char* xb = cur + (rt * 16 + li) * kLmRowBytes + lg * 16;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const f16x8 bx = as_h8(*reinterpret_cast<const lds_u32x4*>(xb + s * 64));
#pragma unroll
            for (int a = 0; a < TPW; ++a) acc[a][rt] = mfma_k32(as_h8(wr[k][a][s]), bx, acc[a][rt]);
          }
        }
        if (more) store_x(nxt, xv);  // `nxt` was last read in chunk c-1, before the previous barrier
        __syncthreads();
      }
    });
  }
}

template <int NRT, int TPW, int NW, int WPE, int PD>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
lm_head_argmax_kernel(const f16* __restrict__ x, const f16* __restrict__ w, int n_rows, int hidden,
                      int64_t vocab, uint64_t* __restrict__ keys) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_char* lds = (lds_char*)lds_raw;
  constexpr int kLmThreads = NW * kWave;
  __shared__ uint64_t s_best[NW][NRT * 16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t vbase = (int64_t)blockIdx.x * (NW * TPW * 16) + wv * (TPW * 16);
  f32x4 acc[TPW][NRT];
#pragma unroll
  for (int a = 0; a < TPW; ++a)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) acc[a][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  skinny_mainloop<NRT, TPW, NW, PD>(x, hidden, w, n_rows, hidden, vbase, vocab, 0, hidden / kLmK, lds, acc);
  // acc[a][rt][e]: logit of vocab row vbase + a*16 + 4*lg + e, x row rt*16 + li.
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    uint64_t best = 0;
#pragma unroll
    for (int a = 0; a < TPW; ++a)
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
    for (int q = 0; q < NW; ++q) best = umax64(best, s_best[q][r]);
    if (best) atomicMax(reinterpret_cast<unsigned long long*>(keys + r), (unsigned long long)best);
  }
}

// Per row-tile count (1..8): vocab tiles per wave, waves per workgroup, the
// waves per SIMD the register budget is fitted to, and the weight prefetch
// distance in chunks (2 measured slower everywhere: it spills or costs a
// wave per SIMD).  Measured on MI355X
// over 1..128 rows of the 151,936 x 4096 and x 1024 lm_heads; every entry
// compiles without spills.  Two vocab tiles per wave halve the x traffic
// from LDS per weight byte while the row tiles leave registers for three or
// four waves per SIMD; beyond five row tiles one tile per wave and
// eight-wave workgroups (128 vocab rows per x chunk staged) win.
struct LmCfg { int tpw, nw, wpe, pd; };
constexpr LmCfg kLmTable[kLmMaxRowTiles] = {{2, 4, 4, 1}, {2, 4, 4, 1}, {2, 4, 4, 1}, {2, 4, 3, 1},
                                            {2, 4, 3, 1}, {1, 8, 3, 1}, {1, 8, 3, 1}, {1, 8, 3, 1}};

template <int NRT>
void launch_lm(const f16* x, const f16* w, int rows, int hidden, int64_t vocab, uint64_t* keys, hipStream_t s) {
  constexpr int TPW = kLmTable[NRT - 1].tpw, NW = kLmTable[NRT - 1].nw, WPE = kLmTable[NRT - 1].wpe;
  constexpr int PD = kLmTable[NRT - 1].pd;
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_head_argmax_kernel<NRT, TPW, NW, WPE, PD>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, lm_lds_bytes<NRT>()) == hipSuccess;
  }();
  (void)attr;
  constexpr int kVocabPerWg = NW * TPW * 16;
  const unsigned grid = (unsigned)((vocab + kVocabPerWg - 1) / kVocabPerWg);
  hipLaunchKernelGGL((lm_head_argmax_kernel<NRT, TPW, NW, WPE, PD>), dim3(grid), dim3(NW * 64), lm_lds_bytes<NRT>(), s,
                     x, w, rows, hidden, vocab, keys);
}

template <int... N>
void launch_lm_rows(std::integer_sequence<int, N...>, int nrt, const f16* x, const f16* w, int rows, int hidden,
                    int64_t vocab, uint64_t* keys, hipStream_t s) {
  ((nrt == N + 1 ? launch_lm<N + 1>(x, w, rows, hidden, vocab, keys, s) : void()), ...);
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
  // Rows in passes of at most 128 (each pass streams the weight once), each
  // pass with as many 16-row tiles as it needs.
  for (int64_t r0 = 0; r0 < n_rows; r0 += 128) {
    const int rows = (int)std::min<int64_t>(128, n_rows - r0);
    const f16* xr = xp + r0 * hidden;
    uint64_t* kr = keys + r0;
    launch_lm_rows(std::make_integer_sequence<int, kLmMaxRowTiles>{}, (rows + 15) / 16, xr, wp, rows, (int)hidden,
                   vocab, kr, s);
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
