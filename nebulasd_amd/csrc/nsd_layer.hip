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
// pass of at most 128 rows of x through an LDS ring by 16x16x32 MFMAs; each
// wave folds its logits into one 64-bit key per row, (ordered fp16 value <<
// 32) | ~index, merged with atomicMax so the largest value and then the
// smallest index win.
#include <algorithm>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxNormVecs = 4;  // 16-byte vectors per thread: hidden <= 8192

typedef __attribute__((address_space(1))) u32x4 gbl_u32x4;

__device__ inline f16x8 as_h8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ inline u32x4 as_u4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

// With `part` set, x is the projection whose fp32 split partials part holds
// ([splits][rows][hidden]): summed in split order and rounded to fp16 (the
// GEMM's output rounding) in place of reading x; the normalised row is
// written to x either way.
template <int VPT>
__global__ void __launch_bounds__(kNormThreads)
fused_add_rmsnorm_kernel(f16* __restrict__ x, f16* __restrict__ res, const f16* __restrict__ w, int nvec,
                         int hidden, float eps, const float* __restrict__ part, int splits, int64_t split_stride) {
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
      f16x8 a;
      if (part != nullptr) {
        const float* p = part + row * hidden + 8 * i;
        f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
        for (int q = 1; q < splits; ++q) {
          lo += *reinterpret_cast<const f32x4*>(p + q * split_stride);
          hi += *reinterpret_cast<const f32x4*>(p + q * split_stride + 4);
        }
        a = f16x8{(f16)lo[0], (f16)lo[1], (f16)lo[2], (f16)lo[3], (f16)hi[0], (f16)hi[1], (f16)hi[2], (f16)hi[3]};
      } else {
        a = as_h8(xr[i]);
      }
      const f16x8 b = as_h8(rr[i]);
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

constexpr int kLmK = 128;  // hidden must be a multiple of this (one ring step of k)

// lm_head GEMV + argmax through an LDS ring (1..128 rows of x per pass).
//
// One workgroup per CU streams a balanced range of 16-row vocab tiles, in
// groups of eight tiles (128 vocab rows), in k steps of 128 (256 bytes of a
// row).  Four producer waves bring each step's weight chunk (128 rows x
// 256 B) from memory straight into a slot of a kRgRing-slot LDS ring by
// global_load_lds_dwordx4, four rows x 256 B per instruction: whole 256-byte
// runs of a row per instruction, against the 64-byte pieces of 16 rows that
// a 16x16 MFMA operand loaded into registers gets (measured read rates over
// the Qwen3-8B lm_head: 5.9 against 5.1 TB/s), with kRgRing - 1 steps in
// flight.  The 16-byte chunk q of slot row r sits at chunk q ^ (r & 15), so
// the sixteen rows an operand read touches hit distinct banks.  Consumer
// wave (rt, h) holds x row tile rt in registers (its own loads, three steps
// ahead; x is a few hundred KB and stays in L2), multiplies it by vocab
// tiles [h*TPW, (h+1)*TPW) of the group (A = weight rows, B = x rows, as in
// the register-staged kernel, so every sum runs in the same k order), folds
// its logits into one running key per x row at the end of each group, and
// merges it with one atomicMax at the end.  The two roles never wait on
// each other's loads: each wave's vmcnt counts its own kind only.
// Out-of-range weight rows are fetched from one fixed row (an L2 hit) and
// never used.  Measured on MI355X, Qwen3-8B lm_head: 243 us at 1 row and
// 253 us at 80 (against 266 / 323 for the register-staged kernel).
constexpr int kRgTiles = 8;                             // vocab tiles per group
constexpr int kRgRowBytes = 256;                        // a row's 128 k of one step
constexpr int kRgRing = 4;                              // ring slots: three steps in flight
constexpr int kRgSlot = kRgTiles * 16 * kRgRowBytes;    // 32 KB
constexpr int kRgLds = kRgRing * kRgSlot;
constexpr int kRgProducers = 4;
constexpr int kRgInsPerWave = kRgTiles * 16 / 4 / kRgProducers;  // DMA instructions per producer per step
constexpr int kRgXAhead = 3;                            // steps of x a consumer loads ahead
constexpr int kRgMaxRowTiles = 8;                       // up to 128 rows of x per pass
static_assert(kRgLds <= 160 * 1024, "ring fits the CU's LDS");
static_assert(kRgInsPerWave * (kRgRing - 1) <= 63, "vmcnt range");

// Consumer waves per x row tile: 8, 4, then 1 for 3..8 row tiles (a second
// wave per tile would load the tile's x again: measured slower at 64-80 rows).
template <int NRT>
constexpr int rg_split() { return NRT == 1 ? 8 : NRT == 2 ? 4 : 1; }
template <int NRT>
constexpr int rg_threads() { return (kRgProducers + NRT * rg_split<NRT>()) * kWave; }

__device__ inline void rg_dma(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(lds_addr), "v"(src) : "memory", "m0");
}
template <int N>
__device__ inline void rg_wait_n() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}
// A producer's loads of all but its n most recent steps are complete
// (0 <= n <= kRgRing - 2).
template <int N>
__device__ inline void rg_wait_steps_n() {
  if constexpr (N * kRgInsPerWave <= 63) rg_wait_n<N * kRgInsPerWave>();
  else rg_wait_n<0>();
}
__device__ inline void rg_wait_steps(int n) {
  static_assert(kRgRing <= 6, "wait table");
  switch (n) {
    case 1: rg_wait_steps_n<1>(); break;
    case 2: rg_wait_steps_n<2>(); break;
    case 3: rg_wait_steps_n<3>(); break;
    case 4: rg_wait_steps_n<4>(); break;
    default: rg_wait_n<0>(); break;
  }
}

template <int NRT>
__global__ void __launch_bounds__(rg_threads<NRT>())
lm_ring_kernel(const f16* __restrict__ x, const f16* __restrict__ w, int n_rows, int hidden, int64_t vocab,
               uint64_t* __restrict__ keys) {
  constexpr int SPLIT = rg_split<NRT>(), TPW = kRgTiles / SPLIT, XR = kRgXAhead + 1;
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool producer = wv < kRgProducers;
  const int cw = wv - kRgProducers;  // consumer index
  const int rt = cw % NRT, h = cw / NRT;
  const int64_t n_tiles = (vocab + 15) / 16;
  const int64_t t0 = (int64_t)blockIdx.x * n_tiles / gridDim.x;
  const int64_t t1 = (int64_t)(blockIdx.x + 1) * n_tiles / gridDim.x;
  const int kch = hidden / 128;
  const int steps = (int)((t1 - t0 + kRgTiles - 1) / kRgTiles) * kch;
  const uint32_t ring = (uint32_t)(uintptr_t)lds_raw;

  // Producer wv: instructions j = wv, wv + kRgProducers, ... of step st, slot rows 4j .. 4j+3.
  auto issue = [&](int st) __attribute__((always_inline)) {
    const int g = st / kch, c = st - g * kch;
    const uint32_t slot = ring + (uint32_t)((st % kRgRing) * kRgSlot);
#pragma unroll
    for (int n = 0; n < kRgInsPerWave; ++n) {
      const int j = wv + kRgProducers * n;
      const int r = 4 * j + (lane >> 4);
      const int64_t tile = t0 + (int64_t)g * kRgTiles + (r >> 4);
      const int64_t v = tile * 16 + (r & 15);
      const f16* row = w + (tile < t1 && v < vocab ? v : vocab - 1) * (int64_t)hidden;
      rg_dma(slot + (uint32_t)(4 * j * kRgRowBytes), row + c * 128 + ((lane & 15) ^ (r & 15)) * 8);
    }
  };
  // Consumer: x row tile rt, k = c*128 + 32s + 8*lg .. +7 for s = 0..3 (the B operand of step st).
  const f16* xrow = x + (int64_t)(rt * 16 + li < n_rows ? rt * 16 + li : n_rows - 1) * hidden + 8 * lg;
  auto load_x = [&](u32x4 (&xv)[4], int st) __attribute__((always_inline)) {
    const int c = st % kch;
#pragma unroll
    for (int s = 0; s < 4; ++s) xv[s] = *reinterpret_cast<const u32x4*>(xrow + c * 128 + 32 * s);
  };

  if (producer) {
    int issued = 0;
    while (issued < steps && issued < kRgRing - 1) issue(issued++);
    for (int i = 0; i < steps; ++i) {
      rg_wait_steps(issued - i - 1);            // step i landed (this producer's part) ...
      asm volatile("s_barrier" ::: "memory");   // ... and the other producers'; step i-1's slot is free
      if (issued < steps) issue(issued++);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  // Consumer.  x of step i sits in xv[i % XR].  The main loop runs whole
  // blocks of XR steps unrolled with no guard, so the register ring keeps
  // static indices and no register copy waits on a load in flight; every
  // load is unconditional (steps past the end reload the last step's x).
  // Steps past the last whole block (only when hidden / 128 is not a
  // multiple of XR) load their x just before use.
  f32x4 acc[TPW];
#pragma unroll
  for (int a = 0; a < TPW; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint64_t best = 0;  // this lane's largest key over every group so far (a max folds in any order)
  auto compute = [&](int i, const u32x4 (&xs)[4]) __attribute__((always_inline)) {
    const lds_char* sl = (const lds_char*)lds_raw + (i % kRgRing) * kRgSlot;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int q = (4 * s + lg) ^ li;
      const f16x8 b = as_h8(xs[s]);
#pragma unroll
      for (int a = 0; a < TPW; ++a) {
        const int wr = (h * TPW + a) * 16 + li;
        acc[a] = mfma_k32(as_h8(*reinterpret_cast<const lds_u32x4*>(sl + wr * kRgRowBytes + q * 16)), b, acc[a]);
      }
    }
    if ((i + 1) % kch == 0) {  // group end: acc[a][e] is vocab row 4*lg + e of tile a, x row rt*16 + li
      const int64_t tg = t0 + (int64_t)(i / kch) * kRgTiles + h * TPW;
#pragma unroll
      for (int a = 0; a < TPW; ++a) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t v = (tg + a) * 16 + 4 * lg + e;
          if (tg + a < t1 && v < vocab) best = umax64(best, argmax_key((f16)acc[a][e], (uint32_t)v));
        }
        acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  const int full = steps - steps % XR;
  u32x4 xv[XR][4];
  static_for<kRgXAhead>([&](auto u) {
    constexpr int k = decltype(u)::value;
    load_x(xv[k], k < steps ? k : steps - 1);
  });
  for (int i0 = 0; i0 < full; i0 += XR) {
    static_for<XR>([&](auto u) {
      constexpr int k = decltype(u)::value;  // step i0 + k uses xv[k]; xv[(k + kRgXAhead) % XR] is refilled
      const int i = i0 + k;
      // the refill is issued before the barrier, which the compiler cannot
      // move loads across: it cannot sink it next to the loads' first use
      const int nx = i + kRgXAhead;
      load_x(xv[(k + kRgXAhead) % XR], nx < steps ? nx : steps - 1);
      asm volatile("s_barrier" ::: "memory");  // step i's weight chunk is in its slot
      compute(i, xv[k]);
    });
  }
  for (int i = full; i < steps; ++i) {
    asm volatile("s_barrier" ::: "memory");
    u32x4 xs[4];
    load_x(xs, i);
    compute(i, xs);
  }
  // One key per x row and wave: the four lane groups' rows, then one atomic.
  best = umax64(best, shfl_xor64(best, 16));
  best = umax64(best, shfl_xor64(best, 32));
  const int row = rt * 16 + li;
  if (lg == 0 && row < n_rows && best)
    atomicMax(reinterpret_cast<unsigned long long*>(keys + row), (unsigned long long)best);
}

int rg_grid() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

template <int NRT>
void launch_rg(const f16* x, const f16* w, int rows, int hidden, int64_t vocab, uint64_t* keys, hipStream_t s) {
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_ring_kernel<NRT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kRgLds) == hipSuccess;
  }();
  (void)attr;
  const int64_t n_tiles = (vocab + 15) / 16;
  const unsigned grid = (unsigned)std::min<int64_t>(rg_grid(), n_tiles);
  hipLaunchKernelGGL(lm_ring_kernel<NRT>, dim3(grid), dim3(rg_threads<NRT>()), kRgLds, s, x, w, rows, hidden, vocab,
                     keys);
}

template <int... N>
void launch_rg_rows(std::integer_sequence<int, N...>, int nrt, const f16* x, const f16* w, int rows, int hidden,
                    int64_t vocab, uint64_t* keys, hipStream_t s) {
  ((nrt == N + 1 ? launch_rg<N + 1>(x, w, rows, hidden, vocab, keys, s) : void()), ...);
}

// ---- up/gate projection + SiLU·mul ----------------------------------------
//
// y[r][j] = fp16(up * fp16(silu(gate))) with up = fp16(x[r] . W[j]) and
// gate = fp16(x[r] . W[I + j]), W the stacked [2I, hidden] up_gate_proj
// weight: the reference's up/gate GEMM followed by silu_and_mul, with the
// same two fp16 roundings, without writing the [rows, 2I] product.  Same
// main loop as the lm_head kernel: one workgroup per CU owns a balanced
// range of 16-column output tiles, taken TO at a time; a group's ring slot
// holds the TO up tiles then the TO gate tiles (32*TO weight rows x 256 B of
// one k step of 128), brought in by four producer waves with
// global_load_lds_dwordx4; one consumer wave per 16-row tile of x holds its
// x rows in registers, loaded kUgXAhead steps ahead.  An up tile and its gate
// tile land in the same lane layout, so the SiLU·mul runs on the
// accumulators.  Ring depth grows as the slot shrinks, so every shape keeps
// about 100 KB in flight per CU.
template <int TO>
constexpr int ug_ring() { return TO == 1 ? 16 : TO == 2 ? 8 : TO == 3 ? 6 : TO == 4 ? 4 : 3; }
template <int TO>
constexpr int ug_xahead() { return TO == 1 ? 5 : TO == 2 ? 4 : 3; }
template <int TO>
constexpr int ug_slot() { return 2 * TO * 16 * kRgRowBytes; }
template <int TO>
constexpr int ug_lds() { return ug_ring<TO>() * ug_slot<TO>(); }
constexpr int kUgMaxTiles = 6;  // output tiles per group (12 weight tiles, a 48 KB slot)

// All but this producer's n most recent DMA instructions are complete.
__device__ inline void ug_wait(int n) {
#define NSD_UG_CASE(k) \
  case k:              \
    rg_wait_n<k>();    \
    break;
  switch (n) {
    NSD_UG_CASE(0) NSD_UG_CASE(1) NSD_UG_CASE(2) NSD_UG_CASE(3) NSD_UG_CASE(4) NSD_UG_CASE(5) NSD_UG_CASE(6)
    NSD_UG_CASE(7) NSD_UG_CASE(8) NSD_UG_CASE(9) NSD_UG_CASE(10) NSD_UG_CASE(11) NSD_UG_CASE(12)
    NSD_UG_CASE(13) NSD_UG_CASE(14) NSD_UG_CASE(15) NSD_UG_CASE(16) NSD_UG_CASE(17) NSD_UG_CASE(18)
    NSD_UG_CASE(19) NSD_UG_CASE(20) NSD_UG_CASE(21) NSD_UG_CASE(22) NSD_UG_CASE(23) NSD_UG_CASE(24)
    NSD_UG_CASE(25) NSD_UG_CASE(26) NSD_UG_CASE(27) NSD_UG_CASE(28) NSD_UG_CASE(29) NSD_UG_CASE(30)
    default: rg_wait_n<0>(); break;
  }
#undef NSD_UG_CASE
}

template <int NRT, int TO>
__global__ void __launch_bounds__((kRgProducers + NRT) * kWave)
up_gate_silu_kernel(const f16* __restrict__ x, const f16* __restrict__ w, f16* __restrict__ y, int n_rows,
                    int hidden, int inter) {
  constexpr int G = 2 * TO, RING = ug_ring<TO>(), SLOT = ug_slot<TO>(), XA = ug_xahead<TO>(), XR = XA + 1;
  static_assert((RING - 1) * G <= 30, "wait table");
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_tiles = inter / 16;
  const int t0 = (int)((int64_t)blockIdx.x * n_tiles / gridDim.x);
  const int t1 = (int)((int64_t)(blockIdx.x + 1) * n_tiles / gridDim.x);
  const int kch = hidden / 128;
  const int steps = (t1 - t0 + TO - 1) / TO * kch;
  const uint32_t ring = (uint32_t)(uintptr_t)lds_raw;

  if (wv < kRgProducers) {
    // Producer wv: instructions j = wv, wv + 4, ... of a step, slot rows
    // 4j .. 4j+3; slot row r < 16*TO is up tile r/16 of the group, the rest
    // the same gate tiles.  Tiles past the range fetch the range's last one.
    auto issue = [&](int st) __attribute__((always_inline)) {
      const int g = st / kch, c = st - g * kch;
      const uint32_t slot = ring + (uint32_t)((st % RING) * SLOT);
#pragma unroll
      for (int n = 0; n < G; ++n) {
        const int j = wv + kRgProducers * n;
        const int r = 4 * j + (lane >> 4);
        const int half = r >= 16 * TO, rr = r - half * 16 * TO;
        const int tile = t0 + g * TO + (rr >> 4);
        const int64_t v = (int64_t)half * inter + (int64_t)(tile < t1 ? tile : t1 - 1) * 16 + (rr & 15);
        rg_dma(slot + (uint32_t)(4 * j * kRgRowBytes), w + v * hidden + c * 128 + ((lane & 15) ^ (r & 15)) * 8);
      }
    };
    int issued = 0;
    while (issued < steps && issued < RING - 1) issue(issued++);
    for (int i = 0; i < steps; ++i) {
      ug_wait((issued - i - 1) * G);            // step i landed (this producer's part) ...
      asm volatile("s_barrier" ::: "memory");   // ... and the others'; step i-1's slot is free
      if (issued < steps) issue(issued++);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  // Consumer: x row tile rt, k = c*128 + 32s + 8*lg .. +7 (the B operand).
  const int rt = wv - kRgProducers;
  const int row = rt * 16 + li;
  const f16* xrow = x + (int64_t)(row < n_rows ? row : n_rows - 1) * hidden + 8 * lg;
  auto load_x = [&](u32x4 (&xv)[4], int st) __attribute__((always_inline)) {
    const int c = st % kch;
#pragma unroll
    for (int s = 0; s < 4; ++s) xv[s] = *reinterpret_cast<const u32x4*>(xrow + c * 128 + 32 * s);
  };
  f32x4 acc[G];
#pragma unroll
  for (int a = 0; a < G; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int i, const u32x4 (&xs)[4]) __attribute__((always_inline)) {
    const lds_char* sl = (const lds_char*)lds_raw + (i % RING) * SLOT;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int q = (4 * s + lg) ^ li;
      const f16x8 b = as_h8(xs[s]);
#pragma unroll
      for (int a = 0; a < G; ++a)
        acc[a] = mfma_k32(as_h8(*reinterpret_cast<const lds_u32x4*>(sl + (a * 16 + li) * kRgRowBytes + q * 16)), b,
                          acc[a]);
    }
    if ((i + 1) % kch == 0) {  // group end: acc[a][e] is column 4*lg + e of tile a, x row `row`
      const int tg = t0 + (i / kch) * TO;
#pragma unroll
      for (int a = 0; a < TO; ++a) {
        if (tg + a < t1 && row < n_rows) {
          f16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16 up = (f16)acc[a][e];
            const float g = (float)(f16)acc[TO + a][e];
            const f16 sg = (f16)(g / (1.f + expf(-g)));
            o[e] = (f16)((float)up * (float)sg);
          }
          *reinterpret_cast<f16x4*>(y + (int64_t)row * inter + (tg + a) * 16 + 4 * lg) = o;
        }
      }
#pragma unroll
      for (int a = 0; a < G; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // x of step i sits in xv[i % XR]; the main loop runs whole blocks of XR
  // steps with no guard (static register indices, unconditional loads).
  const int full = steps - steps % XR;
  u32x4 xv[XR][4];
  static_for<XA>([&](auto u) {
    constexpr int k = decltype(u)::value;
    load_x(xv[k], k < steps ? k : steps - 1);
  });
  for (int i0 = 0; i0 < full; i0 += XR) {
    static_for<XR>([&](auto u) {
      constexpr int k = decltype(u)::value;
      const int i = i0 + k;
      const int nx = i + XA;
      load_x(xv[(k + XA) % XR], nx < steps ? nx : steps - 1);
      asm volatile("s_barrier" ::: "memory");  // step i's weight chunk is in its slot
      compute(i, xv[k]);
    });
  }
  for (int i = full; i < steps; ++i) {
    asm volatile("s_barrier" ::: "memory");
    u32x4 xs[4];
    load_x(xs, i);
    compute(i, xs);
  }
}

template <int NRT, int TO>
void launch_ug(const f16* x, const f16* w, f16* y, int rows, int hidden, int inter, int grid, hipStream_t s) {
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&up_gate_silu_kernel<NRT, TO>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, ug_lds<TO>()) == hipSuccess;
  }();
  (void)attr;
  hipLaunchKernelGGL((up_gate_silu_kernel<NRT, TO>), dim3(grid), dim3((kRgProducers + NRT) * kWave), ug_lds<TO>(), s,
                     x, w, y, rows, hidden, inter);
}

template <int NRT>
void launch_ug_to(int to, const f16* x, const f16* w, f16* y, int rows, int hidden, int inter, int grid,
                  hipStream_t s) {
  switch (to) {
    case 1: launch_ug<NRT, 1>(x, w, y, rows, hidden, inter, grid, s); break;
    case 2: launch_ug<NRT, 2>(x, w, y, rows, hidden, inter, grid, s); break;
    case 3: launch_ug<NRT, 3>(x, w, y, rows, hidden, inter, grid, s); break;
    case 4: launch_ug<NRT, 4>(x, w, y, rows, hidden, inter, grid, s); break;
    default: launch_ug<NRT, 6>(x, w, y, rows, hidden, inter, grid, s); break;
  }
}

template <int... N>
void launch_ug_rows(std::integer_sequence<int, N...>, int nrt, int to, const f16* x, const f16* w, f16* y, int rows,
                    int hidden, int inter, int grid, hipStream_t s) {
  ((nrt == N + 1 ? launch_ug_to<N + 1>(to, x, w, y, rows, hidden, inter, grid, s) : void()), ...);
}

}  // namespace
}  // namespace nsd

using namespace nsd;

static int fused_add_rmsnorm(void* x, void* residual, const void* weight, int64_t n_rows, int64_t hidden, float eps,
                             const float* part, int splits, void* stream) {
  if (n_rows < 0 || hidden <= 0) return fail(NSD_ERR_INVALID, "fused_add_rmsnorm: bad shape");
  if (n_rows == 0) return NSD_OK;
  if (!x || !residual || !weight) return fail(NSD_ERR_INVALID, "fused_add_rmsnorm: null pointer");
  if (hidden % 8 || hidden > 8 * kNormThreads * kMaxNormVecs)
    return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: hidden=%lld (need a multiple of 8, <= %d)",
                (long long)hidden, 8 * kNormThreads * kMaxNormVecs);
  if (!aligned16(x) || !aligned16(residual) || !aligned16(weight) || (part && !aligned16(part)))
    return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: pointers must be 16-byte aligned");
  if (n_rows > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "fused_add_rmsnorm: too many rows");
  const int nvec = (int)(hidden / 8);
  const int vpt = (nvec + kNormThreads - 1) / kNormThreads;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)n_rows), dim3(kNormThreads), 0, as_stream(stream),
                       static_cast<f16*>(x), static_cast<f16*>(residual), static_cast<const f16*>(weight), nvec,
                       (int)hidden, eps, part, splits, n_rows * hidden);
  };
  switch (vpt) {
    case 1: go(fused_add_rmsnorm_kernel<1>); break;
    case 2: go(fused_add_rmsnorm_kernel<2>); break;
    case 3: go(fused_add_rmsnorm_kernel<3>); break;
    default: go(fused_add_rmsnorm_kernel<4>); break;
  }
  return launch_status("fused_add_rmsnorm");
}

extern "C" int nsd_fused_add_rmsnorm_inplace(void* x, void* residual, const void* weight, int64_t n_rows,
                                             int64_t hidden, float eps, void* stream) {
  return fused_add_rmsnorm(x, residual, weight, n_rows, hidden, eps, nullptr, 1, stream);
}

extern "C" int nsd_fused_add_rmsnorm_partials(const float* partials, int splits, void* out, void* residual,
                                              const void* weight, int64_t n_rows, int64_t hidden, float eps,
                                              void* stream) {
  if (partials == nullptr || splits < 1 || splits > 8)
    return fail(NSD_ERR_INVALID, "fused_add_rmsnorm_partials: %d splits (1..8) of partials", splits);
  return fused_add_rmsnorm(out, residual, weight, n_rows, hidden, eps, partials, splits, stream);
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
    launch_rg_rows(std::make_integer_sequence<int, kRgMaxRowTiles>{}, (rows + 15) / 16, xr, wp, rows, (int)hidden,
                   vocab, kr, s);
    if (int e = launch_status("lm_head_argmax")) return e;
  }
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)((n_rows + 255) / 256)), dim3(256), 0, s, keys, tokens,
                     (int)n_rows);
  return launch_status("lm_head_argmax finalize");
}

extern "C" int nsd_up_gate_silu_and_mul(const void* x, const void* up_gate, void* y, int64_t n_rows, int64_t hidden,
                                        int64_t inter, void* stream) {
  if (n_rows < 0 || hidden <= 0 || inter <= 0) return fail(NSD_ERR_INVALID, "up_gate_silu_and_mul: bad shape");
  if (n_rows == 0) return NSD_OK;
  if (!x || !up_gate || !y) return fail(NSD_ERR_INVALID, "up_gate_silu_and_mul: null pointer");
  if (hidden % kLmK || hidden > INT32_MAX / 2)
    return fail(NSD_ERR_UNSUPPORTED, "up_gate_silu_and_mul: hidden=%lld (need a multiple of %d)", (long long)hidden,
                kLmK);
  if (inter % 16 || inter > INT32_MAX / 2)
    return fail(NSD_ERR_UNSUPPORTED, "up_gate_silu_and_mul: inter=%lld (need a multiple of 16)", (long long)inter);
  if (!aligned16(x) || !aligned16(up_gate) || !aligned16(y))
    return fail(NSD_ERR_UNSUPPORTED, "up_gate_silu_and_mul: pointers must be 16-byte aligned");
  bool served = false;
  if (int rc = up_gate_silu_gated(x, up_gate, y, n_rows, hidden, inter, stream, &served)) return rc;
  if (served) return NSD_OK;
  const hipStream_t s = as_stream(stream);
  const int n_tiles = (int)(inter / 16);
  const int grid = std::min(rg_grid(), n_tiles);
  const int per = (n_tiles + grid - 1) / grid;  // output tiles of the busiest workgroup
  const int to = per <= 4 ? per : per <= 6 ? 6 : kUgMaxTiles;
  const f16* xp = static_cast<const f16*>(x);
  // Rows in passes of at most 128 (each pass streams the weight once).
  for (int64_t r0 = 0; r0 < n_rows; r0 += 128) {
    const int rows = (int)std::min<int64_t>(128, n_rows - r0);
    launch_ug_rows(std::make_integer_sequence<int, kRgMaxRowTiles>{}, (rows + 15) / 16, to, xp + r0 * hidden,
                   static_cast<const f16*>(up_gate), static_cast<f16*>(y) + r0 * inter, rows, (int)hidden, (int)inter,
                   grid, s);
    if (int e = launch_status("up_gate_silu_and_mul")) return e;
  }
  return NSD_OK;
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
