// Projection GEMMs of decode/verify batches for gfx950 (MI355X).
//
// y[rows, n] = x[rows, k] . W[n, k]^T (fp16 in, fp32 sums) for the q/k/v, O
// and down projections of a layer at decode/verify batch sizes (rows <= 128).
// The weight is the whole of the traffic (x is at most 3 MB and stays in L2),
// so the kernel is a stream of W through the compute units:
//
//   - the work is cut into (n-tile of TN columns, k-range) units, one
//     workgroup each, about one per compute unit: TN columns over all of k
//     would give each CU too little of W and make it re-read all of x, so
//     k is split into `splits` ranges and every unit writes fp32 partial
//     sums [split][rows][n]; the consumer of the projection (the next
//     add-RMSNorm, the QK-norm/RoPE/KV-store prologue, or a small sum pass)
//     adds the splits in split order and rounds to fp16 once, which is the
//     GEMM output rounding of F.linear;
//   - a workgroup streams its unit in steps of 128 k through a ring of LDS
//     slots filled by global_load_lds_dwordx4 (each instruction brings four
//     256-byte row chunks), a slot holding the step's TN weight rows and the
//     step's x rows, with two steps in flight; rows are XOR-swizzled per
//     16-byte chunk so the 16 rows an MFMA operand read touches hit distinct
//     banks;
//   - v_mfma_f32_16x16x32_f16 with A = weight rows, B = x rows: for TN >= 64
//     each wave owns TN/64 of the 16-column n-tiles over the whole step, for
//     TN = 16 and 32 each wave owns one of the step's four 32-k sub-steps
//     over every output tile and the four waves' sums are added in LDS, in
//     wave order, at the end;
//   - a gated unit serves the FFN's up/gate projection: 48 up and the
//     matching 48 gate rows over all of k, the SiLU-and-mul applied to the
//     accumulators, fp16 output (no partials).
//
// Measured on MI355X against hipBLASLt (the library F.linear uses), µs per
// call with the weights rotated past the MALL: Qwen3-8B at 80 rows, O
// 4096x4096 10.5 (16.6), down 12288 -> 4096 23.6-25 (40.9), q/k/v 4096 ->
// 6144 15.5 (23.2); Qwen3-0.6B at 64 rows, q/k/v 5.4 (11.6), O 4.2 (10.6),
// down 4.9 (9.3).
#include <algorithm>
#include <atomic>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int kKStep = 128;                 // k per ring step
constexpr int kStepRowBytes = kKStep * 2;   // one row's chunk of a step
constexpr int kGemmThreads = 256;
constexpr int kGemmLds = 156 * 1024;        // LDS one workgroup may use
constexpr int kMaxSplits = 8;
constexpr int kMaxRowTiles = 8;             // 128 rows

__device__ inline int chunk_swizzle(int row) { return row & 15; }

__device__ inline void gemm_dma(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}
template <int N>
__device__ inline void gemm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline void gemm_barrier() { asm volatile("s_barrier" ::: "memory"); }

// GATED: the FFN's up/gate projection with SiLU-and-mul in the epilogue:
// the unit's TN weight rows are TN/2 up rows then the same TN/2 gate rows
// (W = [up; gate], 2 * n rows), over all of k, and the unit writes fp16
// h = fp16(up) * fp16(silu(fp16(gate))) for its TN/2 columns.
//
// How the four waves share a step's MFMAs (kMode): 0 -- each wave one of the
// four 32-k sub-steps over every output tile, summed across waves in LDS at
// the end (TN 16, 32); 1 -- each wave TN/64 of the 16-column tiles over the
// whole step (TN >= 64); 2 -- GATED: wave w (< TN/32) the up tile w and its
// gate tile over the whole step, so the SiLU-and-mul needs no exchange.
template <int MT, int TN, bool GATED = false>
struct LinearShape {
  static constexpr int kRows = TN + 16 * MT;            // rows of one slot: weight, then x
  static constexpr int kSlot = kRows * kStepRowBytes;
  static constexpr int kRing = 3 * kSlot <= kGemmLds ? 3 : 2;
  static constexpr int kLds = kRing * kSlot;
  static constexpr int kDmaPerWave = kRows / 16;        // 4 rows per instruction, 4 waves
  static constexpr int kMode = GATED ? 2 : TN >= 64 ? 1 : 0;
  static_assert(kRing * kSlot <= kGemmLds, "ring");
  static_assert(kMode != 0 || 4 * (TN / 16) * MT * 1024 <= kLds, "reduction buffer");
  static_assert(kMode != 2 || (TN / 32 <= 4 && TN % 32 == 0), "one up/gate tile pair per wave");
};

// Unit u = (n-tile u % n_tiles, split u / n_tiles); split s covers steps
// [s T / splits, (s+1) T / splits) of the T = k / 128 steps.
template <int MT, int TN, bool GATED = false>
__global__ __launch_bounds__(kGemmThreads) void linear_partials_kernel(const f16* __restrict__ x,
                                                                       const f16* __restrict__ w,
                                                                       float* __restrict__ part, int rows,
                                                                       int n, int k, int splits,
                                                                       int n_tiles, f16* __restrict__ y) {
  using S = LinearShape<MT, TN, GATED>;
  constexpr int R = S::kRing;
  constexpr int NI = S::kDmaPerWave;
  constexpr int NJ = TN / 16;
  constexpr int M = S::kMode;
  constexpr int NJW = M == 1 ? NJ / 4 : M == 2 ? 2 : NJ;  // n-tiles per wave
  constexpr int KSUB = M == 0 ? 1 : 4;                     // 32-k sub-steps per wave per step
  extern __shared__ __align__(16) char smem_raw[];
  lds_char* ring = (lds_char*)smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int nt = blockIdx.x % n_tiles, split = blockIdx.x / n_tiles;
  const int n0 = nt * (GATED ? TN / 2 : TN);
  const bool computes = M != 2 || wave < NJ / 2;
  auto tile_of = [&](int j) { return M == 1 ? wave * NJW + j : M == 2 ? wave + j * (NJ / 2) : j; };
  const int T = k / kKStep;
  const int t0 = (int)((int64_t)split * T / splits);
  const int steps = (int)((int64_t)(split + 1) * T / splits) - t0;

  // DMA instruction i of this wave brings rows 4(4i + wave) .. +3 of a slot;
  // lane l the 16-byte chunk (l % 16) ^ swizzle(row) of row l / 16 of them.
  const f16* src[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (4 * i + wave) * 4 + (lane >> 4);
    const int chunk = (lane & 15) ^ chunk_swizzle(row);
    // weight row of slot row `row` (GATED: up rows, then the gate rows n further on)
    const int wrow = !GATED || row < TN / 2 ? n0 + row : n + n0 + row - TN / 2;
    const f16* base = row < TN ? w + (int64_t)wrow * k
                               : x + (int64_t)(row - TN < rows ? row - TN : rows - 1) * k;  // pad rows: a real row
    src[i] = base + (int64_t)t0 * kKStep + chunk * 8;
  }
  auto issue = [&](int t) {
    const lds_char* slot = ring + (t % R) * S::kSlot;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      gemm_dma((uint32_t)(uintptr_t)(slot + (4 * i + wave) * 1024), src[i] + (int64_t)t * kKStep);
  };
  f32x4 acc[NJW][MT];
#pragma unroll
  for (int j = 0; j < NJW; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  int issued = 0;
  for (; issued < R - 1 && issued < steps; ++issued) issue(issued);
  for (int t = 0; t < steps; ++t) {
    // this wave's loads of step t have landed (the ring's later steps may
    // still be in flight), then every wave's; the slot of step t-1 is free
    if (issued - t - 1 >= R - 2) gemm_wait<(R - 2) * NI>();
    else gemm_wait<0>();
    gemm_barrier();
    if (issued < steps) issue(issued++);
    const lds_char* sl = ring + (t % R) * S::kSlot;
    if (!computes) continue;
#pragma unroll
    for (int kk = 0; kk < KSUB; ++kk) {
      const int ch = 4 * (M == 0 ? wave : kk) + lg;  // lane group's 8 k of the sub-step
      f16x8 a[NJW], b[MT];
#pragma unroll
      for (int j = 0; j < NJW; ++j) {
        const int row = 16 * tile_of(j) + lr;
        a[j] = *(const lds_f16x8*)(sl + row * kStepRowBytes + ((ch ^ chunk_swizzle(row)) << 4));
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int row = TN + 16 * i + lr;
        b[i] = *(const lds_f16x8*)(sl + row * kStepRowBytes + ((ch ^ chunk_swizzle(row)) << 4));
      }
#pragma unroll
      for (int j = 0; j < NJW; ++j)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[j][i] = mfma_k32(a[j], b[i], acc[j][i]);
    }
  }
  // lane (lg, lr) holds columns 4lg .. 4lg+3 of an n-tile for row lr of an
  // m-tile: 16 contiguous bytes of the partial row (no partials when gated)
  float* out = GATED ? nullptr : part + (int64_t)split * rows * n;
  auto store = [&](int j, int i, f32x4 v) {
    const int m = 16 * i + lr;
    if (m < rows) *reinterpret_cast<f32x4*>(out + (int64_t)m * n + n0 + 16 * j + 4 * lg) = v;
  };
  if constexpr (M == 1) {
#pragma unroll
    for (int j = 0; j < NJW; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) store(tile_of(j), i, acc[j][i]);
  } else if constexpr (M == 2) {
    // up tile `wave` and its gate tile leave the same lane layout: the
    // SiLU-and-mul of silu_and_mul_kernel on the fp16-rounded sums
    if (!computes) return;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = 16 * i + lr;
      if (m >= rows) continue;
      f16x4 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16 up = (f16)acc[0][i][e];
        const float gf = (float)(f16)acc[1][i][e];
        const f16 sg = (f16)(gf / (1.f + expf(-gf)));
        h[e] = (f16)((float)up * (float)sg);
      }
      *reinterpret_cast<f16x4*>(y + (int64_t)m * n + n0 + 16 * wave + 4 * lg) = h;
    }
  } else {
    __syncthreads();  // the ring is drained: its LDS holds the waves' sums
    f32x4* red = reinterpret_cast<f32x4*>(smem_raw);  // [wave][tile][lane]
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) red[(wave * NJ * MT + j * MT + i) * 64 + lane] = acc[j][i];
    __syncthreads();
    for (int tile = wave; tile < NJ * MT; tile += 4) {
      f32x4 v = red[tile * 64 + lane];
#pragma unroll
      for (int q = 1; q < 4; ++q) v += red[(q * NJ * MT + tile) * 64 + lane];
      store(tile / MT, tile % MT, v);
    }
  }
}

// y[i] = fp16(sum over splits of part[s][i]), eight elements per thread.
__global__ __launch_bounds__(256) void sum_partials_kernel(const float* __restrict__ part, int splits,
                                                           int64_t per_split, f16* __restrict__ y) {
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < per_split / 8; v += (int64_t)gridDim.x * 256) {
    f32x4 lo = *reinterpret_cast<const f32x4*>(part + 8 * v);
    f32x4 hi = *reinterpret_cast<const f32x4*>(part + 8 * v + 4);
    for (int s = 1; s < splits; ++s) {
      lo += *reinterpret_cast<const f32x4*>(part + s * per_split + 8 * v);
      hi += *reinterpret_cast<const f32x4*>(part + s * per_split + 8 * v + 4);
    }
    f16x8 h = {(f16)lo[0], (f16)lo[1], (f16)lo[2], (f16)lo[3], (f16)hi[0], (f16)hi[1], (f16)hi[2], (f16)hi[3]};
    *reinterpret_cast<f16x8*>(y + 8 * v) = h;
  }
}

struct LinearConfig {
  int tn = 0, splits = 0;
};

// Column tile and k-split for an n x k projection on `cus` compute units:
// the configuration whose units fill the most of whole rounds of one unit
// per CU, with at least four steps per unit where k allows; ties go to the
// 64-column tile (measured fastest where several fill the chip), then 128,
// 32, 16.
LinearConfig choose_linear(int64_t n, int64_t k, int cus) {
  LinearConfig best;
  double best_fill = -1.0;
  const int64_t steps = k / kKStep;
  for (int tn : {64, 128, 32, 16}) {
    if (n % tn) continue;
    const int64_t tiles = n / tn;
    const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(kMaxSplits, steps / 4));
    const int64_t splits = std::max<int64_t>(1, std::min<int64_t>(cap, cus / tiles));
    const int64_t units = tiles * splits;
    const int64_t rounds = (units + cus - 1) / cus;
    const double fill = (double)units / (double)(rounds * cus);
    if (fill > best_fill + 1e-9) {
      best_fill = fill;
      best.tn = tn;
      best.splits = (int)splits;
    }
  }
  return best;
}

// Compute units of the current device (queried once per device: the
// decoder stack asks for every projection it enqueues).
int device_cus(int* cus) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *cus = c;
      return NSD_OK;
    }
  }
  if (e == hipSuccess) e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail(NSD_ERR_HIP, "linear: %s", hipGetErrorString(e));
  if (*cus < 1) return fail(NSD_ERR_HIP, "linear: device %d reports %d compute units", dev, *cus);
  if (dev >= 0 && dev < kMaxDevices) cached[dev].store(*cus, std::memory_order_relaxed);
  return NSD_OK;
}

int check_linear(int64_t n_rows, int64_t n_out, int64_t n_in, const char* who) {
  if (n_rows < 1 || n_rows > 16 * kMaxRowTiles)
    return fail(NSD_ERR_UNSUPPORTED, "%s: n_rows=%lld outside [1, %d]", who, (long long)n_rows, 16 * kMaxRowTiles);
  if (n_out < 16 || n_out % 16 || n_in < kKStep || n_in % kKStep || n_out > INT32_MAX || n_in > INT32_MAX)
    return fail(NSD_ERR_UNSUPPORTED, "%s: n_out=%lld (a multiple of 16), n_in=%lld (a multiple of 128)", who,
                (long long)n_out, (long long)n_in);
  return NSD_OK;
}

template <int MT, int TN>
int launch_linear(const f16* x, const f16* w, float* part, int rows, int n, int k, int splits, hipStream_t st) {
  using S = LinearShape<MT, TN>;
  // raise the dynamic-LDS limit once per process: a function-local static is
  // initialised exactly once even when several threads launch at once, and
  // a failure stays reported on every later call
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&linear_partials_kernel<MT, TN>), hipFuncAttributeMaxDynamicSharedMemorySize,
      S::kLds);
  if (attr != hipSuccess) return fail(NSD_ERR_HIP, "linear: LDS attribute: %s", hipGetErrorString(attr));
  const int n_tiles = n / TN;
  hipLaunchKernelGGL((linear_partials_kernel<MT, TN>), dim3(n_tiles * splits), dim3(kGemmThreads), S::kLds, st, x,
                     w, part, rows, n, k, splits, n_tiles, nullptr);
  return launch_status("linear");
}

// The gated (up/gate + SiLU-and-mul) unit: 48 up and 48 gate columns over
// all of k, one unit per 48 output columns.
constexpr int kGatedTile = 96;
constexpr int kGatedMaxRowTiles = 7;  // three ring slots fit up to 112 rows (128 rows: the ring kernel, 1.5 us faster)

template <int MT>
int launch_gated(const f16* x, const f16* w, f16* y, int rows, int inter, int hidden, hipStream_t st) {
  using S = LinearShape<MT, kGatedTile, true>;
  static const hipError_t attr = hipFuncSetAttribute(  // once per process, as in launch_linear
      reinterpret_cast<const void*>(&linear_partials_kernel<MT, kGatedTile, true>),
      hipFuncAttributeMaxDynamicSharedMemorySize, S::kLds);
  if (attr != hipSuccess) return fail(NSD_ERR_HIP, "up_gate: LDS attribute: %s", hipGetErrorString(attr));
  const int n_tiles = inter / (kGatedTile / 2);
  hipLaunchKernelGGL((linear_partials_kernel<MT, kGatedTile, true>), dim3(n_tiles), dim3(kGemmThreads), S::kLds, st,
                     x, w, nullptr, rows, inter, hidden, 1, n_tiles, y);
  return launch_status("up_gate_silu_and_mul");
}

template <int... I>
int launch_gated_rows(std::integer_sequence<int, I...>, int mt, const f16* x, const f16* w, f16* y, int rows,
                      int inter, int hidden, hipStream_t st) {
  int rc = NSD_ERR_UNSUPPORTED;
  ((mt == I + 1 ? (rc = launch_gated<I + 1>(x, w, y, rows, inter, hidden, st), 0) : 0), ...);
  return rc;
}

template <int TN, int... I>
int launch_linear_rows(std::integer_sequence<int, I...>, int mt, const f16* x, const f16* w, float* part, int rows,
                       int n, int k, int splits, hipStream_t st) {
  int rc = NSD_ERR_UNSUPPORTED;
  ((mt == I + 1 ? (rc = launch_linear<I + 1, TN>(x, w, part, rows, n, k, splits, st), 0) : 0), ...);
  return rc;
}

}  // namespace

int up_gate_silu_gated(const void* x, const void* up_gate, void* y, int64_t n_rows, int64_t hidden, int64_t inter,
                       void* stream, bool* served) {
  *served = false;
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  const int64_t units = inter / (kGatedTile / 2);
  // one unit per CU or close to it (fewer units leave CUs idle: the older
  // kernel spreads small shapes better)
  if (inter % (kGatedTile / 2) || units * 10 < cus * 9 || units > cus || n_rows > 16 * kGatedMaxRowTiles ||
      hidden % kKStep)
    return NSD_OK;
  *served = true;
  return launch_gated_rows(std::make_integer_sequence<int, kGatedMaxRowTiles>{}, (int)((n_rows + 15) / 16),
                           static_cast<const f16*>(x), static_cast<const f16*>(up_gate), static_cast<f16*>(y),
                           (int)n_rows, (int)inter, (int)hidden, as_stream(stream));
}

}  // namespace nsd

using namespace nsd;

extern "C" int nsd_linear_splits(int64_t n_rows, int64_t n_out, int64_t n_in, int* splits) {
  if (splits == nullptr) return fail(NSD_ERR_INVALID, "linear_splits: null output");
  if (int rc = check_linear(n_rows, n_out, n_in, "linear_splits")) return rc;
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  *splits = choose_linear(n_out, n_in, cus).splits;
  return NSD_OK;
}

extern "C" int nsd_linear_partials(const void* x, const void* w, float* partials, int64_t n_rows, int64_t n_out,
                                   int64_t n_in, void* stream) {
  if (int rc = check_linear(n_rows, n_out, n_in, "linear_partials")) return rc;
  if (!x || !w || !partials) return fail(NSD_ERR_INVALID, "linear_partials: null pointer");
  if (!aligned16(x) || !aligned16(w) || !aligned16(partials))
    return fail(NSD_ERR_UNSUPPORTED, "linear_partials: pointers must be 16-byte aligned");
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  const LinearConfig c = choose_linear(n_out, n_in, cus);
  const int mt = (int)((n_rows + 15) / 16);
  const auto* xp = static_cast<const f16*>(x);
  const auto* wp = static_cast<const f16*>(w);
  const hipStream_t st = as_stream(stream);
  const auto seq = std::make_integer_sequence<int, kMaxRowTiles>{};
  const int rows = (int)n_rows, n = (int)n_out, k = (int)n_in;
  switch (c.tn) {
    case 16: return launch_linear_rows<16>(seq, mt, xp, wp, partials, rows, n, k, c.splits, st);
    case 32: return launch_linear_rows<32>(seq, mt, xp, wp, partials, rows, n, k, c.splits, st);
    case 64: return launch_linear_rows<64>(seq, mt, xp, wp, partials, rows, n, k, c.splits, st);
    default: return launch_linear_rows<128>(seq, mt, xp, wp, partials, rows, n, k, c.splits, st);
  }
}

extern "C" int nsd_sum_partials(const float* partials, int splits, void* y, int64_t n_rows, int64_t n_out,
                                void* stream) {
  if (n_rows < 0 || n_out < 8 || n_out % 8 || splits < 1 || splits > kMaxSplits)
    return fail(NSD_ERR_INVALID, "sum_partials: rows=%lld n_out=%lld splits=%d", (long long)n_rows,
                (long long)n_out, splits);
  if (n_rows == 0) return NSD_OK;
  if (!partials || !y) return fail(NSD_ERR_INVALID, "sum_partials: null pointer");
  if (!aligned16(partials) || !aligned16(y))
    return fail(NSD_ERR_UNSUPPORTED, "sum_partials: pointers must be 16-byte aligned");
  const int64_t per = n_rows * n_out;
  const unsigned grid = (unsigned)std::min<int64_t>((per / 8 + 255) / 256, 1024);
  hipLaunchKernelGGL(sum_partials_kernel, dim3(grid), dim3(256), 0, as_stream(stream), partials, splits, per,
                     static_cast<f16*>(y));
  return launch_status("sum_partials");
}
