// Paged verify/decode attention for gfx950 (MI355X).
//
// Work unit.  A verify group is q_len consecutive rows of one sequence whose
// seq_lens rise by one (ctx+1 .. ctx+q_len); a decode row is a group with
// q_len = 1.  For one (group, kv head) -- a "segment" -- the GQA group x
// q_len query rows (up to 64) are packed as the N dimension of fp16 MFMAs,
// so each K/V tile of the segment is read from HBM exactly once:
//
//   S^T[token][row] = K[token][:] . Q[row][:]            (A = K, B = Q^T)
//   O^T[dim][row]  += V^T[dim][token] . P^T[token][row]  (A = V^T, B = P^T)
//
// Both products use v_mfma_f32_16x16x32_f16: S^T with k = 32 of the 128 head
// dims per instruction, O^T with k = the 32 tokens of a two-block step.  Both
// leave a lane holding one query row (lane & 15) of a 16-row tile, so a row's
// online-softmax state lives in one lane column, and the S^T result of a step
// is already the P^T operand of the PV product (see the token order below).
//
// Work split.  The host planner cuts the stream of (segment, 16-token block)
// work into contiguous ranges of near-equal cost, one per workgroup
// ("worker"), two workgroups per compute unit.  A workgroup streams its
// range through a ring of kRing LDS slots, each holding one block's K tile
// then V tile, brought straight from HBM by global_load_lds_dwordx4 (each of
// the four waves brings 1 KB of K and 1 KB of V of every block).  The ring
// advances two blocks per step: one barrier hands two landed slots to the
// compute and the slots of the previous step back to the loads, with
// kRing - 2 blocks in flight.  The DMA offsets of every block come from a table the workgroup
// builds in LDS before it starts, so a step costs each wave a few scalar
// instructions.
//
// Wave r < NT computes row tile r (rows 16r .. 16r+15 of the segment's
// group) over all 128 dims: its scores, one online softmax over the step's
// 32 tokens, and the PV products.  No softmax state is merged across waves,
// and every output is summed in block order by one wave, so a call's results
// do not depend on timing: identical inputs give identical bits.  The K rows
// of the two blocks are fed to the two score MFMAs in the order that leaves
// lane group g holding tokens 8g .. 8g+7 of both, which is the k order of the
// 16x16x32 PV MFMA's operand: S^T feeds PV without moving a value.  Both
// blocks of a step belong to one piece; a piece with an odd block count ends
// with a one-block step (its second half masked, both halves read from the
// one slot).  Segments cut across
// workers write partials (normalised O in fp16, log2-sum-exp in fp32: the
// merged result stays within one more fp16 rounding of the fp32 merge, and
// the partial stores, a few MB per call, cost half the time), and a second,
// small launch merges each such segment's partials in slot order (the
// reference's phase 2): the attention kernel then ends as soon as its
// workgroups have stored their last results.
//
// Layouts (reference swiftLLM/swiftllm/worker/kernels/paged_attn.py):
//   k/v cache [N, L, Hkv, 16, 128] fp16, block (blk, layer, head) = 4 KB
//   contiguous at ((blk*L + layer)*Hkv + head)*16*128 (:49-50, :70-71).
#include <mutex>
#include <type_traits>
#include <utility>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int D = kHeadDim;          // 128
constexpr int BS = kBlockTokens;     // 16
constexpr int kRowBytes = D * 2;     // one fp16 row of K or V
constexpr int kTile = BS * kRowBytes;  // one (block, layer, head) tile: 4 KB
// A ring slot holds a block's K tile then its V tile.  Slots sit 8 KB + 128 B
// apart, so the two slots a step reads start in opposite halves of the
// 256-byte bank window (their K rows then never share banks).
constexpr int kSlot = 2 * kTile + 128;
constexpr int kRing = 4;             // ring slots: one step of 2 blocks in flight
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr float kLn2 = 0.69314718055994531f;
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xF << 8);  // s_waitcnt vmcnt(0), other counters open
constexpr float kLazyMax = 8.f;      // the running max moves only when exceeded by 2^8
// Item table entry: element offset of the block's tile in the cache, with
// this bit set for a masked block (an id outside the pool).
constexpr uint64_t kMasked = 1ull << 62;
constexpr int kMaxWorkerItems = kMaxWorkerBlocks;

// LDS: ring, the worker's item table, its piece records.
constexpr int kLdsItems = kRing * kSlot;
constexpr int kLdsRecs = kLdsItems + kMaxWorkerItems * 8;
constexpr int kLdsBytes = kLdsRecs + kMaxWorkerPieces * kPieceWords * 4;
static_assert(2 * (kLdsBytes + 256) <= 160 * 1024, "two workgroups per compute unit");
static_assert(kMaxGroupRows <= 16 * kWaves, "one wave per 16-row tile");

// 16-byte chunk c of row t of a ring tile sits at chunk c ^ swizzle(t).  K
// rows are read 16 rows x one chunk per MFMA operand, the rows of a lane
// group being {0-3, 8-11} or {4-7, 12-15} of one tile (or all 16 for the
// query rows): swz_k is injective on each of those sets modulo 8 and on all
// 16 rows.  V rows are read by transposing reads, 4 rows x 32 bytes per 16
// lanes, over rows {0-3, 8-11} or {4-7, 12-15} per 32 lanes: swz_v gives
// those rows 8 distinct even chunk offsets, so the 32-byte pairs stay whole
// and disjoint.
__device__ inline int swz_k(int t) { return (t ^ ((t >> 3) << 2)) & 15; }
__device__ inline int swz_v(int t) { return (2 * swz_k(t)) & 15; }

struct AttnArgs {
  const f16* q;            // [R, Hq, D]
  f16* o;                  // [R, Hq, D]
  float* lse;              // [R, Hq] natural log, optional
  const f16* k_cache;
  const f16* v_cache;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* workers;  // plan: worker table
  const int32_t* pieces;   // plan: piece records
  f16* part_o;             // [slots, rows_max, D]  normalised O
  float* part_lse;         // [slots, rows_max]  (log2 domain)
  const int32_t* combines; // plan: combine records of the segments cut across workers
  int32_t* status;
  int64_t num_blocks;
  int64_t blk_stride;      // elements per cache block: L*Hkv*16*128
  int num_layers, layer, hq, hkv, gqa, rows_max;
  int piece_stride;        // plan: piece records per worker
  float scale_log2;        // softmax_scale * log2(e)
};

// The ring's loads and waits are written as inline asm: the compiler does not
// see them, so it neither drains the loads in flight before every LDS read of
// the ring nor reorders its own LDS reads across the asm (memory clobber).
// The compiler's own vector-memory operations in the loop (output and partial
// stores) only make the explicit vmcnt waits stricter, never too loose.
__device__ inline void ring_load(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}
template <int N>
__device__ inline void wait_ring_n() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}
// Wait until this wave's loads of all but the n most recently issued ring
// items are complete (two loads per item); 0 <= n <= kRing - 1.
__device__ inline void wait_ring(int n) {
  static_assert(kRing <= 8, "wait table");
  switch (n) {
    case 0: wait_ring_n<0>(); break;
    case 1: wait_ring_n<2>(); break;
    case 2: wait_ring_n<4>(); break;
    case 3: wait_ring_n<6>(); break;
    case 4: wait_ring_n<8>(); break;
    case 5: wait_ring_n<10>(); break;
    case 6: wait_ring_n<12>(); break;
    default: wait_ring_n<14>(); break;
  }
}
__device__ inline void barrier() { asm volatile("s_barrier" ::: "memory"); }

// Max and sum over the four 16-lane rows of a wave (lanes l, l^16, l^32,
// l^48) with gfx950's row-swap moves: v_permlane16_swap pairs rows 0-1 and
// 2-3, v_permlane32_swap pairs rows 0-2 and 1-3; every lane ends with the
// same value.
__device__ inline float rows_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float rows_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ inline uint32_t lds_address(const lds_char* p) {
  return (uint32_t)(uintptr_t)p;
}

// Second launch: merge the partials of the segments cut across workers.
// Workgroup (c, g) merges rows 16g .. 16g+15 of combine record c; thread
// (row, 8 dims), slots folded in slot order with a running max (online
// log-sum-exp), eight slots' loads in flight at a time.  Same exp2-domain
// combine as phase 2 of the reference (paged_attn.py:128-149).  The kernel
// boundary orders it after every partial store of the attention launch.
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a, int row_groups) {
  const int32_t* c = a.combines + kPieceWords * (blockIdx.x / row_groups);
  const int n = 16 * (blockIdx.x % row_groups) + (threadIdx.x >> 4);
  const int h = c[kCombHead], first = c[kCombFirst], n_slots = c[kCombSlots];
  if (n >= c[kCombQLen] * a.gqa) return;
  const int d8 = threadIdx.x & 15;
  const f16* po = a.part_o + ((int64_t)first * a.rows_max + n) * D + 8 * d8;
  const float* pl = a.part_lse + (int64_t)first * a.rows_max + n;
  const int64_t sstride = (int64_t)a.rows_max * D;  // elements between slots
  float M = -INFINITY, W = 0.f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n_slots; s0 += 8) {
    f32x4 v0[8], v1[8];
    float ls[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sidx = s0 + u < n_slots ? s0 + u : s0;
      ls[u] = s0 + u < n_slots ? pl[(int64_t)sidx * a.rows_max] : -INFINITY;
      const f16x8 h = *reinterpret_cast<const f16x8*>(po + sidx * sstride);
      v0[u] = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
      v1[u] = f32x4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
    }
    float mb = M;
#pragma unroll
    for (int u = 0; u < 8; ++u) mb = fmaxf(mb, ls[u]);
    // slot 0 covers token 0, which every row attends: mb is finite from the
    // first round on, and M = -inf only there (acc and W are 0)
    const float scale = exp2f(M - mb);
    acc0 *= scale;
    acc1 *= scale;
    W *= scale;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float wgt = exp2f(ls[u] - mb);
      acc0 += v0[u] * wgt;
      acc1 += v1[u] * wgt;
      W += wgt;
    }
    M = mb;
  }
  const float inv = 1.f / W;
  const int qi = n / a.gqa, gh = n - qi * a.gqa;
  const int64_t orow = (int64_t)(c[kCombRowStart] + qi) * a.hq + h * a.gqa + gh;
  f16x8 hv = {(f16)(acc0[0] * inv), (f16)(acc0[1] * inv), (f16)(acc0[2] * inv),
              (f16)(acc0[3] * inv), (f16)(acc1[0] * inv), (f16)(acc1[1] * inv),
              (f16)(acc1[2] * inv), (f16)(acc1[3] * inv)};
  *reinterpret_cast<f16x8*>(a.o + orow * D + 8 * d8) = hv;
  if (d8 == 0 && a.lse != nullptr) a.lse[orow] = (M + __log2f(W)) * kLn2;
}

template <int NT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void paged_attn_kernel(AttnArgs a) {
  extern __shared__ __align__(16) char smem_raw[];
  lds_char* ring = (lds_char*)smem_raw;
  uint64_t* s_items = (uint64_t*)(smem_raw + kLdsItems);
  int32_t* s_rec = (int32_t*)(smem_raw + kLdsRecs);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;   // row of a 16-row tile (B/D column)
  const int lg = lane >> 4;   // k-group of the MFMA operands
  const bool computes = wave < NT;  // this wave's row tile: rows 16*wave .. +15

  // The worker's records sit at a fixed stride in the plan, so they load in
  // parallel with the worker-table row that counts them.
  const int wid = blockIdx.x;
  const int32_t* wrow = a.workers + kWorkerWords * wid;
  const int n_pc = wrow[1] - wrow[0];  // <= piece_stride <= kMaxWorkerPieces (host-checked)
  const int32_t* recs = a.pieces + (int64_t)wid * a.piece_stride * kPieceWords;
  for (int i = threadIdx.x; i < a.piece_stride * kPieceWords; i += kThreads) s_rec[i] = recs[i];
  __syncthreads();

  auto rec = [&](int p, int f) {
    return __builtin_amdgcn_readfirstlane(s_rec[p * kPieceWords + f]);
  };
  // ring items of piece p: its blocks
  auto items_of = [&](int p) { return rec(p, kPieceBlkEnd) - rec(p, kPieceBlkBegin); };
  int n_items = 0;
  for (int p = 0; p < n_pc; ++p) n_items += items_of(p);  // <= kMaxWorkerItems

  // Query rows of this wave's row tile for every piece, as the B operand of
  // the score MFMA (lane (lg, lr): dims 32kk + 8lg .. +7 of row lr); rows
  // past a group read its row 0 and are never written.
  f16x8 qall[kMaxWorkerPieces][4];
  if (computes) {
#pragma unroll
    for (int p = 0; p < kMaxWorkerPieces; ++p) {
      const int pp = p < n_pc ? p : 0;
      const int32_t* r = s_rec + pp * kPieceWords;
      const int n = 16 * wave + lr;
      const int nr = n < r[kPieceQLen] * a.gqa ? n : 0;
      const int qi = nr / a.gqa, gh = nr - qi * a.gqa;
      const f16* qrow = a.q + ((int64_t)(r[kPieceRowStart] + qi) * a.hq + r[kPieceHead] * a.gqa + gh) * D;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        qall[p][kk] = n_pc > 0 ? *reinterpret_cast<const f16x8*>(qrow + 32 * kk + 8 * lg) : f16x8{};
    }
  }
  // Item table: one lane per item of the worker.
  {
    const int64_t head_tile = (int64_t)a.layer * a.hkv * BS * D;
    for (int k = threadIdx.x; k < n_items; k += kThreads) {
      int p = 0, base = 0;
      while (p + 1 < n_pc) {
        const int nb = s_rec[p * kPieceWords + kPieceBlkEnd] - s_rec[p * kPieceWords + kPieceBlkBegin];
        if (k < base + nb) break;
        base += nb;
        ++p;
      }
      const int32_t* r = s_rec + p * kPieceWords;
      const int id = a.bt[(int64_t)r[kPieceSeqId] * a.bt_stride + r[kPieceBlkBegin] + k - base];
      const bool ok = id >= 0 && id < a.num_blocks;  // others read block 0, masked
      if (!ok) flag_status(a.status, NSD_STATUS_BAD_BLOCK);
      s_items[k] = (uint64_t)((int64_t)(ok ? id : 0) * a.blk_stride + head_tile +
                              (int64_t)r[kPieceHead] * BS * D) |
                   (ok ? 0ull : kMasked);
    }
  }

  // The query loads complete here, before the ring loads the compiler does
  // not see are issued (a wait for them later would drain the ring).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();  // item table in LDS

  // ---- producer: wave w brings K rows 4w .. 4w+3 and the same V rows ------
  const int ld_tok = 4 * wave + (lane >> 4);
  const f16* k_src = a.k_cache + ld_tok * D + (((lane & 15) ^ swz_k(ld_tok)) << 3);
  const f16* v_src = a.v_cache + ld_tok * D + (((lane & 15) ^ swz_v(ld_tok)) << 3);
  int issued = 0, pslot = 0;
  auto issue = [&]() {
    const uint64_t e = s_items[issued];
    // both halves zero-extended (readfirstlane returns a signed int)
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)e);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(e >> 32)) &
                        (uint32_t)((kMasked - 1) >> 32);
    const int64_t off = (int64_t)(((uint64_t)hi << 32) | lo);
    const lds_char* sl = ring + pslot * kSlot;
    ring_load(lds_address(sl + wave * 1024), k_src + off);
    ring_load(lds_address(sl + kTile + wave * 1024), v_src + off);
    ++issued;
    pslot = pslot + 1 == kRing ? 0 : pslot + 1;
  };
  while (issued < n_items && issued < kRing - 2) issue();

  // ---- consumer ------------------------------------------------------------
  // Score MFMA row i of tile x holds token 8(i/4) + 4x + i%4 of the step's 32
  // (tokens 0-15 in the step's first slot, 16-31 in the second), so lane
  // group g ends with tokens 8g .. 8g+7.
  const int t1 = 8 * (lr >> 2) + (lr & 3), t2 = t1 + 4;
  const int krow1 = (t1 & 15) * kRowBytes, krow2 = (t2 & 15) * kRowBytes;
  const int ksw1 = swz_k(t1 & 15), ksw2 = swz_k(t2 & 15);
  const bool kb1 = t1 >= 16, kb2 = t2 >= 16;
  // transposing V reads: lane (lg, lr) addresses token 8lg + lr/4 (+4 for
  // the high half), dims 4(lr%4) .. +3 of each 16-dim tile
  const int vt_lo = (8 * lg + (lr >> 2)) & 15, vt_hi = vt_lo + 4;
  const bool vb = lg >= 2;  // tokens 16-31: the step's second slot
  const int vrow_lo = kTile + vt_lo * kRowBytes + 8 * (lr & 1);
  const int vrow_hi = kTile + vt_hi * kRowBytes + 8 * (lr & 1);
  const int vsw_lo = swz_v(vt_lo), vsw_hi = swz_v(vt_hi);
  const int vc = (lr & 3) >> 1;

  int cp = 0, ck = 0, cslot = 0;  // piece, item within the piece, ring slot
  int c_items = n_pc > 0 ? items_of(0) : 0;
  int c_blk0 = n_pc > 0 ? rec(0, kPieceBlkBegin) : 0;
  float m = -INFINITY, l = 0.f;  // running max (exp2 domain) and row sum of this lane's row
  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  f16x8 qf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) qf[kk] = qall[0][kk];
  int row_len = 0;  // seq_len of this lane's row (causal bound inside the group)
  int ctx = 0;
  auto start_piece = [&](int p) {
    const int n = 16 * wave + lr;
    const int q_len = rec(p, kPieceQLen);
    ctx = rec(p, kPieceCtx);
    row_len = n < q_len * a.gqa ? ctx + n / a.gqa + 1 : ctx + q_len;
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pp = 0; pp < kMaxWorkerPieces; ++pp)
      if (pp == p) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qf[kk] = qall[pp][kk];
      }
  };
  if (n_pc > 0) start_piece(0);
  // End of piece p: this wave's 16 rows of the output, or of the segment's
  // partial.
  auto store_piece = [&](int p) __attribute__((always_inline)) {
    if (!computes) return;
    const float lt = rows_sum(l);
    const int n = 16 * wave + lr;
    if (n < rec(p, kPieceQLen) * a.gqa) {
      const int slot = rec(p, kPieceSlot);
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const float lse2 = lt > 0.f ? m + __log2f(lt) : -INFINITY;
      const int qi = n / a.gqa, gh = n - qi * a.gqa;
      const int64_t orow = (int64_t)(rec(p, kPieceRowStart) + qi) * a.hq + rec(p, kPieceHead) * a.gqa + gh;
      if (slot < 0) {
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
          const f32x4 ov = acc[mt] * inv;
          f16x4 hv = {(f16)ov[0], (f16)ov[1], (f16)ov[2], (f16)ov[3]};
          *reinterpret_cast<f16x4*>(a.o + orow * D + 16 * mt + 4 * lg) = hv;
        }
        if (lg == 0 && a.lse != nullptr) a.lse[orow] = lse2 * kLn2;
      } else {
        f16* po = a.part_o + ((int64_t)slot * a.rows_max + n) * D + 4 * lg;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
          const f32x4 ov = acc[mt] * inv;
          f16x4 hv = {(f16)ov[0], (f16)ov[1], (f16)ov[2], (f16)ov[3]};
          *reinterpret_cast<f16x4*>(po + 16 * mt) = hv;
        }
        if (lg == 0) a.part_lse[(int64_t)slot * a.rows_max + n] = lse2;
      }
    }
  };

  int done = -1;  // a finished piece whose rows are not stored yet
  for (int i = 0; i < n_items;) {
    // two blocks of the piece, or its last one
    const int step = ck + 2 <= c_items ? 2 : 1;
    wait_ring(issued - i - step);  // this step's blocks landed (this wave's part) ...
    barrier();                     // ... and every wave's; the previous step's slots are free
    // The piece that ended with the previous step is stored here, ahead of
    // this step's loads: the stores then complete in the shadow of those
    // loads instead of delaying the wait for them (a wave's vmcnt retires
    // its memory operations in order, stores included).  The accumulators
    // are reset for the next piece after that.
    if (done >= 0) {
      store_piece(done);
      done = -1;
      start_piece(cp);
    }
    while (issued < n_items && issued < i + kRing) issue();
    const lds_char* sa = ring + cslot * kSlot;
    const lds_char* sb = step == 2 ? ring + (cslot + 1 == kRing ? 0 : cslot + 1) * kSlot : sa;
    if (computes) {
      const uint32_t fa = (uint32_t)(s_items[i] >> 32);
      const uint32_t fb = step == 2 ? (uint32_t)(s_items[i + 1] >> 32) : (uint32_t)(kMasked >> 32);
      const bool ma = __builtin_amdgcn_readfirstlane(fa) & (uint32_t)(kMasked >> 32);
      const bool mb = __builtin_amdgcn_readfirstlane(fb) & (uint32_t)(kMasked >> 32);
      // S^T of the two score tiles: lane (lg, lr) gets tokens 8lg + j (s1)
      // and 8lg + 4 + j (s2), j = 0..3, of query row lr
      f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = {0.f, 0.f, 0.f, 0.f};
      {
        const lds_char* k1 = (kb1 ? sb : sa) + krow1;
        const lds_char* k2 = (kb2 ? sb : sa) + krow2;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const f16x8 a1 = *(const lds_f16x8*)(k1 + (((4 * kk + lg) ^ ksw1) << 4));
          const f16x8 a2 = *(const lds_f16x8*)(k2 + (((4 * kk + lg) ^ ksw2) << 4));
          s1 = mfma_k32(a1, qf[kk], s1);
          s2 = mfma_k32(a2, qf[kk], s2);
        }
      }
      // V^T operands of the 8 dim tiles (issued before the softmax)
      f16x8 va[8];
      {
        const lds_char* vs = vb ? sb : sa;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
          const f16x4 lo = ds_read_tr16(vs + vrow_lo + (((2 * mt + vc) ^ vsw_lo) << 4));
          const f16x4 hi = ds_read_tr16(vs + vrow_hi + (((2 * mt + vc) ^ vsw_hi) << 4));
          va[mt] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
      // online softmax over the step's 32 tokens (exp2 domain)
      float sv[8] = {s1[0], s1[1], s1[2], s1[3], s2[0], s2[1], s2[2], s2[3]};
      const int tok0 = (c_blk0 + ck) * BS;  // first token of the step in the segment
      if (ma || mb || tok0 + 2 * BS > ctx + 1) {  // some token may lie past a row's length
        const bool masked = lg < 2 ? ma : mb;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int t = tok0 + 8 * lg + j;
          if (masked || t >= row_len) sv[j] = -INFINITY;
        }
      }
      float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                       fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      mx = rows_max(mx) * a.scale_log2;  // -inf stays -inf (scale > 0)
      // Lazy running max: move it only when a score exceeds it by 2^8 (the
      // weights stay below 256, exact enough in fp16 and far from fp32
      // overflow); one decision per wave.
      if (__builtin_amdgcn_ballot_w64(mx > m + kLazyMax) != 0) {
        const float m_new = fmaxf(m, mx);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - m_new);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] *= alpha;
        m = m_new;
      }
      const float m_use = m == -INFINITY ? 0.f : m;
      f16x8 pb;
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], a.scale_log2, -m_use));
        psum += pj;
        pb[j] = (f16)pj;
      }
      l += psum;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) acc[mt] = mfma_k32(va[mt], pb, acc[mt]);
    }
    i += step;
    ck += step;
    cslot += step;
    if (cslot >= kRing) cslot -= kRing;
    if (ck == c_items) {  // end of the piece: stored after the next barrier
      done = cp;
      ck = 0;
      if (++cp < n_pc) {
        c_items = items_of(cp);
        c_blk0 = rec(cp, kPieceBlkBegin);
      }
    }
  }
  if (done >= 0) store_piece(done);

}

template <int NT>
int launch_nt(const AttnArgs& args, int grid, hipStream_t stream) {
  static bool attr_set = false;  // per-process: raise the dynamic-LDS limit once
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_attn_kernel<NT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess)
      return fail(NSD_ERR_HIP, "paged_attention: LDS attribute: %s", hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL(paged_attn_kernel<NT>, dim3(grid), dim3(kThreads), kLdsBytes, stream, args);
  return launch_status("paged_attention");
}

template <int NT>
int occupancy_nt(int* blocks) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(
             blocks, reinterpret_cast<const void*>(&paged_attn_kernel<NT>), kThreads,
             kLdsBytes) == hipSuccess
             ? NSD_OK
             : NSD_ERR_HIP;
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_attn_num_workers(int max_rows, int* n_workers) {
  if (n_workers == nullptr) return fail(NSD_ERR_INVALID, "num_workers: null output");
  if (max_rows < 1 || max_rows > kMaxGroupRows)
    return fail(NSD_ERR_INVALID, "num_workers: max_rows=%d outside [1, 64]", max_rows);
  int dev = 0, cus = 0, occ = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail(NSD_ERR_HIP, "num_workers: %s", hipGetErrorString(e));
  const int nt = (max_rows + 15) / 16;
  int rc = nt == 1 ? occupancy_nt<1>(&occ)
         : nt == 2 ? occupancy_nt<2>(&occ)
         : nt == 3 ? occupancy_nt<3>(&occ)
                   : occupancy_nt<4>(&occ);
  if (rc) return fail(rc, "num_workers: occupancy query failed");
  *n_workers = cus * (occ > 0 ? occ : 1);
  return NSD_OK;
}

// Scratch of nsd_paged_attention_noalloc: one copy of this array per GPU the
// library runs on, held until the process ends; it holds the partials.
static __device__ __align__(256) char scratch[NSD_NOALLOC_SCRATCH_BYTES];

namespace {

// Bytes of the partials a plan needs: normalised O (fp16) and log2-sum-exp
// (fp32) per partial slot and row, rounded up to 256 bytes.
int64_t plan_partial_bytes(const int32_t* plan_host) {
  return ((int64_t)plan_host[kPlanSlots] * plan_host[kPlanRowsMax] * (int64_t)(D * 2 + 4) + 255) / 256 * 256;
}

// Shared body of the two attention entry points: `part` holds the partials
// (`part_capacity` bytes).
int paged_attention_impl(const void* q, void* o, float* lse, const void* k_cache,
                         const void* v_cache, int64_t num_blocks, int num_layers, int layer,
                         int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                         const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                         const int32_t* plan_host, const int32_t* plan_dev, void* part,
                         int64_t part_capacity, float softmax_scale, int32_t* status,
                         void* stream) {
  if (head_dim != D) return fail(NSD_ERR_UNSUPPORTED, "paged_attention: head_dim=%d (only 128)", head_dim);
  if (block_size != BS)
    return fail(NSD_ERR_UNSUPPORTED, "paged_attention: block_size=%d (only 16)", block_size);
  if (!plan_host || !plan_dev) return fail(NSD_ERR_INVALID, "paged_attention: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != kPlanVersionValue)
    return fail(NSD_ERR_INVALID, "paged_attention: not a plan (bad magic/version)");
  if (plan_host[kPlanHq] != num_q_heads || plan_host[kPlanHkv] != num_kv_heads)
    return fail(NSD_ERR_INVALID, "paged_attention: plan built for Hq=%d Hkv=%d, called with %d/%d",
                plan_host[kPlanHq], plan_host[kPlanHkv], num_q_heads, num_kv_heads);
  if (num_layers <= 0 || layer < 0 || layer >= num_layers || num_blocks <= 0 || bt_stride <= 0 ||
      bt_rows <= 0)
    return fail(NSD_ERR_INVALID,
                "paged_attention: layer=%d of %d, blocks=%lld, block table %lld x %lld", layer,
                num_layers, (long long)num_blocks, (long long)bt_rows, (long long)bt_stride);
  const int grid = plan_host[kPlanWorkers];
  const int n_combine = plan_host[kPlanCombines];
  const int rows_max = plan_host[kPlanRowsMax];
  const int n_rows_plan = plan_host[kPlanRows];
  if (n_rows_plan == 0 || grid == 0) return NSD_OK;
  if (!q || !o || !k_cache || !v_cache || !block_table)
    return fail(NSD_ERR_INVALID, "paged_attention: null pointer");
  if (!aligned16(q) || !aligned16(o) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(NSD_ERR_INVALID, "paged_attention: q/o/caches must be 16-byte aligned");
  const int nt = (rows_max + 15) / 16;
  const int stride = plan_host[kPlanPieceStride];
  const int64_t n_slots = plan_host[kPlanSlots];
  if (rows_max < 1 || rows_max > kMaxGroupRows || grid % 8 != 0 || stride < 1 ||
      stride > kMaxWorkerPieces || (int64_t)plan_host[kPlanPieces] != (int64_t)grid * stride ||
      plan_host[kPlanMaxBlocks] < 1 || plan_host[kPlanMaxBlocks] > kMaxWorkerBlocks ||
      n_slots < 0 || n_combine < 0)
    return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan header");
  if (plan_host[kPlanBtStride] != bt_stride || plan_host[kPlanBtRows] > bt_rows)
    return fail(NSD_ERR_INVALID,
                "paged_attention: plan built for a block table of %d rows x %d, called with "
                "%lld x %lld",
                plan_host[kPlanBtRows], plan_host[kPlanBtStride], (long long)bt_rows,
                (long long)bt_stride);
  // the kernel trusts the records it claims blocks from: check every one
  // against the buffers and LDS layouts it will touch
  const int gqa = num_q_heads / num_kv_heads;
  const int32_t* wt = plan_host + plan_host[kPlanOffWorkers];
  const int32_t* pr = plan_host + plan_host[kPlanOffPieces];
  for (int w = 0; w < grid; ++w) {
    const int32_t* row = wt + kWorkerWords * w;
    if (row[0] != w * stride || row[1] < row[0] || row[1] - row[0] > stride)
      return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (worker %d)", w);
    int64_t blocks = 0;
    for (int i = row[0]; i < row[1]; ++i) {
      const int32_t* r = pr + kPieceWords * i;
      const int nb = r[kPieceBlkEnd] - r[kPieceBlkBegin];
      const bool base_ok = r[kPieceKvBase] == blocks;
      blocks += nb;
      const bool split_ok =
          r[kPieceSlot] < 0 ||
          (r[kPieceComb] >= 0 && r[kPieceComb] < n_combine && r[kPieceCombFirst] >= 0 &&
           r[kPieceCombSlots] >= 1 && r[kPieceCombFirst] + (int64_t)r[kPieceCombSlots] <= n_slots &&
           r[kPieceSlot] >= r[kPieceCombFirst] &&
           r[kPieceSlot] < r[kPieceCombFirst] + r[kPieceCombSlots]);
      if (r[kPieceBlkBegin] < 0 || nb < 1 || r[kPieceBlkEnd] > bt_stride || r[kPieceSeqId] < 0 ||
          r[kPieceSeqId] >= bt_rows || r[kPieceHead] < 0 || r[kPieceHead] >= num_kv_heads ||
          r[kPieceQLen] < 1 || (int64_t)r[kPieceQLen] * gqa > rows_max ||
          r[kPieceRowStart] < 0 || (int64_t)r[kPieceRowStart] + r[kPieceQLen] > n_rows_plan ||
          !base_ok || blocks > kMaxWorkerBlocks || !split_ok)
        return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (piece %d)", i);
    }
  }
  // ... and every combine record against the partials and the output rows
  const int32_t* cr = plan_host + plan_host[kPlanOffCombines];
  for (int c = 0; c < n_combine; ++c) {
    const int32_t* r = cr + kPieceWords * c;
    if (r[kCombHead] < 0 || r[kCombHead] >= num_kv_heads || r[kCombFirst] < 0 ||
        r[kCombSlots] < 2 || (int64_t)r[kCombFirst] + r[kCombSlots] > n_slots ||
        r[kCombQLen] < 1 || (int64_t)r[kCombQLen] * gqa > rows_max || r[kCombRowStart] < 0 ||
        (int64_t)r[kCombRowStart] + r[kCombQLen] > n_rows_plan)
      return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (combine %d)", c);
  }
  const int64_t part_bytes = plan_partial_bytes(plan_host);
  if (n_combine > 0 && (part == nullptr || part_capacity < part_bytes || !aligned16(part)))
    return fail(NSD_ERR_WORKSPACE,
                "paged_attention: workspace holds %lld partial bytes, the plan needs %lld",
                (long long)part_capacity, (long long)part_bytes);

  AttnArgs args;
  args.q = static_cast<const f16*>(q);
  args.o = static_cast<f16*>(o);
  args.lse = lse;
  args.k_cache = static_cast<const f16*>(k_cache);
  args.v_cache = static_cast<const f16*>(v_cache);
  args.bt = block_table;
  args.bt_stride = bt_stride;
  args.workers = plan_dev + plan_host[kPlanOffWorkers];
  args.pieces = plan_dev + plan_host[kPlanOffPieces];
  args.part_o = static_cast<f16*>(part);
  args.part_lse = reinterpret_cast<float*>(static_cast<f16*>(part) + n_slots * rows_max * D);
  args.combines = plan_dev + plan_host[kPlanOffCombines];
  args.status = status;
  args.num_blocks = num_blocks;
  args.blk_stride = (int64_t)num_layers * num_kv_heads * BS * D;
  args.num_layers = num_layers;
  args.layer = layer;
  args.hq = num_q_heads;
  args.hkv = num_kv_heads;
  args.gqa = gqa;
  args.rows_max = rows_max;
  args.piece_stride = stride;
  args.scale_log2 = softmax_scale * 1.4426950408889634f;

  hipStream_t st = as_stream(stream);
  const int rc = nt == 1   ? launch_nt<1>(args, grid, st)
                 : nt == 2 ? launch_nt<2>(args, grid, st)
                 : nt == 3 ? launch_nt<3>(args, grid, st)
                           : launch_nt<4>(args, grid, st);
  if (rc != NSD_OK || n_combine == 0) return rc;
  hipLaunchKernelGGL(combine_kernel, dim3(n_combine * nt), dim3(256), 0, st, args, nt);
  return launch_status("paged_attention: partial merge");
}

constexpr int64_t kScratchBytes = int64_t(NSD_NOALLOC_SCRATCH_BYTES);

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch_ptr[kMaxScratchDevices] = {};  // device address of `scratch`, per device

// Device address of the current device's scratch, looked up on the first
// call on that device (the array's host-side name is not a device address).
int scratch_for_current_device(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NSD_ERR_HIP, "paged_attention_noalloc: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(NSD_ERR_UNSUPPORTED, "paged_attention_noalloc: device %d >= %d", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(NSD_ERR_HIP, "paged_attention_noalloc: scratch address: %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return NSD_OK;
}

}  // namespace

extern "C" int nsd_paged_attention(const void* q, void* o, float* lse, const void* k_cache,
                                   const void* v_cache, int64_t num_blocks, int num_layers,
                                   int layer, int num_q_heads, int num_kv_heads, int head_dim,
                                   int block_size, const int32_t* block_table, int64_t bt_rows,
                                   int64_t bt_stride, const int32_t* plan_host,
                                   const int32_t* plan_dev,
                                   void* workspace, int64_t workspace_bytes, float softmax_scale,
                                   int32_t* status, void* stream) {
  return paged_attention_impl(q, o, lse, k_cache, v_cache, num_blocks, num_layers, layer,
                              num_q_heads, num_kv_heads, head_dim, block_size, block_table,
                              bt_rows, bt_stride, plan_host, plan_dev, workspace, workspace_bytes,
                              softmax_scale, status, stream);
}

extern "C" int nsd_paged_attention_noalloc(const void* q, void* o, float* lse,
                                           const void* k_cache, const void* v_cache,
                                           int64_t num_blocks, int num_layers, int layer,
                                           int num_q_heads, int num_kv_heads, int head_dim,
                                           int block_size, const int32_t* block_table,
                                           int64_t bt_rows, int64_t bt_stride,
                                           const int32_t* plan_host,
                                           const int32_t* plan_dev, float softmax_scale,
                                           int32_t* status, void* stream) {
  if (!plan_host) return fail(NSD_ERR_INVALID, "paged_attention_noalloc: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != kPlanVersionValue)
    return fail(NSD_ERR_INVALID, "paged_attention_noalloc: not a plan (bad magic/version)");
  const int64_t part_bytes = plan_partial_bytes(plan_host);
  if (part_bytes > kScratchBytes)
    return fail(NSD_ERR_WORKSPACE,
                "paged_attention_noalloc: the plan needs %lld partial bytes; the static scratch "
                "holds %lld (use nsd_paged_attention with a workspace)",
                (long long)part_bytes, (long long)kScratchBytes);
  char* base = nullptr;
  const int rc = scratch_for_current_device(&base);
  if (rc != NSD_OK) return rc;
  return paged_attention_impl(q, o, lse, k_cache, v_cache, num_blocks, num_layers, layer,
                              num_q_heads, num_kv_heads, head_dim, block_size, block_table,
                              bt_rows, bt_stride, plan_host, plan_dev, base, kScratchBytes,
                              softmax_scale, status, stream);
}
