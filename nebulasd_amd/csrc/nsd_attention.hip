// Paged verify/decode attention for gfx950 (MI355X).
//
// Work unit.  A verify group is q_len consecutive rows of one sequence whose
// seq_lens rise by one (ctx+1 .. ctx+q_len); a decode row is a group with
// q_len = 1.  For one (group, kv head) -- a "segment" -- the GQA group x
// q_len query rows (up to 48) are packed as the N dimension of fp16 MFMAs,
// so each K/V tile of the segment is read from HBM exactly once:
//
//   S^T[token][row] = K[token][:] . Q[row][:]            (A = K, B = Q^T)
//   O^T[dim][row]  += V^T[dim][token] . P^T[token][row]  (A = V^T, B = P^T)
//
// S^T uses v_mfma_f32_16x16x32_f16 (k = 32 of the 128 head dims per
// instruction), O^T v_mfma_f32_16x16x16_f16 (k = the 16 tokens of a block).
// Both leave lane (i, g) holding rows i of four consecutive tokens or dims
// 4g .. 4g+3, so the S^T of a block is already the P^T operand of its PV
// product, and a row's online-softmax state lives in one lane column.
//
// Work split.  The host planner cuts every segment into near-equal pieces
// of 16-token blocks (starting on multiples of four blocks, so the waves get
// equal counts); one workgroup of four waves streams one piece.  The pieces
// that fit the device's workgroup slots are bound to workgroups ahead of
// the launch (workgroup i runs on XCD i % 8; the two pieces that share a CU
// pair a long one with a short one); any more (more segments than slots)
// are claimed at run time, one device-scope add per later workgroup, so an
// XCD whose slots free up early takes more.
// Wave w streams blocks w, w + 4, ... of the piece: it brings each block's
// K tile and V tile (4 KB each) straight from HBM into its own LDS double
// buffer with global_load_lds_dwordx4 and computes the previous block while
// the next one is in flight, with no barrier in the loop; the four waves'
// softmax states are merged at the end of the piece.  The block ids are
// read from the block table once per piece, one lane per block.
//
// Ring rows are XOR-swizzled per 16-byte chunk (swz_k, swz_v) by permuting
// which source chunk each lane's DMA fetches, so the score MFMA's K reads
// (16 rows x one chunk per operand) and the transposing V reads
// (ds_read_b64_tr_b16, 4 rows x 32 bytes per 16 lanes) are conflict-free.
// Row maxima and sums across the four 16-lane rows of a wave use gfx950's
// v_permlane16_swap / v_permlane32_swap.  The running max is lazy: it moves
// only when a wave-wide vote finds a score 2^8 above it (exact after the
// final normalisation).
//
// Deterministic by construction: which blocks a piece covers, which wave
// sums which block and the merge order are fixed by the plan; segments cut
// into several pieces write partials (normalised O in fp16, log2-sum-exp in
// fp32) to fixed slots, and a second, small launch merges each such
// segment's slots in slot order (the reference's phase 2).  Identical inputs
// give identical bits whichever CU or workgroup runs which piece.
//
// Layouts (reference swiftLLM/swiftllm/worker/kernels/paged_attn.py):
//   k/v cache [N, L, Hkv, 16, 128] fp16, block (blk, layer, head) = 4 KB
//   contiguous at ((blk*L + layer)*Hkv + head)*16*128 (:49-50, :70-71).
#include <mutex>

#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int D = kHeadDim;           // 128
constexpr int BS = kBlockTokens;      // 16
constexpr int kRowBytes = D * 2;      // one fp16 row of K or V
constexpr int kTile = BS * kRowBytes; // one (block, layer, head) tile: 4 KB
constexpr int kSlot = 2 * kTile;      // a buffer slot: the block's K tile, then its V tile
constexpr int kSlots = 2;             // each wave's double buffer
constexpr int kWaves = 4;             // waves per workgroup (per piece)
constexpr int kThreads = kWaves * kWave;
constexpr int kWaveLds = kSlots * kSlot;
constexpr int kLdsBytes = kWaves * kWaveLds;  // 64 KB: two workgroups per CU
// End-of-piece merge of the waves' softmax states, per 16-row tile: each
// wave's accumulators (8 dim tiles x f32x4 per lane), then its row max and
// row sum (16 floats each); it reuses the buffer's LDS.
constexpr int kMergeAcc = 8 * kWave * 16;
constexpr int kMergeWave = kMergeAcc + 2 * 16 * 4;
static_assert(kWaves * kMergeWave <= kLdsBytes, "merge fits in the buffer's LDS");
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLazyMax = 8.f;       // the running max moves only when exceeded by 2^8
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xF << 8);  // s_waitcnt vmcnt(0), other counters open
#ifndef NSD_ATTN_COMBINE_TABLE
#define NSD_ATTN_COMBINE_TABLE 1
#endif
constexpr bool kUseCombineTable = NSD_ATTN_COMBINE_TABLE != 0;
#ifndef NSD_ATTN_PIECE_TABLE
#define NSD_ATTN_PIECE_TABLE 1
#endif
constexpr bool kUsePieceTable = NSD_ATTN_PIECE_TABLE != 0;
static_assert(kMaxGroupRows <= 48, "at most three 16-row tiles per wave");
static_assert(kMaxPieceBlocks <= kWaves * kWave, "one block id per lane of its wave");

// 16-byte chunk x of row t of a K tile sits at chunk x ^ swz_k(t): the score
// operand reads 16 rows x one chunk, and any 8 consecutive rows land on 8
// distinct chunks.  V rows are read by transposing reads over rows 4g .. 4g+3
// (32 bytes each per 16 lanes): swz_v keeps each 32-byte pair whole and gives
// the 4 rows 4 distinct pairs.
__device__ inline int swz_k(int t) { return t & 7; }
__device__ inline int swz_v(int t) { return 2 * (t & 3); }

struct AttnArgs {
  const f16* q;            // [R, Hq, D]
  f16* o;                  // [R, Hq, D]
  float* lse;              // [R, Hq] natural log, optional
  const f16* k_cache;
  const f16* v_cache;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* pieces;   // plan: piece records, one per workgroup
  f16* part_o;             // [slots, rows_max, D]  normalised O
  float* part_lse;         // [slots, rows_max]  (log2 domain)
  const int32_t* combines; // plan: combine records of the segments cut into pieces
  int32_t* claim;          // claim counter of the claimed records (zero between calls)
  int n_static;            // workgroups below this stream the record of their index
  int n_claimed;           // records after those, claimed in order by the later workgroups
  int n_claim_wgs;         // the later workgroups (each claims once)
  int piece_table;         // 1: the static pieces' block-table positions are in the PieceTable argument
  int32_t* status;
  int64_t num_blocks;
  int64_t blk_stride;      // elements per cache block: L*Hkv*16*128
  int num_layers, layer, hq, hkv, gqa, rows_max;
  float scale_log2;        // softmax_scale * log2(e)
};

// The buffer's loads and waits are inline asm: the compiler does not see
// them, so it neither drains the loads in flight before every LDS read of
// the buffer nor moves its own LDS reads across the asm (memory clobber).
// No other vector-memory operation is issued inside the block loop.  The
// loads are non-temporal: every K/V byte is read once per call, and keeping
// it out of the caches' replacement made the decode and ragged-verify calls
// 7-10% faster than the default policy on the same pieces.
__device__ inline void dma_load(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}
template <int N>
__device__ inline void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

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

// Second launch: merge the partials of the segments cut into pieces, the
// same exp2-domain combine as phase 2 of the reference
// (paged_attn.py:128-149).  The kernel boundary orders it after every partial
// store of the attention launch.
// Row n (of the segment's q_len x GQA rows), dims 8 d8 .. 8 d8 + 7, of a
// split segment of kv head `head` whose partials sit in slots [first, first
// + n_slots): the slots folded in slot order with a running max (online
// log-sum-exp), eight slots' loads in flight at a time, and the row stored.
__device__ inline void merge_row(const AttnArgs& a, int head, int first, int n_slots, int row_start, int n,
                                 int d8) {
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
  const int64_t orow = (int64_t)(row_start + qi) * a.hq + head * a.gqa + gh;
  f16x8 hv = {(f16)(acc0[0] * inv), (f16)(acc0[1] * inv), (f16)(acc0[2] * inv),
              (f16)(acc0[3] * inv), (f16)(acc1[0] * inv), (f16)(acc1[1] * inv),
              (f16)(acc1[2] * inv), (f16)(acc1[3] * inv)};
  *reinterpret_cast<f16x8*>(a.o + orow * D + 8 * d8) = hv;
  if (d8 == 0 && a.lse != nullptr) a.lse[orow] = (M + __log2f(W)) * kLn2;
}

// Workgroup (c, g) merges rows 16g .. 16g+15 of combine record c, one thread
// per (row, 8 dims).
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a, int row_groups) {
  const int32_t* c = a.combines + kPieceWords * (blockIdx.x / row_groups);
  const int n = 16 * (blockIdx.x % row_groups) + (threadIdx.x >> 4);
  if (n >= c[kCombQLen] * a.gqa) return;
  merge_row(a, c[kCombHead], c[kCombFirst], c[kCombSlots], c[kCombRowStart], n, threadIdx.x & 15);
}

// The combine records of plans with at most kCombineTableMax of them, packed
// into the launch's arguments (64 bits each: first slot 20, slots 8, kv head
// 8, first row 20, q_len 8), so that a workgroup reads its record with the
// arguments instead of one more dependent load.
constexpr int kCombineTableMax = 448;
struct CombineTable {
  uint64_t e[kCombineTableMax];
};

// Workgroup (c, g) = (blockIdx.x, blockIdx.y): the entry's address depends on
// the workgroup index alone, so it loads with the other arguments.
__global__ __launch_bounds__(256) void combine_table_kernel(AttnArgs a, CombineTable tab) {
  const uint64_t e = tab.e[blockIdx.x];
  const int n = 16 * (int)blockIdx.y + (threadIdx.x >> 4);
  if (n >= (int)(e >> 56) * a.gqa) return;
  merge_row(a, (int)((e >> 28) & 0xff), (int)(e & 0xfffff), (int)((e >> 20) & 0xff), (int)((e >> 36) & 0xfffff), n,
            threadIdx.x & 15);
}

// One workgroup streams one piece: blocks [blk_begin, blk_end) of a (group,
// kv head) segment, for all of the group's query rows (NT tiles of 16 rows).
// Block j goes to wave j % 4, which streams its blocks through its own
// double buffer and keeps its own softmax state; the four states are merged
// in wave order at the end.
// Block-table positions of the static pieces (32 bits each: seq_id 16, first
// block 16), packed into the launch's arguments when there are at most
// kPieceTableMax of them: a workgroup's block ids then load beside its
// record instead of after it.
constexpr int kPieceTableMax = 920;
struct PieceTable {
  uint32_t e[kPieceTableMax];
};

// The fused prologue (nsd_paged_attention_fused): the rows' q, k and v as
// the q/k/v projection left them, either fp16 rows (row strides in
// elements) or that projection's fp32 split partials [splits][rows][(Hq +
// 2 Hkv) * D] summed in split order and rounded to fp16 (the GEMM output
// rounding); the QK-norm weights (or null), the RoPE tables and the caches
// the new K/V rows are written to.
struct FusedArgs {
  const f16* q;
  const f16* k;
  const f16* v;
  int64_t q_rs, k_rs, v_rs;
  const float* part;
  int64_t part_rs, split_stride;
  int splits;
  const f16* qn;
  const f16* kn;
  float eps;
  const f16* cos_c;
  const f16* sin_c;
  f16* kc;
  f16* vc;
};
struct NoFused {};

template <int NT, class Extra = NoFused>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void paged_attn_kernel(AttnArgs a, PieceTable pt, Extra fx) {
  constexpr bool FUSED = std::is_same_v<Extra, FusedArgs>;
  extern __shared__ __align__(16) char smem_raw[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  lds_char* lds_all = (lds_char*)smem_raw;
  const lds_char* lds = lds_all + wave * kWaveLds;
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

  int rec_idx = blockIdx.x;
  if (rec_idx >= a.n_static) {
    // claim the next record: one device-scope add per workgroup; the last
    // workgroup to claim (every later workgroup claims exactly once) sets
    // the counter back to zero for the next call
    __shared__ int s_ticket;
    if (threadIdx.x == 0) {
      const int t = __hip_atomic_fetch_add(a.claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t == a.n_claim_wgs - 1) __hip_atomic_store(a.claim, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_ticket = t;
    }
    __syncthreads();
    const int t = s_ticket;
    if (t >= a.n_claimed) return;
    rec_idx = a.n_static + t;
  }
  // a static workgroup with the table reads block ids right away (lanes past
  // the piece read a clamped, in-row column and are discarded below)
  const bool tabled = a.piece_table != 0 && (int)blockIdx.x < a.n_static;
  int tab_id = 0;
  if (tabled) {
    const uint32_t e = pt.e[blockIdx.x];
    int64_t col = (int64_t)(e >> 16) + wave + kWaves * lane;
    col = col < a.bt_stride ? col : a.bt_stride - 1;
    tab_id = a.bt[(int64_t)(e & 0xffffu) * a.bt_stride + col];
  }
  // the whole record in one round of scalar loads: the index is uniform and
  // the plan is read-only to the kernel (constant address space)
  using const_i32p = const __attribute__((address_space(4))) int32_t*;
  const const_i32p rec = (const_i32p)(uintptr_t)(a.pieces + (int64_t)__builtin_amdgcn_readfirstlane(rec_idx) * kPieceWords);
  int32_t rv[kPieceWords];
#pragma unroll
  for (int i = 0; i < kPieceWords; ++i) rv[i] = rec[i];
  // every field is used before the empty-record test, so the loads go out
  // together rather than the rest after that test
  asm volatile("" ::"s"(rv[0]), "s"(rv[1]), "s"(rv[2]), "s"(rv[3]), "s"(rv[4]), "s"(rv[5]), "s"(rv[6]),
               "s"(rv[7]), "s"(rv[8]), "s"(rv[9]), "s"(rv[10]), "s"(rv[11]));
  const int q_len = rv[kPieceQLen];
  if (q_len == 0) return;  // an empty record
  const int head = rv[kPieceHead], blk0 = rv[kPieceBlkBegin];
  const int nb = rv[kPieceBlkEnd] - blk0;  // 1 .. kMaxPieceBlocks (host-checked)
  const int my_n = nb > wave ? (nb - wave + kWaves - 1) / kWaves : 0;  // this wave's blocks
  const int row_start = rv[kPieceRowStart], ctx = rv[kPieceCtx];
  const int lr = lane & 15;   // row of a 16-row tile (B/D column)
  const int lg = lane >> 4;   // k-group of the MFMA operands
  const int n_rows = q_len * a.gqa;

  // Block ids of this wave's blocks (block wave + 4i on lane i); ids outside
  // the pool read block 0 and are masked.
  int64_t boff = 0;
  bool bad = false;
  if (lane < my_n) {
    const int id = tabled ? tab_id : a.bt[(int64_t)rv[kPieceSeqId] * a.bt_stride + blk0 + wave + kWaves * lane];
    bad = id < 0 || id >= a.num_blocks;
    boff = (int64_t)(bad ? 0 : id) * a.blk_stride + ((int64_t)a.layer * a.hkv + head) * BS * D;
  }
  const uint64_t bad_mask = __builtin_amdgcn_ballot_w64(bad);
  if (bad_mask != 0 && lane == 0) flag_status(a.status, NSD_STATUS_BAD_BLOCK);

  // DMA sources: load c of a tile fills rows 4c .. 4c+3 (lane l: row 4c + l/16,
  // stored chunk l % 16), fetching the chunk the swizzle puts there.
  int ksrc[4], vsrc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int t = 4 * c + lg;
    ksrc[c] = t * D + (((lane & 15) ^ swz_k(t)) << 3);
    vsrc[c] = t * D + (((lane & 15) ^ swz_v(t)) << 3);
  }
  auto issue = [&](int jj) __attribute__((always_inline)) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)boff, jj);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)boff >> 32), jj);
    const int64_t off = (int64_t)(((uint64_t)hi << 32) | lo);
    const f16* kb = a.k_cache + off;
    const f16* vb = a.v_cache + off;
    const uint32_t slot = lds_base + (jj & 1) * kSlot;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's earlier reads are done
#pragma unroll
    for (int c = 0; c < 4; ++c) dma_load(slot + c * 1024, kb + ksrc[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c) dma_load(slot + kTile + c * 1024, vb + vsrc[c]);
  };
  // one half of block jj's slot: its K tile (v = false) or its V tile
  auto issue_half = [&](int jj, bool v) __attribute__((always_inline)) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)boff, jj);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)boff >> 32), jj);
    const int64_t off = (int64_t)(((uint64_t)hi << 32) | lo);
    const f16* b = (v ? a.v_cache : a.k_cache) + off;
    const uint32_t dst = lds_base + (jj & 1) * kSlot + (v ? kTile : 0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this half's earlier reads are done
#pragma unroll
    for (int c = 0; c < 4; ++c) dma_load(dst + c * 1024, b + (v ? vsrc[c] : ksrc[c]));
  };

  // The first two blocks' loads go out before the query rows', so the rows
  // arrive under the blocks' latency; then everything issued so far has
  // landed (the builtin also tells the compiler its own loads are done, so
  // it inserts no wait for them inside the loop, which would drain the
  // buffer loads too: vmcnt retires in order).
  //
  // Fused prologue.  Rows are computed in the layout of the score MFMA's B
  // operand: lane (lg, lr) holds dims 32kk + 8lg .. +7 of its row (kk < 4),
  // so dims d and d + 64 (a RoPE pair) sit in one lane.  The prologue sums
  // x_d^2 + x_{d+64}^2 over a butterfly of lanes d ^ 32, ^ 16, ^ 8, ^ 4, ^ 2,
  // ^ 1; here that is the same tree: in the lane over kk, across lanes l ^ 32
  // and l ^ 16 (the lg bits), then in the lane over j.  Every value is then
  // the prologue's, bit for bit.
  //
  // New K/V rows: token i of the group sits at position ctx + i of its
  // sequence, in block (ctx + i) / 16.  The wave that streams such a block
  // writes the block's new rows (lane row lr: token own_lo + lr) and has
  // those stores done before it issues the block's DMA: before its first two
  // blocks' loads when the block is one of those, else under the start's
  // wait.  The tokens span at most four consecutive blocks, so a wave owns
  // at most one of them.
  int own_jj = -1, own_lo = 0, own_hi = 0;
  if constexpr (FUSED) {
    const int b_first = ctx / BS, b_last = (ctx + q_len - 1) / BS;
    for (int b = b_first; b <= b_last; ++b) {
      const int rel = b - blk0;
      if (rel >= 0 && rel < nb && (rel & (kWaves - 1)) == wave) {
        own_jj = rel / kWaves;
        own_lo = b * BS - ctx > 0 ? b * BS - ctx : 0;
        own_hi = (b + 1) * BS - ctx < q_len ? (b + 1) * BS - ctx : q_len;
      }
    }
  }
  // a bad block is flagged above and gets no stores
  const bool own = FUSED && own_jj >= 0 && !((bad_mask >> own_jj) & 1);
  // One row of head hd (Hq q heads, then Hkv k, then Hkv v) of the q/k/v
  // projection's fp16 output, in the row layout.
  auto load_row = [&](int64_t r, int hd, f16x8 (&h)[4]) __attribute__((always_inline)) {
    if constexpr (FUSED) {
      if (fx.part == nullptr) {
        const f16* src = hd < a.hq ? fx.q + r * fx.q_rs + (int64_t)hd * D
                         : hd < a.hq + a.hkv ? fx.k + r * fx.k_rs + (int64_t)(hd - a.hq) * D
                                             : fx.v + r * fx.v_rs + (int64_t)(hd - a.hq - a.hkv) * D;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) h[kk] = *reinterpret_cast<const f16x8*>(src + 32 * kk + 8 * lg);
      } else {
        // the splits summed in split order, a split's eight loads together
        const float* prow = fx.part + r * fx.part_rs + (int64_t)hd * D + 8 * lg;
        f32x4 acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = *reinterpret_cast<const f32x4*>(prow + 32 * (c >> 1) + 4 * (c & 1));
        for (int s2 = 1; s2 < fx.splits; ++s2) {
          const float* ps = prow + (int64_t)s2 * fx.split_stride;
          f32x4 add[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) add[c] = *reinterpret_cast<const f32x4*>(ps + 32 * (c >> 1) + 4 * (c & 1));
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[c] += add[c];
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h[kk][j] = f16_of(acc[2 * kk][j]);
            h[kk][j + 4] = f16_of(acc[2 * kk + 1][j]);
          }
      }
    }
  };
  // the norm weights of a row (any readable row when there is no norm)
  auto load_w = [&](const f16* w, f16x8 (&w8)[4]) __attribute__((always_inline)) {
    if constexpr (FUSED) {
      const f16* src = w != nullptr ? w : fx.cos_c;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) w8[kk] = *reinterpret_cast<const f16x8*>(src + 32 * kk + 8 * lg);
    }
  };
  // the RoPE angles of position pos: cos dims 0..63 in cs[0..1], sin in cs[2..3]
  auto load_cs = [&](int64_t pos, f16x8 (&cs)[4]) __attribute__((always_inline)) {
    if constexpr (FUSED) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        cs[kk] = *reinterpret_cast<const f16x8*>(fx.cos_c + pos * (D / 2) + 32 * kk + 8 * lg);
        cs[kk + 2] = *reinterpret_cast<const f16x8*>(fx.sin_c + pos * (D / 2) + 32 * kk + 8 * lg);
      }
    }
  };
  // h RMS-normalised with weights w8 when `norm`, then rotated by cs
  auto norm_rope = [&](const f16x8 (&h)[4], bool norm, const f16x8 (&w8)[4], const f16x8 (&cs)[4],
                       f16x8 (&out)[4]) __attribute__((always_inline)) {
    if constexpr (!FUSED) return;
    float x[4][8];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) x[kk][j] = (float)h[kk][j];
    if (norm) {
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] = sq_pair(x[0][j], x[2][j]) + sq_pair(x[1][j], x[3][j]);
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] += __shfl_xor(u[j], 32, kWave);
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] += __shfl_xor(u[j], 16, kWave);
      const float ss = ((u[0] + u[4]) + (u[2] + u[6])) + ((u[1] + u[5]) + (u[3] + u[7]));
      float eps = 0.f;
      if constexpr (FUSED) eps = fx.eps;
      const float rstd = 1.f / sqrtf(ss / (float)D + eps);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) x[kk][j] = (float)f16_of(x[kk][j] * rstd * (float)w8[kk][j]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float c = (float)cs[kk][j], sn = (float)cs[kk + 2][j];
        out[kk][j] = f16_of(rope_lo(x[kk][j], x[kk + 2][j], c, sn));
        out[kk + 2][j] = f16_of(rope_hi(x[kk][j], x[kk + 2][j], c, sn));
      }
  };
  f16x8 nk[4], nv[4], nkw[4], ncs[4];  // the new rows' k, v, k-norm weights, angles
  auto load_new = [&]() __attribute__((always_inline)) {
    if constexpr (FUSED) {
      const int i = own_lo + lr < own_hi ? own_lo + lr : own_lo;
      load_row(row_start + i, a.hq + head, nk);
      load_row(row_start + i, a.hq + a.hkv + head, nv);
      load_w(fx.kn, nkw);
      load_cs(ctx + i, ncs);
    }
  };
  auto store_new = [&]() __attribute__((always_inline)) {
    if constexpr (FUSED) {
      f16x8 ko[4];
      norm_rope(nk, fx.kn != nullptr, nkw, ncs, ko);
      if (own_lo + lr < own_hi) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)boff, own_jj);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)boff >> 32), own_jj);
        const int64_t at = (int64_t)(((uint64_t)hi << 32) | lo) + (int64_t)((ctx + own_lo + lr) % BS) * D;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          *reinterpret_cast<f16x8*>(fx.kc + at + 32 * kk + 8 * lg) = ko[kk];
          *reinterpret_cast<f16x8*>(fx.vc + at + 32 * kk + 8 * lg) = nv[kk];
        }
      }
    }
  };
  const bool own_early = own && own_jj <= 1;
  if (own_early) {
    load_new();
    store_new();
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the new rows are in the cache before their block's DMA
  }
  if (my_n > 0) issue(0);
  if (my_n > 1) issue(1);
  // Query rows of each row tile as the B operand of the score MFMA (lane
  // (lg, lr): dims 32kk + 8lg .. +7 of row lr); rows past the group read its
  // row 0 and are never stored.
  f16x8 qf[NT][4];
  if constexpr (!FUSED) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int n = 16 * t + lr;
      const int nr = n < n_rows ? n : 0;
      const int qi = nr / a.gqa, gh = nr - qi * a.gqa;
      const f16* qrow = a.q + ((int64_t)(row_start + qi) * a.hq + head * a.gqa + gh) * D;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[t][kk] = *reinterpret_cast<const f16x8*>(qrow + 32 * kk + 8 * lg);
    }
  } else if constexpr (NT == 1) {
    // One row tile: every wave builds it (rows past the group read its row
    // 0 and are never stored), its loads before its arithmetic; no barrier.
    const bool own_late = own && !own_early;
    if (own_late) load_new();
    const int nr = lr < n_rows ? lr : 0;
    const int qi = nr / a.gqa, gh = nr - qi * a.gqa;
    f16x8 qh[4], qcs[4], qw[4];
    load_w(fx.qn, qw);
    load_row(row_start + qi, head * a.gqa + gh, qh);
    load_cs(ctx + qi, qcs);
    if (own_late) store_new();
    norm_rope(qh, fx.qn != nullptr, qw, qcs, qf[0]);
  } else {
    // Wave t < NT builds row tile t (rows past the group are zero and never
    // stored) into the LDS after the buffers; after a barrier every wave
    // reads all the tiles.  The wave's loads (the new rows', its tile's) go
    // out before its arithmetic.
    const bool own_late = own && !own_early;
    if (own_late) load_new();
    const bool builds = wave < NT;  // uniform over the wave
    const int n = 16 * wave + lr;
    f16x8 qh[4], qcs[4], qw[4];
    if (builds) {
      load_w(fx.qn, qw);
      const int nr = n < n_rows ? n : 0;
      const int qi = nr / a.gqa, gh = nr - qi * a.gqa;
      if (n < n_rows) {
        load_row(row_start + qi, head * a.gqa + gh, qh);
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qh[kk] = f16x8{};
      }
      load_cs(ctx + qi, qcs);
    }
    if (own_late) store_new();
    lds_char* qlds = lds_all + kLdsBytes;
    if (builds) {
      f16x8 qo[4];
      norm_rope(qh, fx.qn != nullptr, qw, qcs, qo);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) *(lds_f16x8*)(qlds + ((wave * 4 + kk) * kWave + lane) * 16) = qo[kk];
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[t][kk] = *(const lds_f16x8*)(qlds + ((t * 4 + kk) * kWave + lane) * 16);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

  // LDS read addresses (bytes within a slot): the score operand of k-step kk
  // (row lr, chunk 4kk + lg) and the transposing V read of dim tile mt (row
  // 4lg + lr/4, dims 16mt + 4(lr%4) .. +3).
  int kaddr[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) kaddr[kk] = lr * kRowBytes + (((4 * kk + lg) ^ swz_k(lr)) << 4);
  const int vrow = 4 * lg + (lr >> 2);
  const int vaddr0 = kTile + vrow * kRowBytes + 8 * (lr & 1);
  const int vsw = swz_v(vrow), vc = (lr & 3) >> 1;

  int row_len[NT];  // causal bound of this lane's row in each tile
  float m[NT], l[NT];
  f32x4 acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = 16 * t + lr;
    row_len[t] = n < n_rows ? ctx + n / a.gqa + 1 : ctx + q_len;
    m[t] = -INFINITY;
    l[t] = 0.f;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // One row tile: a block's K and V tiles are waited for and refilled
  // separately (the next-but-one block's K goes out once this block's
  // scores are read, its V once the PV product is); more tiles: a whole
  // block at a time.
  constexpr bool kHalves = NT == 1;
  for (int jj = 0; jj < my_n; ++jj) {
    const bool more1 = jj + 1 < my_n, more2 = jj + 2 < my_n;
    if constexpr (kHalves) {
      // blocks 0 and 1 landed before the loop; for a later block, its K tile
      // is in once at most V(jj), K(jj+1), V(jj+1) are outstanding
      if (jj > 1) {
        if (more1) wait_vm<12>();
        else wait_vm<4>();
      }
    } else if (jj > 0) {  // blocks 0 and 1 are in; block jj + 1 goes into the slot block jj - 1 freed
      if (more1) {
        issue(jj + 1);
        wait_vm<8>();  // this block landed; the next stays in flight
      } else {
        wait_vm<0>();
      }
    }
    const lds_char* sl = lds + (jj & 1) * kSlot;
    const int blk = blk0 + wave + kWaves * jj;
    // S^T of each row tile: lane (lg, lr) gets tokens 4lg .. 4lg+3 of row lr
    f32x4 s[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const f16x8 kop = *(const lds_f16x8*)(sl + kaddr[kk]);
#pragma unroll
      for (int t = 0; t < NT; ++t) s[t] = mfma_k32(kop, qf[t][kk], s[t]);
    }
    if (kHalves && more2) issue_half(jj + 2, false);  // block jj's K tile is read
    const int tok0 = blk * BS + 4 * lg;  // this lane's first token
    const bool masked = (bad_mask >> jj) & 1;
    const bool edge = masked || (blk + 1) * BS > ctx + 1;  // a token may lie past a row's length
    f16x4 pb[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float sv[4] = {s[t][0], s[t][1], s[t][2], s[t][3]};
      if (edge) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (masked || tok0 + r >= row_len[t]) sv[r] = -INFINITY;
      }
      float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      mx = rows_max(mx) * a.scale_log2;  // -inf stays -inf (scale > 0)
      // lazy running max: one decision per wave and tile
      if (__builtin_amdgcn_ballot_w64(mx > m[t] + kLazyMax) != 0) {
        const float m_new = fmaxf(m[t], mx);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[t] - m_new);
        l[t] *= alpha;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) acc[t][mt] *= alpha;
        m[t] = m_new;
      }
      const float m_use = m[t] == -INFINITY ? 0.f : m[t];
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], a.scale_log2, -m_use));
        psum += pj;
        pb[t][r] = (f16)pj;
      }
      l[t] += psum;
    }
    // V(jj) is in once at most K(jj+1), V(jj+1) and K(jj+2) are outstanding
    if (kHalves && jj > 1) {
      if (more2) wait_vm<12>();
      else if (more1) wait_vm<8>();
      else wait_vm<0>();
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const f16x4 va = ds_read_tr16(sl + vaddr0 + (((2 * mt + vc) ^ vsw) << 4));
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t][mt] = mfma_k16(va, pb[t], acc[t][mt]);
    }
    if (kHalves && more2) issue_half(jj + 2, true);  // block jj's V tile is read
  }

  // Merge the four waves' states, one row tile at a time, through the
  // buffer's LDS: wave w then owns dim tiles 2w, 2w + 1 of every row, sums
  // the waves' accumulators for them in wave order, and stores them (the
  // output, or the segment's partial).  Wave 0 writes the rows' LSE.
  const int slot = rv[kPieceSlot];
  float* mrg = (float*)smem_raw;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float lt = rows_sum(l[t]);
    __syncthreads();  // the buffer (or the previous tile's merge) is no longer read
    float* mine = mrg + wave * (kMergeWave / 4);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<f32x4*>(mine + (mt * kWave + lane) * 4) = acc[t][mt];
    if (lg == 0) {
      mine[kMergeAcc / 4 + lr] = m[t];
      mine[kMergeAcc / 4 + 16 + lr] = lt;
    }
    __syncthreads();
    float mw[kWaves], lw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      mw[v] = mrg[v * (kMergeWave / 4) + kMergeAcc / 4 + lr];
      lw[v] = mrg[v * (kMergeWave / 4) + kMergeAcc / 4 + 16 + lr];
      M = fmaxf(M, mw[v]);
    }
    float L = 0.f, sc[kWaves];
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      sc[v] = mw[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[v] - M);
      L += lw[v] * sc[v];
    }
    const int n = 16 * t + lr;
    if (n < n_rows) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const int qi = n / a.gqa, gh = n - qi * a.gqa;
      const int64_t orow = (int64_t)(row_start + qi) * a.hq + head * a.gqa + gh;
      f16* dst = slot < 0 ? a.o + orow * D : a.part_o + ((int64_t)slot * a.rows_max + n) * D;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int mt = 2 * wave + h;
        f32x4 o4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < kWaves; ++v)
          o4 += *reinterpret_cast<const f32x4*>(mrg + v * (kMergeWave / 4) + (mt * kWave + lane) * 4) * sc[v];
        o4 *= inv;
        *reinterpret_cast<f16x4*>(dst + 16 * mt + 4 * lg) = f16x4{(f16)o4[0], (f16)o4[1], (f16)o4[2], (f16)o4[3]};
      }
      if (wave == 0 && lg == 0) {
        const float lse2 = L > 0.f ? M + __log2f(L) : -INFINITY;
        if (slot >= 0) a.part_lse[(int64_t)slot * a.rows_max + n] = lse2;
        else if (a.lse != nullptr) a.lse[orow] = lse2 * kLn2;
      }
    }
  }
}

template <int NT>
int launch_nt(const AttnArgs& args, const PieceTable& pt, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((paged_attn_kernel<NT, NoFused>), dim3(grid), dim3(kThreads), kLdsBytes, stream, args, pt,
                     NoFused{});
  return launch_status("paged_attention");
}

// The fused kernel's LDS: the buffers, then its query row tiles (4 KB each)
// when it has more than one.
template <int NT>
constexpr int fused_lds_bytes() { return kLdsBytes + (NT > 1 ? NT * 16 * D * 2 : 0); }
static_assert(2 * fused_lds_bytes<3>() <= 160 * 1024, "two fused workgroups per CU");

template <int NT>
int launch_nt_fused(const AttnArgs& args, const PieceTable& pt, const FusedArgs& f, int grid, hipStream_t stream) {
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_attn_kernel<NT, FusedArgs>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, fused_lds_bytes<NT>());
  if (attr != hipSuccess)
    return fail(NSD_ERR_HIP, "paged_attention_fused: LDS attribute: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL((paged_attn_kernel<NT, FusedArgs>), dim3(grid), dim3(kThreads), fused_lds_bytes<NT>(), stream,
                     args, pt, f);
  return launch_status("paged_attention_fused");
}

template <int NT>
int occupancy_nt(int* blocks) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(
             blocks, reinterpret_cast<const void*>(&paged_attn_kernel<NT, NoFused>), kThreads, kLdsBytes) == hipSuccess
             ? NSD_OK
             : NSD_ERR_HIP;
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_attn_num_workers(int max_rows, int* n_workers) {
  if (n_workers == nullptr) return fail(NSD_ERR_INVALID, "num_workers: null output");
  if (max_rows < 1 || max_rows > kMaxGroupRows)
    return fail(NSD_ERR_INVALID, "num_workers: max_rows=%d outside [1, %d]", max_rows, kMaxGroupRows);
  int dev = 0, cus = 0, occ = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail(NSD_ERR_HIP, "num_workers: %s", hipGetErrorString(e));
  const int nt = (max_rows + 15) / 16;
  int rc = nt == 1 ? occupancy_nt<1>(&occ) : nt == 2 ? occupancy_nt<2>(&occ) : occupancy_nt<3>(&occ);
  if (rc) return fail(rc, "num_workers: occupancy query failed");
  *n_workers = cus * (occ > 0 ? occ : 1);  // one piece per workgroup
  return NSD_OK;
}

// Scratch of nsd_paged_attention_noalloc: one copy of this array per GPU the
// library runs on, held until the process ends; it holds the partials.
static __device__ __align__(256) char scratch[NSD_NOALLOC_SCRATCH_BYTES];

namespace {

// Workspace bytes a plan needs: the claim counter (when it has claimed
// records) and the partials.
int64_t plan_partial_bytes(const int32_t* plan_host) {
  return plan_workspace_bytes(plan_host[kPlanSlots], plan_host[kPlanRowsMax]);
}

// Shared body of the two attention entry points: `part` holds the partials
// (`part_capacity` bytes).
int paged_attention_impl(const void* q, void* o, float* lse, const void* k_cache,
                         const void* v_cache, int64_t num_blocks, int num_layers, int layer,
                         int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                         const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                         const int32_t* plan_host, const int32_t* plan_dev, void* part,
                         int64_t part_capacity, float softmax_scale, int32_t* status,
                         void* stream, const FusedArgs* fused = nullptr) {
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
  if ((!q && !fused) || !o || !k_cache || !v_cache || !block_table)
    return fail(NSD_ERR_INVALID, "paged_attention: null pointer");
  if ((!fused && !aligned16(q)) || !aligned16(o) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(NSD_ERR_INVALID, "paged_attention: q/o/caches must be 16-byte aligned");
  const int nt = (rows_max + 15) / 16;
  const int64_t n_slots = plan_host[kPlanSlots];
  const int n_static = plan_host[kPlanStatic], n_claimed = plan_host[kPlanClaimed];
  const int n_records = plan_host[kPlanPieces];
  if (rows_max < 1 || rows_max > kMaxGroupRows || n_static < 0 || n_static % kXcds != 0 || n_claimed < 0 ||
      n_records != n_static + n_claimed || grid < n_records || (n_claimed == 0 && grid != n_static) ||
      plan_host[kPlanMaxBlocks] < 1 || plan_host[kPlanMaxBlocks] > kMaxPieceBlocks || n_slots < 0 ||
      n_combine < 0)
    return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan header");
  if (plan_host[kPlanBtStride] != bt_stride || plan_host[kPlanBtRows] > bt_rows)
    return fail(NSD_ERR_INVALID,
                "paged_attention: plan built for a block table of %d rows x %d, called with "
                "%lld x %lld",
                plan_host[kPlanBtRows], plan_host[kPlanBtStride], (long long)bt_rows,
                (long long)bt_stride);
  // the kernel trusts the records it streams blocks from: check every one
  // against the buffers it will touch
  const int gqa = num_q_heads / num_kv_heads;
  const int32_t* pr = plan_host + plan_host[kPlanOffPieces];
  for (int i = 0; i < n_records; ++i) {
    const int32_t* r = pr + kPieceWords * i;
    if (r[kPieceQLen] == 0) continue;  // an empty record: its workgroup exits at once
    const int nb = r[kPieceBlkEnd] - r[kPieceBlkBegin];
    const bool split_ok =
        r[kPieceSlot] < 0 ||
        (r[kPieceComb] >= 0 && r[kPieceComb] < n_combine && r[kPieceCombFirst] >= 0 &&
         r[kPieceCombSlots] >= 2 && r[kPieceCombFirst] + (int64_t)r[kPieceCombSlots] <= n_slots &&
         r[kPieceSlot] >= r[kPieceCombFirst] && r[kPieceSlot] < r[kPieceCombFirst] + r[kPieceCombSlots]);
    if (r[kPieceBlkBegin] < 0 || nb < 1 || nb > kMaxPieceBlocks || r[kPieceBlkEnd] > bt_stride ||
        r[kPieceSeqId] < 0 || r[kPieceSeqId] >= bt_rows || r[kPieceHead] < 0 ||
        r[kPieceHead] >= num_kv_heads || r[kPieceQLen] < 1 || (int64_t)r[kPieceQLen] * gqa > rows_max ||
        r[kPieceRowStart] < 0 || (int64_t)r[kPieceRowStart] + r[kPieceQLen] > n_rows_plan ||
        r[kPieceCtx] < 0 || !split_ok)
      return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (piece %d)", i);
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
  if ((n_combine > 0 || n_claimed > 0) && (part == nullptr || part_capacity < part_bytes || !aligned16(part)))
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
  args.pieces = plan_dev + plan_host[kPlanOffPieces];
  char* ws = static_cast<char*>(part);
  args.claim = n_claimed > 0 ? reinterpret_cast<int32_t*>(ws) : nullptr;
  args.n_static = n_static;
  args.n_claimed = n_claimed;
  args.n_claim_wgs = grid - n_static;
  args.part_o = reinterpret_cast<f16*>(ws + kClaimBytes);
  args.part_lse = reinterpret_cast<float*>(args.part_o + n_slots * rows_max * D);
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
  args.scale_log2 = softmax_scale * 1.4426950408889634f;

  hipStream_t st = as_stream(stream);
  // the static pieces' block-table positions, when they fit the arguments
  PieceTable pt;
  args.piece_table = kUsePieceTable && n_static <= kPieceTableMax ? 1 : 0;
  for (int i = 0; args.piece_table && i < n_static; ++i) {
    const int32_t* r = pr + kPieceWords * i;
    const bool live = r[kPieceQLen] != 0;
    const int32_t sid = live ? r[kPieceSeqId] : 0, b0 = live ? r[kPieceBlkBegin] : 0;
    if (sid >= (1 << 16) || b0 >= (1 << 16)) {
      args.piece_table = 0;
      break;
    }
    pt.e[i] = (uint32_t)sid | (uint32_t)b0 << 16;
  }
  const int rc = fused != nullptr
                     ? (nt == 1   ? launch_nt_fused<1>(args, pt, *fused, grid, st)
                        : nt == 2 ? launch_nt_fused<2>(args, pt, *fused, grid, st)
                                  : launch_nt_fused<3>(args, pt, *fused, grid, st))
                 : nt == 1 ? launch_nt<1>(args, pt, grid, st)
                 : nt == 2 ? launch_nt<2>(args, pt, grid, st)
                           : launch_nt<3>(args, pt, grid, st);
  if (rc != NSD_OK || n_combine == 0) return rc;
  const int32_t* crec = plan_host + plan_host[kPlanOffCombines];
  bool packed = kUseCombineTable && n_combine <= kCombineTableMax;
  CombineTable tab;
  for (int c = 0; packed && c < n_combine; ++c) {
    const int32_t* r = crec + kPieceWords * c;
    if (r[kCombFirst] >= (1 << 20) || r[kCombSlots] >= 256 || r[kCombHead] >= 256 || r[kCombRowStart] >= (1 << 20) ||
        r[kCombQLen] >= 256) {
      packed = false;
      break;
    }
    tab.e[c] = (uint64_t)r[kCombFirst] | (uint64_t)r[kCombSlots] << 20 | (uint64_t)r[kCombHead] << 28 |
               (uint64_t)r[kCombRowStart] << 36 | (uint64_t)r[kCombQLen] << 56;
  }
  if (packed)
    hipLaunchKernelGGL(combine_table_kernel, dim3(n_combine, nt), dim3(256), 0, st, args, tab);
  else
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

extern "C" int nsd_paged_attention_fused(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
                                         const void* v, int64_t v_row_stride, const float* partials, int splits,
                                         const void* q_norm_w, const void* k_norm_w, float eps,
                                         const void* cos_cache, const void* sin_cache, int64_t n_positions, void* o,
                                         float* lse, void* k_cache, void* v_cache, int64_t num_blocks,
                                         int num_layers, int layer, int num_q_heads, int num_kv_heads, int head_dim,
                                         int block_size, const int32_t* block_table, int64_t bt_rows,
                                         int64_t bt_stride, const int32_t* plan_host, const int32_t* plan_dev,
                                         void* workspace, int64_t workspace_bytes, float softmax_scale,
                                         int32_t* status, void* stream) {
  if (!plan_host) return fail(NSD_ERR_INVALID, "paged_attention_fused: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != kPlanVersionValue)
    return fail(NSD_ERR_INVALID, "paged_attention_fused: not a plan (bad magic/version)");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(NSD_ERR_INVALID, "paged_attention_fused: num_q_heads=%d, num_kv_heads=%d", num_q_heads,
                num_kv_heads);
  const int64_t rows = plan_host[kPlanRows];
  const int64_t heads = (int64_t)num_q_heads + 2 * num_kv_heads;
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(NSD_ERR_INVALID, "paged_attention_fused: pass both norm weights or neither");
  if (!cos_cache || !sin_cache || n_positions <= 0 || !aligned16(cos_cache) || !aligned16(sin_cache) ||
      (q_norm_w && (!aligned16(q_norm_w) || !aligned16(k_norm_w))))
    return fail(NSD_ERR_INVALID, "paged_attention_fused: RoPE tables and norm weights must be 16-byte aligned");
  if (partials != nullptr) {
    if (splits < 1 || splits > 16 || !aligned16(partials))
      return fail(NSD_ERR_INVALID, "paged_attention_fused: splits=%d (1..16), partials 16-byte aligned", splits);
  } else if (!q || !k || !v || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
             q_row_stride < (int64_t)num_q_heads * D || k_row_stride < (int64_t)num_kv_heads * D ||
             v_row_stride < (int64_t)num_kv_heads * D || q_row_stride % 8 != 0 || k_row_stride % 8 != 0 ||
             v_row_stride % 8 != 0) {
    return fail(NSD_ERR_INVALID,
                "paged_attention_fused: q/k/v rows (16-byte aligned, strides multiples of 8 covering the heads)");
  }
  // every position in the tables; every sequence's new rows in one group
  const int n_groups = plan_host[kPlanGroups];
  const int32_t* grp = plan_host + plan_host[kPlanOffGroups];
  for (int g = 0; g < n_groups; ++g) {
    const int32_t* gr = grp + 4 * g;
    if ((int64_t)gr[3] + gr[1] > n_positions)
      return fail(NSD_ERR_INVALID, "paged_attention_fused: position %lld outside the %lld-row RoPE tables",
                  (long long)gr[3] + gr[1] - 1, (long long)n_positions);
  }
  if (!plan_keeps_sequences_whole(plan_host))
    return fail(NSD_ERR_UNSUPPORTED,
                "paged_attention_fused: a sequence's rows span several verify groups (run the prologue, then "
                "paged_attention)");
  FusedArgs f;
  f.q = static_cast<const f16*>(q);
  f.k = static_cast<const f16*>(k);
  f.v = static_cast<const f16*>(v);
  f.q_rs = q_row_stride;
  f.k_rs = k_row_stride;
  f.v_rs = v_row_stride;
  f.part = partials;
  f.part_rs = heads * D;
  f.split_stride = rows * heads * D;
  f.splits = splits;
  f.qn = static_cast<const f16*>(q_norm_w);
  f.kn = static_cast<const f16*>(k_norm_w);
  f.eps = eps;
  f.cos_c = static_cast<const f16*>(cos_cache);
  f.sin_c = static_cast<const f16*>(sin_cache);
  f.kc = static_cast<f16*>(k_cache);
  f.vc = static_cast<f16*>(v_cache);
  return paged_attention_impl(nullptr, o, lse, k_cache, v_cache, num_blocks, num_layers, layer, num_q_heads,
                              num_kv_heads, head_dim, block_size, block_table, bt_rows, bt_stride, plan_host,
                              plan_dev, workspace, workspace_bytes, softmax_scale, status, stream, &f);
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
