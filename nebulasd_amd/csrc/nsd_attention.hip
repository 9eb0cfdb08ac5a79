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
// S^T uses v_mfma_f32_16x16x32_f16 (k = head dim), O^T uses
// v_mfma_f32_16x16x16_f16 (k = the 16 tokens of one cache block).  Both leave
// a lane holding one query row (lane & 15) of a 16-row tile, so a row's
// online-softmax state lives in one lane column, and the S^T result of a
// block is already the P^T operand of the PV product (lane group g holds
// tokens 4g..4g+3).
//
// Data path per wave and 16-token block:
//   K : 16-byte global loads straight into the MFMA A layout (registers);
//   V : coalesced 16-byte global loads -> per-wave LDS staging (rows padded
//       to 272 B) -> ds_read_b64_tr_b16 transposing reads = V^T A operand;
//   Q : staged once per piece in LDS, read as the B operand.
// A one-block register ring holds the K/V loads of the wave's next block;
// its K is refilled as soon as S^T has consumed it and its V as soon as it
// is staged in LDS.  Eight waves per compute unit (two per SIMD) keep eight
// blocks in flight; the 64-row shape spills a few registers that only the
// per-piece code touches.
//
// Work split.  The host planner cuts the stream of (segment, 16-token block)
// work into contiguous ranges of near-equal cost, one per workgroup
// ("worker"), and there is one workgroup per compute unit.  The workgroup's
// waves claim its range a group of ring-depth blocks at a time from a
// counter in LDS, so a wave that streams faster takes more groups, and merge
// their softmax states through LDS at the end of each piece (in two rounds
// of 64 dims when all eight waves' states for 48 or 64 rows would not fit).  Segments cut
// across workers write fp32 partials (normalised O, log2-sum-exp); the
// workgroup that writes a segment's last partial merges them in the same
// launch.
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

constexpr int D = kHeadDim;         // 128
constexpr int BS = kBlockTokens;     // 16
constexpr int ROWB = D * 2 + 16;     // LDS bytes per staged fp16 row (padded: 16 B bank shift)
constexpr int RS = D + 4;            // LDS row stride (floats) for the wave merge
constexpr float kLn2 = 0.69314718055994531f;


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
  float* part_o;           // [slots, rows_max, D]
  float* part_lse;         // [slots, rows_max]  (log2 domain)
  int32_t* counters;       // [combines] arrival counters, zero between calls
  int32_t* status;
  int64_t num_blocks;
  int64_t blk_stride;      // elements per cache block: L*Hkv*16*128
  int num_layers, layer, hq, hkv, gqa, rows_max;
  int piece_stride;        // plan: piece records per worker
  float scale_log2;        // softmax_scale * log2(e)
};


// Worker id of this workgroup: hardware dispatches workgroup i to XCD i % 8,
// so consecutive workers (which share segments) land on the same XCD/L2.
__device__ inline int worker_id() {
  const int nb = gridDim.x;  // multiple of 8
  const int b = blockIdx.x;
  return (b & 7) * (nb >> 3) + (b >> 3);
}

// Per row-tile count NT: K/V ring depth (= blocks per claimed group) and
// waves per workgroup, shared with the planner.
template <int NT>
struct Tune {
  static constexpr int stages = ring_stages(NT);
  static constexpr int waves = attn_waves(NT);
};

// LDS byte sizes: Q rows, then max(per-wave V staging, wave merge).  The
// merge passes every wave's fp32 state (NT*16 rows of D dims, plus m and l)
// through LDS, in one round when it fits beside Q, else in two rounds of
// D/2 dims each.
constexpr int kLdsDynMax = 160 * 1024 - 2048;  // a compute unit's LDS less the static arrays
static_assert(kMaxWorkerPieces * (kPieceWords + 1) * 4 + 4 <= 2048, "static LDS arrays");
template <int NT>
constexpr int lds_q_bytes() { return NT * 16 * ROWB; }
template <int NT>
constexpr int lds_v_bytes() { return Tune<NT>::waves * BS * ROWB; }
template <int NT>
constexpr int merge_cols() {
  return lds_q_bytes<NT>() + Tune<NT>::waves * NT * 16 * (RS + 2) * 4 <= kLdsDynMax ? D : D / 2;
}
template <int NT>
constexpr int merge_stride() { return merge_cols<NT>() + 4; }  // floats per merged row
template <int NT>
constexpr int lds_merge_bytes() { return Tune<NT>::waves * NT * 16 * (merge_stride<NT>() + 2) * 4; }
// At least half the LDS of a compute unit, so that one workgroup holds a
// compute unit: its waves then share the unit's work through the claims.
constexpr int kLdsHalfCu = 80 * 1024 + 16;
template <int NT>
constexpr size_t lds_bytes() {
  const int need = lds_q_bytes<NT>() + (lds_v_bytes<NT>() > lds_merge_bytes<NT>()
                                            ? lds_v_bytes<NT>()
                                            : lds_merge_bytes<NT>());
  return need > kLdsHalfCu ? need : kLdsHalfCu;
}
static_assert(lds_bytes<1>() <= kLdsDynMax && lds_bytes<2>() <= kLdsDynMax &&
                  lds_bytes<3>() <= kLdsDynMax && lds_bytes<4>() <= kLdsDynMax,
              "attention LDS exceeds a compute unit");



// Partials cross workgroups (and XCDs, whose L2s are not coherent with each
// other inside a kernel).  They are written and read with device-scope (sc1)
// vector accesses through a raw buffer resource, which the L2 keeps coherent
// without the whole-cache write-back and invalidate of an agent-scope fence.
constexpr int kDeviceScope = 16;              // cache-policy bit of sc1 on gfx950
constexpr int kRawBufferConfig = 0x00020000;  // raw 32-bit buffer, no format conversion

__device__ inline __amdgpu_buffer_rsrc_t raw_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes,
                                           kRawBufferConfig);
}
__device__ inline void store_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kDeviceScope);
}
__device__ inline f32x4 load_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDeviceScope));
}

// Merge the partials of a segment cut across workers (run by the workgroup
// that wrote the segment's last partial): thread (row, 8 dims), slots folded
// with a running max (online log-sum-exp), eight slots' loads in flight at a
// time.  Same exp2-domain combine as phase 2 of the reference
// (paged_attn.py:128-149).
__device__ void combine_segment(const AttnArgs& a, int h, int first, int n_slots, int row_start,
                                int n_rows) {
  const int d8 = threadIdx.x & 15;
  const uint32_t sbytes = (uint32_t)a.rows_max * D * 4;  // one slot's O partial
  const __amdgpu_buffer_rsrc_t ro =
      raw_buffer(a.part_o + (int64_t)first * a.rows_max * D, (uint32_t)n_slots * sbytes);
  const float* pl_base = a.part_lse + (int64_t)first * a.rows_max;
  for (int n = threadIdx.x >> 4; n < n_rows; n += blockDim.x / 16) {
    const uint32_t off = ((uint32_t)n * D + 8 * d8) * 4;
    float M = -INFINITY, W = 0.f;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_slots; s0 += 8) {
      f32x4 v0[8], v1[8];
      float ls[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sidx = s0 + u < n_slots ? s0 + u : s0;
        const float l = __hip_atomic_load(pl_base + (int64_t)sidx * a.rows_max + n,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ls[u] = s0 + u < n_slots ? l : -INFINITY;
        v0[u] = load_coherent(ro, sidx * sbytes + off);
        v1[u] = load_coherent(ro, sidx * sbytes + off + 16);
      }
      float mb = M;
#pragma unroll
      for (int u = 0; u < 8; ++u) mb = fmaxf(mb, ls[u]);
      const float scale = exp2f(M - mb);  // M = -inf at start: 0 (acc and W are 0)
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
    const int64_t orow = (int64_t)(row_start + qi) * a.hq + h * a.gqa + gh;
    f16x8 hv = {(f16)(acc0[0] * inv), (f16)(acc0[1] * inv), (f16)(acc0[2] * inv),
                (f16)(acc0[3] * inv), (f16)(acc1[0] * inv), (f16)(acc1[1] * inv),
                (f16)(acc1[2] * inv), (f16)(acc1[3] * inv)};
    *reinterpret_cast<f16x8*>(a.o + orow * D + 8 * d8) = hv;
    if (d8 == 0 && a.lse != nullptr) a.lse[orow] = (M + __log2f(W)) * kLn2;
  }
}

template <int NT>
__global__ __launch_bounds__(Tune<NT>::waves * kWave)
__attribute__((amdgpu_waves_per_eu(Tune<NT>::waves / 4)))
void paged_attn_kernel(AttnArgs a) {
  constexpr int NW = Tune<NT>::waves;
  constexpr int S = Tune<NT>::stages;       // ring depth = blocks per claimed group
  constexpr int NTHR = NW * kWave;
  constexpr int QU = NT * 16 * (D / 8);     // 16-byte units of the staged Q rows
  constexpr int QI = (QU + NTHR - 1) / NTHR;
  constexpr int kPad = INT32_MIN;           // block id of a padding block (masked, reads block 0)
  extern __shared__ __align__(16) char smem_raw[];
  __shared__ int32_t s_rec[kMaxWorkerPieces * kPieceWords];  // this worker's piece records
  __shared__ int s_last[kMaxWorkerPieces];  // piece pc completed its split segment: combine it
  __shared__ int s_claim;                   // first group of blocks nobody has claimed
  lds_char* smem = (lds_char*)smem_raw;
  lds_char* s_q = smem;                                   // [NT*16][ROWB]
  constexpr int MC = merge_cols<NT>();     // dims merged per round
  constexpr int MS = merge_stride<NT>();
  float* s_acc = (float*)(smem_raw + lds_q_bytes<NT>());  // merge: [NW][NT*16][MS] (aliases V)
  float* s_ml = s_acc + NW * NT * 16 * MS;                // merge: [NW][2][NT*16]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;   // row within a 16-row tile (B/D column)
  const int lg = lane >> 4;   // k-group of the MFMA operands
  lds_char* s_v = smem + lds_q_bytes<NT>() + wave * BS * ROWB;  // this wave's V staging
  // transposing-read address of dim tile 0: lane (g, a = lane % 16) points at
  // token 4g + a/4, dims 4*(a%4) .. +3
  const lds_char* tr_src = s_v + (4 * lg + (lr >> 2)) * ROWB + 8 * (lr & 3);

  // The worker's records sit at a fixed stride in the plan, so they load in
  // parallel with the worker-table row that counts them.
  const int wid = worker_id();
  const int32_t* wrow = a.workers + kWorkerWords * wid;
  const int n_pc = wrow[1] - wrow[0];  // <= piece_stride <= kMaxWorkerPieces (host-checked)
  const int32_t* recs = a.pieces + (int64_t)wid * a.piece_stride * kPieceWords;
  for (int i = threadIdx.x; i < a.piece_stride * kPieceWords; i += NTHR) s_rec[i] = recs[i];
  if (threadIdx.x < kMaxWorkerPieces) s_last[threadIdx.x] = 0;
  if (threadIdx.x == 0) s_claim = NW;  // groups 0 .. NW-1 go one per wave
  __syncthreads();

  // Group g of the worker is blocks [S*j, S*j + S) of the piece p holding it,
  // j = g - (groups of the pieces before p); each wave processes the groups
  // it claims in claim order, so its groups only grow.
  auto rec = [&](int p, int f) {
    return __builtin_amdgcn_readfirstlane(s_rec[p * kPieceWords + f]);
  };
  auto gstart = [&](int p) { return p == 0 ? 0 : rec(p - 1, kPieceGroupEnd); };
  const int n_groups = n_pc > 0 ? rec(n_pc - 1, kPieceGroupEnd) : 0;
  // piece of group g, searching on from piece p; n_pc past the last group
  auto resolve = [&](int g, int p) {
    if (g >= n_groups) return n_pc;
    while (g >= rec(p, kPieceGroupEnd)) ++p;
    return p;
  };
  // raw block ids of group g of piece p in lanes 0 .. S-1 (kPad past the piece)
  auto group_ids = [&](int g, int p) -> int {
    int64_t idx = 0;
    bool ok = false;
    if (p < n_pc) {
      const int b0 = rec(p, kPieceBlkBegin);
      const int blk = (g - gstart(p)) * S + lane;
      ok = lane < S && blk < rec(p, kPieceBlkEnd) - b0;
      idx = (int64_t)rec(p, kPieceSeqId) * a.bt_stride + b0 + blk;
    }
    const int v = a.bt[ok ? idx : 0];
    return ok ? v : kPad;
  };
  auto claim_group = [&]() {  // lane 0 receives the claimed group
    int c = 0;
    if (lane == 0) c = atomicAdd(&s_claim, 1);
    return c;
  };
  auto head_base = [&](const f16* cache, int p) {
    const int h = p < n_pc ? rec(p, kPieceHead) : 0;
    return cache + ((int64_t)a.layer * a.hkv + h) * BS * D;
  };
  // Q rows of piece p, 16 B per thread and step (unit u: row u/16, column
  // u%16).  Every lane loads: lanes past the piece's rows (or past the last
  // piece) read q[0], and staging writes zeros for them.
  auto q_rows = [&](int p) { return p < n_pc ? rec(p, kPieceQLen) * a.gqa : 0; };
  auto store_q = [&](int p, const u32x4 (&qv)[QI]) {
    const int n_rows = q_rows(p);
#pragma unroll
    for (int i = 0; i < QI; ++i) {
      const int u = threadIdx.x + i * NTHR;
      if (u < QU)
        *(lds_u32x4*)(s_q + (u >> 4) * ROWB + (u & 15) * 16) =
            (u >> 4) < n_rows ? qv[i] : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto load_q = [&](int p, u32x4 (&qv)[QI]) {
    const int n_rows = q_rows(p);
    const int row_start = p < n_pc ? rec(p, kPieceRowStart) : 0;
    const int h = p < n_pc ? rec(p, kPieceHead) : 0;
#pragma unroll
    for (int i = 0; i < QI; ++i) {
      const int n = (threadIdx.x + i * NTHR) >> 4;
      const int qi = n / a.gqa, gh = n - qi * a.gqa;
      const u32x4* src = reinterpret_cast<const u32x4*>(
          a.q + ((int64_t)(row_start + qi) * a.hq + h * a.gqa + gh) * D + (threadIdx.x & 15) * 8);
      qv[i] = *(n < n_rows ? src : reinterpret_cast<const u32x4*>(a.q));
    }
  };

  // Ring of in-flight K/V blocks: stage st holds block st of a group.  Every
  // refill issues its loads (a padding or out-of-pool block reads pool block
  // 0 and is masked), so the compiler counts the loads in flight behind each
  // block exactly and never drains the ring early.
  bool bad_block = false;  // reported once, at the end
  f16x8 kr[S][4];
  u32x4 vr[S][4];
  int bid[S];
  // pool offset of block `id` (padding and bad ids read block 0; bid < 0 masks them)
  auto block_offset = [&](auto stage, int id) -> int64_t {
    constexpr int st = decltype(stage)::value;
    const bool ok = id >= 0 && id < a.num_blocks;
    bad_block |= !ok && id != kPad;
    bid[st] = ok ? id : -1;
    return (int64_t)(ok ? id : 0) * a.blk_stride;
  };
  auto issue_k = [&](auto stage, const f16* kb, int64_t off) {
    constexpr int st = decltype(stage)::value;
    const f16* kp = kb + off + lr * D + lg * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kr[st][kk] = *reinterpret_cast<const f16x8*>(kp + kk * 32);
  };
  auto issue_v = [&](auto stage, const f16* vb, int64_t off) {
    constexpr int st = decltype(stage)::value;
    const f16* vp = vb + off + lg * D + lr * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) vr[st][i] = *reinterpret_cast<const u32x4*>(vp + 4 * i * D);
  };

  // Claims run one group ahead of the refills: while group g_cur is
  // processed, the ring is refilled with g_nxt (ids known) and the ids of
  // the group after it are loaded.
  // Q of the first piece loads first, so staging it waits for nothing else.
  u32x4 qv[QI];
  load_q(0, qv);
  int g_cur = wave;
  const int p_cur = resolve(g_cur, 0);
  const int cur_ids = group_ids(g_cur, p_cur);
  int g_nxt = __builtin_amdgcn_readfirstlane(claim_group());
  int p_nxt = resolve(g_nxt, p_cur);
  int nxt_ids = group_ids(g_nxt, p_nxt);
  int claim = claim_group();  // the group after g_nxt
  {
    const f16* kb = head_base(a.k_cache, p_cur);
    const f16* vb = head_base(a.v_cache, p_cur);
    static_for<S>([&](auto st) {
      const int64_t off = block_offset(st, __builtin_amdgcn_readlane(cur_ids, decltype(st)::value));
      issue_k(st, kb, off);
      issue_v(st, vb, off);
    });
  }
  const f16* kb_n = head_base(a.k_cache, p_nxt);
  const f16* vb_n = head_base(a.v_cache, p_nxt);
  store_q(0, qv);

  for (int pc = 0; pc < n_pc; ++pc) {
    __syncthreads();  // Q staged; every wave is past the previous piece's merge

    const int q_len = rec(pc, kPieceQLen), ctx = rec(pc, kPieceCtx);
    const int b_begin = rec(pc, kPieceBlkBegin);
    const int g_begin = gstart(pc), g_end = rec(pc, kPieceGroupEnd);
    const int n_rows = q_len * a.gqa;
    const int total = ctx + q_len;  // tokens of the segment
    int sl[NT];  // seq_len of the lane's row (causal bound inside the group)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = 16 * j + lr;
      sl[j] = n < n_rows ? ctx + n / a.gqa + 1 : total;
    }
    float m[NT], l[NT];
    f32x4 acc[NT][8];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    int g_nn = 0, p_nn = n_pc, nn_ids = kPad;  // the group after g_nxt

    // One block: scores, refill the stage, stage V, softmax, PV.  `blk` is
    // the block's index in the segment.
    auto step = [&](auto stage, int blk) {
      constexpr int st = decltype(stage)::value;
      // S^T: lane (lg, lr) gets scores of row 16j+lr for tokens 16*blk + 4lg + i.
      // (Q is re-read from LDS every block rather than held in registers.)
      const lds_char* qrow = s_q + lr * ROWB + lg * 16;
      asm volatile("" : "+v"(qrow));
      f32x4 s[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const f16x8 qb = *(const lds_f16x8*)(qrow + 16 * j * ROWB + kk * 64);
          t = mfma_k32(kr[st][kk], qb, t);
        }
        s[j] = t;
      }
      if constexpr (st == 0) {
        // the group after g_nxt: its ids load ahead of this group's refills
        g_nn = __builtin_amdgcn_readfirstlane(claim);
        p_nn = resolve(g_nn, p_nxt);
        nn_ids = group_ids(g_nn, p_nn);
        claim = claim_group();
      }
      // refill this stage with block st of g_nxt: K now, V once this
      // block's V is staged in LDS (tokens 4i + lg)
      const int id_n = __builtin_amdgcn_readlane(nxt_ids, st);
      const bool valid = bid[st] >= 0;
      const int64_t off_n = block_offset(stage, id_n);
      issue_k(stage, kb_n, off_n);
#pragma unroll
      for (int i = 0; i < 4; ++i) *(lds_u32x4*)(s_v + (4 * i + lg) * ROWB + lr * 16) = vr[st][i];
      issue_v(stage, vb_n, off_n);

      // online softmax in the exp2 domain, one row per lane column
      const int t0 = blk * BS + 4 * lg;
      f16x4 pb[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = (valid && t0 + i < sl[j]) ? s[j][i] * a.scale_log2 : -INFINITY;
          s[j][i] = v;
          mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m[j], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m[j] - m_use);
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = exp2f(s[j][i] - m_use);
          psum += p;
          pb[j][i] = (f16)p;
        }
        l[j] = l[j] * alpha + psum;
        m[j] = m_new;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) acc[j][mt] *= alpha;
      }
      // O^T += V^T P^T, one transposing read per 16-dim tile
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const f16x4 va = ds_read_tr16(tr_src + 32 * mt);
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j][mt] = mfma_k16(va, pb[j], acc[j][mt]);
      }
    };

    // This wave's groups of the piece; the ring carries on into the next
    // piece's groups (or padding) without draining.
    auto group = [&]() {
      // The next piece's Q is loaded ahead of the refills of this wave's last
      // group of the piece (g_nxt lies past it), so the merge that stages it
      // waits for it with the count of loads behind it known.
      if (g_nxt >= g_end && pc + 1 < n_pc) load_q(pc + 1, qv);
      const int blk0 = b_begin + (g_cur - g_begin) * S;
      static_for<S>([&](auto st) { step(st, blk0 + decltype(st)::value); });
      g_cur = g_nxt;
      g_nxt = g_nn;
      p_nxt = p_nn;
      nxt_ids = nn_ids;
      kb_n = head_base(a.k_cache, p_nxt);
      vb_n = head_base(a.v_cache, p_nxt);
    };
    if (g_cur < g_end) {
      do group();
      while (g_cur < g_end);
    } else if (pc + 1 < n_pc) {
      // no group of this piece: load the next Q and wait for it now (this
      // wave has nothing to overlap until the merge)
      load_q(pc + 1, qv);
#pragma unroll
      for (int i = 0; i < QI; ++i) asm volatile("" : "+v"(qv[i]));
    }

    // Row sums across the four k-groups.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      l[j] += __shfl_xor(l[j], 16, kWave);
      l[j] += __shfl_xor(l[j], 32, kWave);
    }

    // Merge the waves' states through LDS, D/MC rounds of MC dims: every
    // wave writes its live rows (acc, m, l; empty if it took no group of the
    // piece), then all threads combine them, four dims per thread and step,
    // and write the fp16 output (or the fp32 partial).
    __syncthreads();  // every wave is done with its V staging (aliased below) and Q
    if (pc + 1 < n_pc) store_q(pc + 1, qv);
    const int slot = rec(pc, kPieceSlot), row_start = rec(pc, kPieceRowStart);
    const int h = rec(pc, kPieceHead);
    const __amdgpu_buffer_rsrc_t rpart =
        raw_buffer(a.part_o + (int64_t)(slot < 0 ? 0 : slot) * a.rows_max * D,
                   (uint32_t)a.rows_max * D * 4);
    static_for<D / MC>([&](auto round) {
      constexpr int r = decltype(round)::value;
      constexpr int MT = MC / 16;  // acc tiles per round
      if (r > 0) __syncthreads();  // every thread has read the previous round
      {
        float* ma = s_acc + wave * NT * 16 * MS;
        float* mm = s_ml + wave * 2 * NT * 16;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int n = 16 * j + lr;
          if (n < n_rows) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              *reinterpret_cast<f32x4*>(ma + n * MS + 16 * mt + 4 * lg) = acc[j][r * MT + mt];
            if (r == 0 && lg == 0) {
              mm[n] = m[j];
              mm[NT * 16 + n] = l[j];
            }
          }
        }
      }
      __syncthreads();
      for (int idx = threadIdx.x; idx < n_rows * (MC / 4); idx += NTHR) {
        const int n = idx / (MC / 4), c4 = idx % (MC / 4);
        const int col = r * MC + 4 * c4;
        float mw[NW], lw[NW], M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          mw[w] = s_ml[w * 2 * NT * 16 + n];
          lw[w] = s_ml[w * 2 * NT * 16 + NT * 16 + n];
          M = fmaxf(M, mw[w]);
        }
        const float M_use = M == -INFINITY ? 0.f : M;
        f32x4 ov = {0.f, 0.f, 0.f, 0.f};
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {  // a wave with no block of the piece has m = -inf
          const float f = exp2f(mw[w] - M_use);
          L += lw[w] * f;
          ov += *reinterpret_cast<const f32x4*>(s_acc + (w * NT * 16 + n) * MS + 4 * c4) * f;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        ov *= inv;
        const int qi = n / a.gqa, gh = n - qi * a.gqa;
        const int64_t orow = (int64_t)(row_start + qi) * a.hq + h * a.gqa + gh;
        const float lse2 = L > 0.f ? M + __log2f(L) : -INFINITY;
        if (slot < 0) {
          f16x4 hv = {(f16)ov[0], (f16)ov[1], (f16)ov[2], (f16)ov[3]};
          *reinterpret_cast<f16x4*>(a.o + orow * D + col) = hv;
          if (col == 0 && a.lse != nullptr) a.lse[orow] = lse2 * kLn2;
        } else {
          store_coherent(rpart, ((uint32_t)n * D + col) * 4, ov);
          if (col == 0)
            __hip_atomic_store(a.part_lse + (int64_t)slot * a.rows_max + n, lse2,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    });
  }

  // Arrivals of split segments, once every wave's partial stores are
  // complete: one per piece, and the workgroup that brings a segment's last
  // arrival merges its partials.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // keeps the stores above
  __builtin_amdgcn_s_waitcnt(0);                           // ... and completed
  __syncthreads();
  if (threadIdx.x < n_pc) {
    const int32_t* r = s_rec + threadIdx.x * kPieceWords;
    if (r[kPieceSlot] >= 0) {
      const int old = __hip_atomic_fetch_add(a.counters + r[kPieceComb], 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      if (old == r[kPieceCombSlots] - 1) s_last[threadIdx.x] = 1;
    }
  }
  __syncthreads();
  for (int pc = 0; pc < n_pc; ++pc) {
    if (s_last[pc]) {
      combine_segment(a, rec(pc, kPieceHead), rec(pc, kPieceCombFirst), rec(pc, kPieceCombSlots),
                      rec(pc, kPieceRowStart), rec(pc, kPieceQLen) * a.gqa);
      if (threadIdx.x == 0)
        __hip_atomic_store(a.counters + rec(pc, kPieceComb), 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (bad_block) flag_status(a.status, NSD_STATUS_BAD_BLOCK);
}

template <int NT>
int launch_nt(const AttnArgs& args, int grid, hipStream_t stream) {
  static bool attr_set = false;  // per-process: raise the dynamic-LDS limit once
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_attn_kernel<NT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds_bytes<NT>());
    if (e != hipSuccess)
      return fail(NSD_ERR_HIP, "paged_attention: LDS attribute: %s", hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL(paged_attn_kernel<NT>, dim3(grid), dim3(Tune<NT>::waves * kWave),
                     lds_bytes<NT>(), stream,
                     args);
  return launch_status("paged_attention");
}

template <int NT>
int occupancy_nt(int* blocks) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(
             blocks, reinterpret_cast<const void*>(&paged_attn_kernel<NT>), Tune<NT>::waves * kWave,
             lds_bytes<NT>()) == hipSuccess
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
// library runs on, held until the process ends.  Arrival counters sit at its
// start (a fixed place, so every call finds them at zero: each launch leaves
// the counters it used at zero), the partials after them.
static __device__ __align__(256) char scratch[NSD_NOALLOC_SCRATCH_BYTES];

namespace {

// Bytes of the fp32 partials a plan needs: normalised O and log2-sum-exp
// per partial slot, rounded up to 256 bytes.
int64_t plan_partial_bytes(const int32_t* plan_host) {
  return ((int64_t)plan_host[kPlanSlots] * plan_host[kPlanRowsMax] * (int64_t)(D + 1) * 4 + 255) /
         256 * 256;
}

// Shared body of the two attention entry points: `part` holds the partials
// (`part_capacity` bytes) and `counters` the arrival counters
// (`counter_capacity` of them, zero between calls).
int paged_attention_impl(const void* q, void* o, float* lse, const void* k_cache,
                         const void* v_cache, int64_t num_blocks, int num_layers, int layer,
                         int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                         const int32_t* block_table, int64_t bt_stride, const int32_t* plan_host,
                         const int32_t* plan_dev, void* part, int64_t part_capacity,
                         int32_t* counters, int64_t counter_capacity, float softmax_scale,
                         int32_t* status, void* stream) {
  if (head_dim != D) return fail(NSD_ERR_UNSUPPORTED, "paged_attention: head_dim=%d (only 128)", head_dim);
  if (block_size != BS)
    return fail(NSD_ERR_UNSUPPORTED, "paged_attention: block_size=%d (only 16)", block_size);
  if (!plan_host || !plan_dev) return fail(NSD_ERR_INVALID, "paged_attention: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != kPlanVersionValue)
    return fail(NSD_ERR_INVALID, "paged_attention: not a plan (bad magic/version)");
  if (plan_host[kPlanHq] != num_q_heads || plan_host[kPlanHkv] != num_kv_heads)
    return fail(NSD_ERR_INVALID, "paged_attention: plan built for Hq=%d Hkv=%d, called with %d/%d",
                plan_host[kPlanHq], plan_host[kPlanHkv], num_q_heads, num_kv_heads);
  if (num_layers <= 0 || layer < 0 || layer >= num_layers || num_blocks <= 0 || bt_stride <= 0)
    return fail(NSD_ERR_INVALID, "paged_attention: layer=%d of %d, blocks=%lld, bt_stride=%lld",
                layer, num_layers, (long long)num_blocks, (long long)bt_stride);
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
      plan_host[kPlanRingStages] != ring_stages(nt) || n_slots < 0 || n_combine < 0)
    return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan header");
  // the kernel trusts the records it claims blocks from: check every one
  // against the buffers and LDS layouts it will touch
  const int gqa = num_q_heads / num_kv_heads;
  const int32_t* wt = plan_host + plan_host[kPlanOffWorkers];
  const int32_t* pr = plan_host + plan_host[kPlanOffPieces];
  for (int w = 0; w < grid; ++w) {
    const int32_t* row = wt + kWorkerWords * w;
    if (row[0] != w * stride || row[1] < row[0] || row[1] - row[0] > stride)
      return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (worker %d)", w);
    int64_t groups = 0;
    for (int i = row[0]; i < row[1]; ++i) {
      const int32_t* r = pr + kPieceWords * i;
      const int nb = r[kPieceBlkEnd] - r[kPieceBlkBegin];
      groups += (nb + ring_stages(nt) - 1) / ring_stages(nt);
      const bool split_ok =
          r[kPieceSlot] < 0 ||
          (r[kPieceComb] >= 0 && r[kPieceComb] < n_combine && r[kPieceCombFirst] >= 0 &&
           r[kPieceCombSlots] >= 1 && r[kPieceCombFirst] + (int64_t)r[kPieceCombSlots] <= n_slots &&
           r[kPieceSlot] >= r[kPieceCombFirst] &&
           r[kPieceSlot] < r[kPieceCombFirst] + r[kPieceCombSlots]);
      if (r[kPieceBlkBegin] < 0 || nb < 1 || r[kPieceBlkEnd] > bt_stride || r[kPieceSeqId] < 0 ||
          r[kPieceHead] < 0 || r[kPieceHead] >= num_kv_heads || r[kPieceQLen] < 1 ||
          (int64_t)r[kPieceQLen] * gqa > rows_max || r[kPieceRowStart] < 0 ||
          (int64_t)r[kPieceRowStart] + r[kPieceQLen] > n_rows_plan || r[kPieceGroupEnd] != groups ||
          !split_ok)
        return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan (piece %d)", i);
    }
  }
  const int64_t part_bytes = plan_partial_bytes(plan_host);
  if (n_combine > 0 && (part == nullptr || part_capacity < part_bytes || !aligned16(part) ||
                        counters == nullptr || counter_capacity < n_combine))
    return fail(NSD_ERR_WORKSPACE,
                "paged_attention: workspace holds %lld partial bytes and %lld counters, the plan "
                "needs %lld and %d",
                (long long)part_capacity, (long long)counter_capacity, (long long)part_bytes,
                n_combine);

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
  args.part_o = static_cast<float*>(part);
  args.part_lse = static_cast<float*>(part) + n_slots * rows_max * D;
  args.counters = counters;
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
  switch (nt) {
    case 1: return launch_nt<1>(args, grid, st);
    case 2: return launch_nt<2>(args, grid, st);
    case 3: return launch_nt<3>(args, grid, st);
    default: return launch_nt<4>(args, grid, st);
  }
}

constexpr int64_t kScratchCounterBytes = 256 * 1024;
constexpr int64_t kScratchBytes = int64_t(NSD_NOALLOC_SCRATCH_BYTES);
static_assert(kScratchBytes > kScratchCounterBytes, "scratch layout");

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch_ptr[kMaxScratchDevices] = {};  // device address of `scratch`, per device

__global__ void zero_words_kernel(int32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// Device address of the current device's scratch.  On the first call on a
// device it is looked up (the array's host-side name is not a device
// address) and its counter region cleared by a fill kernel on `stream`.
int scratch_for_current_device(hipStream_t stream, char** out) {
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
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, stream,
                       static_cast<int32_t*>(ptr), kScratchCounterBytes / 4);
    const int rc = launch_status("paged_attention_noalloc: scratch clear");
    if (rc != NSD_OK) return rc;
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return NSD_OK;
}

}  // namespace

extern "C" int nsd_paged_attention(const void* q, void* o, float* lse, const void* k_cache,
                                   const void* v_cache, int64_t num_blocks, int num_layers,
                                   int layer, int num_q_heads, int num_kv_heads, int head_dim,
                                   int block_size, const int32_t* block_table, int64_t bt_stride,
                                   const int32_t* plan_host, const int32_t* plan_dev,
                                   void* workspace, int64_t workspace_bytes, float softmax_scale,
                                   int32_t* status, void* stream) {
  if (!plan_host) return fail(NSD_ERR_INVALID, "paged_attention: null plan");
  // workspace: partials, then the arrival counters
  const int64_t part_bytes = plan_partial_bytes(plan_host);
  char* ws = static_cast<char*>(workspace);
  const int64_t counters = workspace_bytes > part_bytes ? (workspace_bytes - part_bytes) / 4 : 0;
  return paged_attention_impl(q, o, lse, k_cache, v_cache, num_blocks, num_layers, layer,
                              num_q_heads, num_kv_heads, head_dim, block_size, block_table,
                              bt_stride, plan_host, plan_dev, ws, workspace_bytes,
                              ws ? reinterpret_cast<int32_t*>(ws + part_bytes) : nullptr,
                              counters, softmax_scale, status, stream);
}

extern "C" int nsd_paged_attention_noalloc(const void* q, void* o, float* lse,
                                           const void* k_cache, const void* v_cache,
                                           int64_t num_blocks, int num_layers, int layer,
                                           int num_q_heads, int num_kv_heads, int head_dim,
                                           int block_size, const int32_t* block_table,
                                           int64_t bt_stride, const int32_t* plan_host,
                                           const int32_t* plan_dev, float softmax_scale,
                                           int32_t* status, void* stream) {
  if (!plan_host) return fail(NSD_ERR_INVALID, "paged_attention_noalloc: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != kPlanVersionValue)
    return fail(NSD_ERR_INVALID, "paged_attention_noalloc: not a plan (bad magic/version)");
  const int64_t part_bytes = plan_partial_bytes(plan_host);
  const int64_t n_combine = plan_host[kPlanCombines];
  if (part_bytes > kScratchBytes - kScratchCounterBytes || n_combine * 4 > kScratchCounterBytes)
    return fail(NSD_ERR_WORKSPACE,
                "paged_attention_noalloc: the plan needs %lld partial bytes and %lld counters; "
                "the static scratch holds %lld and %lld (use nsd_paged_attention with a "
                "workspace)",
                (long long)part_bytes, (long long)n_combine,
                (long long)(kScratchBytes - kScratchCounterBytes),
                (long long)(kScratchCounterBytes / 4));
  hipStream_t st = as_stream(stream);
  char* base = nullptr;
  const int rc = scratch_for_current_device(st, &base);
  if (rc != NSD_OK) return rc;
  return paged_attention_impl(q, o, lse, k_cache, v_cache, num_blocks, num_layers, layer,
                              num_q_heads, num_kv_heads, head_dim, block_size, block_table,
                              bt_stride, plan_host, plan_dev, base + kScratchCounterBytes,
                              kScratchBytes - kScratchCounterBytes,
                              reinterpret_cast<int32_t*>(base), kScratchCounterBytes / 4,
                              softmax_scale, status, stream);
}
