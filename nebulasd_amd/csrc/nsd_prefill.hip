// Prefill (prompt) attention for gfx950 (MI355X).
//
// Replaces the reference's prefill attention: flash_attn_varlen_func
// (swiftLLM/swiftllm/worker/layers/transformer_layer.py:7-32, called at
// :151-164 with cu_seqlens_q = cu_seqlens_k = prefill_seq_start_locs_with_end
// and causal=True), which runs one scaled_dot_product_attention per prompt
// after a host copy of cu_seqlens, and the Triton prefill_attention
// (swiftLLM/swiftllm/worker/kernels/prefill_attn.py:10-140).  Position i of a
// prompt attends the prompt's tokens 0..i; q-head h reads kv head
// h / (Hq/Hkv) (the repeat_interleave of transformer_layer.py:20-23).
//
// Work unit: (prompt, kv head, block of P = rows/gqa positions).  The
// workgroup's query rows (128: four waves of 32) are the gqa q-heads of its
// P positions, packed as row n = position_offset * gqa + head_in_group, so
// every K/V tile staged in LDS serves all the q-heads that read it.  Three
// workgroups share a compute unit, so one's loads and barriers overlap the
// others' MFMAs.
//
//   S^T[token][row] = K[token][:] . Q[row][:]            A = K (LDS), B = Q^T (registers)
//   O^T[dim][row]  += V^T[dim][token] . P^T[token][row]  A = V^T (LDS), B = P^T (registers)
//
// Both products use v_mfma_f32_16x16x32_f16.  The PV product takes the 32
// tokens of a tile in one MFMA: its B operand is the P of the tile's two
// 16-token score tiles (lane group g holds tokens 4g..4g+3 of each), and its
// A operand reads V^T for the same tokens (4g..4g+3 and 16+4g..16+4g+3) with
// two transposing LDS reads, so the score registers feed the PV product as
// they are.  Online softmax in the exp2 domain, fp32 state per row.
//
// K/V tiles of 32 tokens are double-buffered in LDS: each tile's global
// loads are issued before the previous tile's MFMAs and written to the other
// buffer after them, one barrier per tile.  A row's running max is raised
// lazily (only past a margin, after a wave-wide vote), so most tiles need no
// cross-lane reduction and no rescaling of the accumulators.  Workgroups are issued from the
// last position block down, so the longest ones (the most tiles under the
// causal mask) start first; the q-blocks of one (prompt, kv head) are
// n_seqs*Hkv workgroups apart, which keeps them on one XCD when that count
// is a multiple of 8.
#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int PD = kHeadDim;        // 128
constexpr int PROWB = PD * 2 + 32;  // LDS bytes per staged token row (32 B bank shift: no conflicts)
constexpr float kLn2f = 0.69314718055994531f;
// A row's running max is raised only when a tile's scores exceed it by more
// than this (log2 units): the softmax terms then stay below 2^8, exact after
// the final normalisation, and most tiles skip rescaling the accumulators.
constexpr float kLazyMax = 8.f;

// Kernel shape: NTW 16-row tiles per wave, NW waves per workgroup, KT tokens
// per K/V tile, PF tiles of global loads in flight, LAZY running-max raise.
template <int NTW_, int NW_, int KT_, int PF_, bool LAZY_, int WPE_ = 1>
struct PrefillCfg {
  static constexpr int NTW = NTW_, NW = NW_, KT = KT_, PF = PF_;
  static constexpr bool LAZY = LAZY_;
  static constexpr int WPE = WPE_;  // minimum waves per SIMD the register budget must allow
  static constexpr int rows = NW * 16 * NTW;  // query rows (position x q-head) per workgroup
  static constexpr int threads = NW * kWave;
  static constexpr int loads = 2 * KT * (PD / 8) / threads;  // 16-byte K/V loads per thread per tile
  static constexpr int lds_bytes = 2 * 2 * KT * PROWB;       // [buffer][K, V][token][padded row]
  static_assert(loads * threads == 2 * KT * (PD / 8), "tile loads split evenly");
  static_assert((KT * (PD / 8)) % threads == 0, "each load is all-K or all-V");
  static_assert(KT % 32 == 0 && (PF == 1 || PF == 2), "tile shape");
};

// The shape every launch uses: 32 rows per wave, four waves, 32-token
// tiles, three workgroups per compute unit (168 VGPRs).  Measured against
// 8-wave workgroups (one per CU), 64-token tiles, a second tile in flight,
// 16- and 64-row waves and the software-pipelined loop, all slower; shapes
// that spill registers were slowest, and so was a software-pipelined loop
// (K one tile ahead of V, the next tile's score MFMAs issued beside the
// softmax).
using PrefillShape = PrefillCfg<2, 4, 32, 1, true, 3>;

struct PrefillArgs {
  const f16* q;               // [T, Hq, D]
  const f16* k;               // [T, Hkv, D]
  const f16* v;               // [T, Hkv, D]
  f16* o;                     // [T, Hq, D]
  float* lse;                 // [T, Hq] natural log, optional
  const int32_t* cu_seqlens;  // [n_seqs + 1]
  const int32_t* seq_order;   // [n_seqs] prompts longest first, or null (natural order)
  int32_t* status;
  int64_t total_tokens;
  int n_seqs, hq, hkv, gqa;
  int positions;              // P = rows per workgroup / gqa
  int max_seqlen;
  int q_blocks;               // ceil(max_seqlen / P)
  float scale_log2;           // softmax_scale * log2(e)
};

template <class C>
__global__ void __launch_bounds__(C::threads) __attribute__((amdgpu_waves_per_eu(C::WPE)))
prefill_attn_kernel(PrefillArgs a) {
  constexpr int NTW = C::NTW, KT = C::KT, NTHR = C::threads, LPT = C::loads;
  constexpr int KH = KT / 16;  // 16-token score tiles per K/V tile
  extern __shared__ __align__(16) char smem_raw[];
  lds_char* s_kv = (lds_char*)smem_raw;  // buffer b, K (0) or V (1): s_kv + (2b + kv) * KT * PROWB

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;  // row of a 16-row tile (B/C column)
  const int lg = lane >> 4;  // k-group of the MFMA operands

  // Work item, last position block first.
  const int per_qb = a.n_seqs * a.hkv;
  const int qb = a.q_blocks - 1 - (int)blockIdx.x / per_qb;
  const int item = (int)blockIdx.x % per_qb;
  const int pos = item / a.hkv, kvh = item - pos * a.hkv;
  // With prompts longest first, a block level's non-empty items are
  // consecutive (cyclically), so in-order dispatch spreads them over the
  // shader engines; rotating each level by its index moves the longest
  // prompts to another engine at every level instead of stacking one
  // engine's slots with them.
  const int rank = (pos + qb) % a.n_seqs;
  const int seq = a.seq_order != nullptr ? a.seq_order[rank] : rank;
  if (seq < 0 || seq >= a.n_seqs) {
    if (threadIdx.x == 0) flag_status(a.status, NSD_STATUS_BAD_SEQ);
    return;
  }
  const int start = a.cu_seqlens[seq];
  const int end = a.cu_seqlens[seq + 1];
  const int P = a.positions;
  const int p0 = qb * P;
  if (start < 0 || end < start || start > a.total_tokens) {
    if (qb == 0 && kvh == 0 && threadIdx.x == 0) flag_status(a.status, NSD_STATUS_BAD_SEQ);
    return;
  }
  // An end past the tokens is cut there, as the reference's slices of
  // q[:num_prefill_tokens] cut the last prompt (its cu_seqlens ends at the
  // forward's token count, model.py:412-415).
  const int len = (int)((int64_t)end < a.total_tokens ? end : a.total_tokens) - start;
  if (qb == 0 && kvh == 0 && threadIdx.x == 0 && len > a.max_seqlen)
    flag_status(a.status, NSD_STATUS_BAD_SEQ);  // positions past the grid's blocks are not computed
  if (p0 >= len) return;

  const int p_end = min(p0 + P, len);      // one past the block's last valid position
  const int n_tiles = (p_end + KT - 1) / KT;
  const int row0 = wave * 16 * NTW;        // this wave's first row in the workgroup
  const int wave_first = p0 + row0 / a.gqa;
  const int wave_last = min(p0 + (row0 + 16 * NTW - 1) / a.gqa, len - 1);
  const bool wave_live = wave_first < len;

  // Q^T fragments (B operand): row n = row0 + 16j + lr, dims 32kk + 8lg .. +7.
  f16x8 qf[NTW][4];
  int pos_row[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int n = row0 + 16 * j + lr;
    const int pq = n / a.gqa;
    pos_row[j] = p0 + pq;
    const int pc = min(pos_row[j], len - 1);  // rows past the prompt read its last row, unused
    const f16* qp = a.q + ((int64_t)(start + pc) * a.hq + kvh * a.gqa + (n - pq * a.gqa)) * PD + 8 * lg;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[j][kk] = *reinterpret_cast<const f16x8*>(qp + 32 * kk);
  }
  // Keep the Q loads ahead of the first tile's: the wait that stores tile 0
  // then covers them, and the tile loop never waits on Q (a wait inside the
  // loop would also drain the next tile's loads every iteration).
  asm volatile("" ::: "memory");

  // K/V tile staging through registers: thread chunk c -> (K or V, token,
  // 16-byte part); tile u is loaded into stage[u % PF].
  u32x4 stage[C::PF][LPT];
  auto load_tile = [&](auto sidx, int t) {
    constexpr int S = decltype(sidx)::value;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = threadIdx.x + i * NTHR;
      const int kv = (i * NTHR) / (KT * (PD / 8));
      const int tok = (c / (PD / 8)) % KT, part = c % (PD / 8);
      const int tk = min(t * KT + tok, len - 1);  // past the prompt: masked, reads its last row
      const f16* base = kv ? a.v : a.k;
      stage[S][i] = *reinterpret_cast<const u32x4*>(base + ((int64_t)(start + tk) * a.hkv + kvh) * PD +
                                                    part * 8);
    }
  };
  auto store_tile = [&](auto sidx, int buf) {
    constexpr int S = decltype(sidx)::value;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = threadIdx.x + i * NTHR;
      const int kv = (i * NTHR) / (KT * (PD / 8));
      const int tok = (c / (PD / 8)) % KT, part = c % (PD / 8);
      *(lds_u32x4*)(s_kv + (2 * buf + kv) * KT * PROWB + tok * PROWB + part * 16) = stage[S][i];
    }
  };

  float m[NTW], l[NTW];  // running max (scaled log2 domain); this lane's share of the sum
  f32x4 acc[NTW][8];     // O^T: dims 16dt + 4lg .. +3 of row 16j + lr
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;

#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float c = a.scale_log2;

  // One K/V tile from LDS buffer `buf`: S^T, mask, online softmax, PV.
  auto compute = [&](int t, int buf) {
    const int t0 = t * KT;
    if (!(wave_live && t0 <= wave_last)) return;  // no row of this wave sees a token of the tile
    const lds_char* kb = s_kv + (2 * buf) * KT * PROWB;
    const lds_char* vb = kb + KT * PROWB;
    // (k-steps outermost: KH * NTW independent accumulators between reuses)
    f32x4 s[KH][NTW];
#pragma unroll
    for (int h = 0; h < KH; ++h)
#pragma unroll
      for (int j = 0; j < NTW; ++j) s[h][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int h = 0; h < KH; ++h) {
        const f16x8 kf = *(const lds_f16x8*)(kb + (16 * h + lr) * PROWB + 64 * kk + 16 * lg);
#pragma unroll
        for (int j = 0; j < NTW; ++j) s[h][j] = mfma_k32(kf, qf[j][kk], s[h][j]);
      }
    }
    // Causal mask where the tile reaches the block's positions (it also
    // hides tokens past the prompt: they lie past every valid row).
    if (t0 + KT - 1 >= p0) {
#pragma unroll
      for (int h = 0; h < KH; ++h)
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t0 + 16 * h + 4 * lg + i > pos_row[j]) s[h][j][i] = -INFINITY;
    }
    // Online softmax in the exp2 domain.  Each lane checks its own scores
    // against the running max; only when some lane of the wave exceeds it by
    // more than kLazyMax are the rows' maxima reduced across the four lane
    // groups and raised (the common case needs no cross-lane traffic).
    float mxs[NTW];
    bool raise = false;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int h = 0; h < KH; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[h][j][i]);
      mxs[j] = mx * c;
      raise |= C::LAZY ? mxs[j] > m[j] + kLazyMax : true;
    }
    if (!C::LAZY || __any(raise)) {
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        mxs[j] = fmaxf(mxs[j], __shfl_xor(mxs[j], 16, kWave));
        mxs[j] = fmaxf(mxs[j], __shfl_xor(mxs[j], 32, kWave));
        const float m_new = fmaxf(m[j], mxs[j]);
        const float alpha = __builtin_amdgcn_exp2f(m[j] - (m_new == -INFINITY ? 0.f : m_new));
        l[j] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[j][dt] *= alpha;
        m[j] = m_new;
      }
    }
    // P^T in the PV operand layout: k-step ks holds tokens 32ks + 4lg + i and
    // 32ks + 16 + 4lg + i.
    f16x8 pf[KT / 32][NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const float m_use = m[j] == -INFINITY ? 0.f : m[j];
      float ps = 0.f;
#pragma unroll
      for (int h = 0; h < KH; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[h][j][i], c, -m_use));
          ps += p;
          pf[h / 2][j][4 * (h % 2) + i] = (f16)p;
        }
      l[j] += ps;
    }
    // O^T += V^T . P^T, 16 dims and 32 tokens per MFMA.
#pragma unroll
    for (int ks = 0; ks < KT / 32; ++ks) {
      const lds_char* vsrc = vb + (32 * ks + 4 * lg + (lr >> 2)) * PROWB + 8 * (lr & 3);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f16x4 lo = ds_read_tr16(vsrc + 32 * dt);
        const f16x4 hi = ds_read_tr16(vsrc + 16 * PROWB + 32 * dt);
        const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[j][dt] = mfma_k32(vf, pf[ks][j], acc[j][dt]);
      }
    }
  };

  // Pipeline: tile t is computed from LDS buffer t % 2 while the loads of
  // tile t + PF are in flight; tile t + 1 (loaded PF - 1 tiles earlier) goes
  // to the other buffer after the compute, then one barrier.
  using std::integral_constant;
  load_tile(integral_constant<int, 0>{}, 0);
  if constexpr (C::PF == 2) {
    if (n_tiles > 1) load_tile(integral_constant<int, 1>{}, 1);
  }
  store_tile(integral_constant<int, 0>{}, 0);
  __syncthreads();
  auto iteration = [&](auto par, int t) {
    constexpr int S = decltype(par)::value;  // t % 2
    if constexpr (C::PF == 1) {
      if (t + 1 < n_tiles) load_tile(integral_constant<int, 0>{}, t + 1);
      compute(t, S);
      if (t + 1 < n_tiles) store_tile(integral_constant<int, 0>{}, S ^ 1);
    } else {
      if (t + 2 < n_tiles) load_tile(integral_constant<int, S>{}, t + 2);
      compute(t, S);
      if (t + 1 < n_tiles) store_tile(integral_constant<int, S ^ 1>{}, S ^ 1);
    }
    __syncthreads();
  };
  for (int t = 0; t < n_tiles; t += 2) {
    iteration(integral_constant<int, 0>{}, t);
    if (t + 1 < n_tiles) iteration(integral_constant<int, 1>{}, t + 1);
  }

  // Normalise and write the valid rows.
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    float lt = l[j];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    const int n = row0 + 16 * j + lr;
    const int pq = n / a.gqa;
    const int pos = p0 + pq;
    if (pos >= len) continue;
    const int head = kvh * a.gqa + (n - pq * a.gqa);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    f16* op = a.o + ((int64_t)(start + pos) * a.hq + head) * PD + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 ov = acc[j][dt] * inv;
      const f16x4 hv = {(f16)ov[0], (f16)ov[1], (f16)ov[2], (f16)ov[3]};
      *reinterpret_cast<f16x4*>(op + 16 * dt) = hv;
    }
    if (lg == 0 && a.lse != nullptr)
      a.lse[(int64_t)(start + pos) * a.hq + head] = lt > 0.f ? (m[j] + __log2f(lt)) * kLn2f : -INFINITY;
  }
}

template <class C>
int launch_prefill(PrefillArgs args, hipStream_t stream) {
  // allow the dynamic LDS once per process: a function-local static is
  // initialised exactly once even when several threads launch at once, and
  // a failure stays reported on every later call
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_attn_kernel<C>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, C::lds_bytes);
  if (attr != hipSuccess) return fail(NSD_ERR_HIP, "prefill_attention: LDS attribute: %s", hipGetErrorString(attr));
  args.positions = C::rows / args.gqa;
  args.q_blocks = (args.max_seqlen + args.positions - 1) / args.positions;
  const int64_t grid = (int64_t)args.q_blocks * args.n_seqs * args.hkv;
  if (grid > INT32_MAX) return fail(NSD_ERR_UNSUPPORTED, "prefill_attention: grid of %lld workgroups", (long long)grid);
  hipLaunchKernelGGL(prefill_attn_kernel<C>, dim3((unsigned)grid), dim3(C::threads), C::lds_bytes, stream, args);
  return launch_status("prefill_attention");
}

}  // namespace
}  // namespace nsd

using namespace nsd;

extern "C" int nsd_prefill_attention(const void* q, const void* k, const void* v, void* o, float* lse,
                                     const int32_t* cu_seqlens, const int32_t* seq_order,
                                     int n_seqs, int max_seqlen,
                                     int64_t total_tokens, int num_q_heads, int num_kv_heads,
                                     int head_dim, float softmax_scale, int32_t* status, void* stream) {
  if (head_dim != PD) return fail(NSD_ERR_UNSUPPORTED, "prefill_attention: head_dim=%d (only 128)", head_dim);
  if (num_kv_heads < 1 || num_q_heads < num_kv_heads || num_q_heads % num_kv_heads != 0)
    return fail(NSD_ERR_INVALID, "prefill_attention: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  const int gqa = num_q_heads / num_kv_heads;
  if (PrefillShape::rows % gqa != 0)
    return fail(NSD_ERR_UNSUPPORTED, "prefill_attention: q-heads per kv head %d must divide %d", gqa,
                PrefillShape::rows);
  if (n_seqs < 0 || max_seqlen < 0 || total_tokens < 0)
    return fail(NSD_ERR_INVALID, "prefill_attention: negative size");
  if (n_seqs == 0 || max_seqlen == 0 || total_tokens == 0) return NSD_OK;
  if (!q || !k || !v || !o || !cu_seqlens) return fail(NSD_ERR_INVALID, "prefill_attention: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(NSD_ERR_INVALID, "prefill_attention: q/k/v/o must be 16-byte aligned");
  if (!(softmax_scale > 0.f)) return fail(NSD_ERR_INVALID, "prefill_attention: softmax_scale must be > 0");
  PrefillArgs args;
  args.q = static_cast<const f16*>(q);
  args.k = static_cast<const f16*>(k);
  args.v = static_cast<const f16*>(v);
  args.o = static_cast<f16*>(o);
  args.lse = lse;
  args.cu_seqlens = cu_seqlens;
  args.seq_order = seq_order;
  args.status = status;
  args.total_tokens = total_tokens;
  args.n_seqs = n_seqs;
  args.hq = num_q_heads;
  args.hkv = num_kv_heads;
  args.gqa = gqa;
  args.max_seqlen = max_seqlen;
  args.scale_log2 = softmax_scale * 1.4426950408889634f;
  return launch_prefill<PrefillShape>(args, as_stream(stream));
}
