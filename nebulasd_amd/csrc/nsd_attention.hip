// Paged verify/decode attention for gfx950 (MI355X).
//
// Work unit.  A verify group is q_len consecutive rows of one sequence whose
// seq_lens rise by one (ctx+1 .. ctx+q_len); a decode row is a group with
// q_len = 1.  For one (group, kv head) -- a "segment" -- the GQA group x
// q_len query rows (up to 64) are packed as the N dimension of fp16 MFMAs,
// so each K/V tile of the segment is read from HBM exactly once:
//
//   S^T[token][row] = K[token][:] . Q[row][:]        (A = K, B = Q^T)
//   O^T[dim][row]  += V^T[dim][token] . P^T[token][row]  (A = V^T, B = P^T)
//
// using v_mfma_f32_16x16x32_f16.  Both products leave a lane holding one
// query row (lane & 15) of a 16-row tile, so the online softmax state of a
// row lives in one lane column and needs only two cross-row shuffles.
// K tiles load straight into the A-operand layout with 16-byte loads; V is
// loaded 16 bytes per lane and transposed 8x8 (halves) inside groups of 8
// lanes with three butterfly exchange stages.
//
// Work split.  The host planner cuts the stream of (segment, 32-token chunk)
// work into equal contiguous ranges, one per workgroup ("worker"); a
// workgroup's four waves take the chunks of a piece round-robin and merge
// their softmax states through LDS.  Segments cut across workers write fp32
// partials (normalised O, log2-sum-exp) that the combine kernel merges.
//
// Layouts (reference swiftLLM/swiftllm/worker/kernels/paged_attn.py):
//   k/v cache [N, L, Hkv, 16, 128] fp16, block (blk, layer, head) = 4 KB
//   contiguous at ((blk*L + layer)*Hkv + head)*16*128 (:49-50, :70-71).
#include "nsd_device.h"

namespace nsd {
namespace {

constexpr int D = kHeadDim;         // 128
constexpr int BS = kBlockTokens;     // 16
constexpr int CT = kChunkTokens;     // 32 tokens = two blocks per MFMA step
constexpr int NW = 4;                // waves per workgroup
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
  const int32_t* plan;
  float* part_o;           // [slots, rows_max, D]
  float* part_lse;         // [slots, rows_max]  (log2 domain)
  int32_t* status;
  int64_t num_blocks;
  int64_t blk_stride;      // elements per cache block: L*Hkv*16*128
  int num_layers, layer, hq, hkv, gqa, rows_max;
  float scale_log2;        // softmax_scale * log2(e)
};

__device__ inline uint32_t xchg(uint32_t v, int mask) {
  return (uint32_t)__shfl_xor((int)v, mask, kWave);
}

// 8x8 transpose of 16-bit elements inside each group of 8 lanes (lane bits
// 0..2): afterwards lane x, element y holds what lane y, element x held.
// Element y of a lane lives in dword y>>1, half y&1.  Each stage swaps one
// lane bit with the matching element bit.
__device__ inline void transpose8x8_b16(u32x4& d, int lane) {
  {  // lane bit 2 <-> element bit 2 (dwords {0,1} vs {2,3})
    const bool b = lane & 4;
    const uint32_t s0 = b ? d[0] : d[2], s1 = b ? d[1] : d[3];
    const uint32_t r0 = xchg(s0, 4), r1 = xchg(s1, 4);
    if (b) { d[0] = r0; d[1] = r1; } else { d[2] = r0; d[3] = r1; }
  }
  {  // lane bit 1 <-> element bit 1 (dwords {0,2} vs {1,3})
    const bool b = lane & 2;
    const uint32_t s0 = b ? d[0] : d[1], s1 = b ? d[2] : d[3];
    const uint32_t r0 = xchg(s0, 2), r1 = xchg(s1, 2);
    if (b) { d[0] = r0; d[2] = r1; } else { d[1] = r0; d[3] = r1; }
  }
  {  // lane bit 0 <-> element bit 0 (halves of each dword)
    const bool b = lane & 1;
    // lanes with bit 0 clear keep low halves and send high halves; the others the reverse.
    const uint32_t sel = b ? 0x05040100u : 0x07060302u;
    const uint32_t s0 = __builtin_amdgcn_perm(d[1], d[0], sel);
    const uint32_t s1 = __builtin_amdgcn_perm(d[3], d[2], sel);
    const uint32_t r0 = xchg(s0, 1), r1 = xchg(s1, 1);
    if (b) {
      d[0] = __builtin_amdgcn_perm(d[0], r0, 0x07060100u);
      d[1] = __builtin_amdgcn_perm(d[1], r0, 0x07060302u);
      d[2] = __builtin_amdgcn_perm(d[2], r1, 0x07060100u);
      d[3] = __builtin_amdgcn_perm(d[3], r1, 0x07060302u);
    } else {
      d[0] = __builtin_amdgcn_perm(r0, d[0], 0x05040100u);
      d[1] = __builtin_amdgcn_perm(r0, d[1], 0x07060100u);
      d[2] = __builtin_amdgcn_perm(r1, d[2], 0x05040100u);
      d[3] = __builtin_amdgcn_perm(r1, d[3], 0x07060100u);
    }
  }
}

__device__ inline f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

__device__ inline f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Worker id of this workgroup: hardware dispatches workgroup i to XCD i % 8,
// so consecutive workers (which share segments) land on the same XCD/L2.
__device__ inline int worker_id() {
  const int nb = gridDim.x;  // multiple of 8
  const int b = blockIdx.x;
  return (b & 7) * (nb >> 3) + (b >> 3);
}

template <int NT>
__global__ __launch_bounds__(NW * kWave) void paged_attn_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  float* s_acc = smem;                          // [NW-1][NT*16][RS]
  float* s_m = smem + (NW - 1) * NT * 16 * RS;  // [NW][NT*16]
  float* s_l = s_m + NW * NT * 16;              // [NW][NT*16]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;   // row within a 16-row tile (B/D column)
  const int lg = lane >> 4;   // k-group of the MFMA operands

  const int32_t* plan = a.plan;
  const int32_t* groups = plan + plan[kPlanOffGroups];
  const int32_t* wstart = plan + plan[kPlanOffWorkerStart];
  const int32_t* pieces = plan + plan[kPlanOffPieces];
  const int w = worker_id();
  const int p_begin = wstart[w], p_end = wstart[w + 1];

  for (int pc = p_begin; pc < p_end; ++pc) {
    const int seg = pieces[4 * pc + 0];
    const int c_begin = pieces[4 * pc + 1];
    const int c_end = pieces[4 * pc + 2];
    const int slot = pieces[4 * pc + 3];
    const int g = seg / a.hkv;
    const int h = seg - g * a.hkv;
    const int row_start = groups[4 * g + 0];
    const int q_len = groups[4 * g + 1];
    const int64_t seq_id = groups[4 * g + 2];
    const int ctx = groups[4 * g + 3];
    const int n_rows = q_len * a.gqa;
    const int total = ctx + q_len;            // tokens of the segment
    const int n_blk = (total + BS - 1) / BS;

    // Q^T as the B operand: lane (lg, lr) holds row 16j+lr, dims kk*32+lg*8..+8.
    f16x8 qb[NT][4];
    int sl[NT];  // seq_len of the lane's row (causal bound inside the group)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = 16 * j + lr;
      if (n < n_rows) {
        const int qi = n / a.gqa, gh = n - qi * a.gqa;
        const f16* qp = a.q + ((int64_t)(row_start + qi) * a.hq + h * a.gqa + gh) * D + lg * 8;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qb[j][kk] = *reinterpret_cast<const f16x8*>(qp + kk * 32);
        sl[j] = ctx + qi + 1;
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qb[j][kk] = f16x8{};
        sl[j] = total;
      }
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

    const int32_t* bt_row = a.bt + seq_id * a.bt_stride;
    const int64_t head_off = ((int64_t)a.layer * a.hkv + h) * BS * D;

    for (int c = c_begin + wave; c < c_end; c += NW) {
      // Block ids of the chunk's two 16-token blocks (the second may not exist).
      int64_t blk[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int bi = 2 * c + tt;
        int64_t id = -1;
        if (bi < n_blk) {
          id = bt_row[bi];
          if (id < 0 || id >= a.num_blocks) {
            if (lane == 0) flag_status(a.status, NSD_STATUS_BAD_BLOCK);
            id = -1;
          }
        }
        blk[tt] = id;
      }

      // K: A operand, lane (lg, lr) = token lr of block tt, dims kk*32+lg*8..+8.
      f16x8 ka[2][4];
      // V: lane (lg, hh = (lane>>3)&1, x = lane&7) loads token T(lg, x) =
      // (x>>2)*16 + 4*lg + (x&3), dims 16*mt + 8*hh .. +8; after the 8x8
      // transpose the lane holds dim 16*mt + lr for tokens T(lg, 0..7).
      u32x4 vr[8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (blk[tt] >= 0) {
          const f16* kp = a.k_cache + blk[tt] * a.blk_stride + head_off + lr * D + lg * 8;
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) ka[tt][kk] = *reinterpret_cast<const f16x8*>(kp + kk * 32);
        } else {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) ka[tt][kk] = f16x8{};
        }
      }
      {
        const int x = lane & 7;
        const int tt = x >> 2;
        const int tok = 4 * lg + (x & 3);
        const int64_t id = blk[tt];
        if (id >= 0) {
          const f16* vp = a.v_cache + id * a.blk_stride + head_off + tok * D + 8 * ((lane >> 3) & 1);
#pragma unroll
          for (int mt = 0; mt < 8; ++mt) vr[mt] = *reinterpret_cast<const u32x4*>(vp + 16 * mt);
        } else {
#pragma unroll
          for (int mt = 0; mt < 8; ++mt) vr[mt] = u32x4{0u, 0u, 0u, 0u};
        }
      }

      // S^T tiles: lane (lg, lr) gets scores of row 16j+lr for tokens
      // 32c + 16tt + 4lg + i, i = 0..3.
      f32x4 s[2][NT];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) t = mfma16x16x32(ka[tt][kk], qb[j][kk], t);
          s[tt][j] = t;
        }

      // Online softmax in the exp2 domain, one row per lane column.
      const int t0 = c * CT + 4 * lg;
      f16x8 pb[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = t0 + 16 * tt + i;
            const float v = t < sl[j] ? s[tt][j][i] * a.scale_log2 : -INFINITY;
            s[tt][j][i] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m[j], mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m[j] - m_use);
        float psum = 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = exp2f(s[tt][j][i] - m_use);
            psum += p;
            pb[j][tt * 4 + i] = (f16)p;
          }
        l[j] = l[j] * alpha + psum;
        m[j] = m_new;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) acc[j][mt] *= alpha;
      }

      // O^T += V^T P^T for the 8 dim tiles.
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        transpose8x8_b16(vr[mt], lane);
        const f16x8 va = as_f16x8(vr[mt]);
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j][mt] = mfma16x16x32(va, pb[j], acc[j][mt]);
      }
    }

    // Row sums across the four k-groups.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      l[j] += __shfl_xor(l[j], 16, kWave);
      l[j] += __shfl_xor(l[j], 32, kWave);
    }

    // Merge the waves' states through LDS (wave 0 finishes the piece).
    if (lg == 0) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        s_m[wave * NT * 16 + 16 * j + lr] = m[j];
        s_l[wave * NT * 16 + 16 * j + lr] = l[j];
      }
    }
    if (wave > 0) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
          *reinterpret_cast<f32x4*>(s_acc + ((wave - 1) * NT * 16 + 16 * j + lr) * RS + 16 * mt +
                                    4 * lg) = acc[j][mt];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int n = 16 * j + lr;
        float mw[NW], M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
          mw[ww] = s_m[ww * NT * 16 + n];
          M = fmaxf(M, mw[ww]);
        }
        const float M_use = M == -INFINITY ? 0.f : M;
        float fw[NW], L = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
          fw[ww] = exp2f(mw[ww] - M_use);
          L += fw[ww] * s_l[ww * NT * 16 + n];
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const bool live = n < n_rows;
        const int qi = n / a.gqa, gh = n - qi * a.gqa;
        const int64_t orow = (int64_t)(row_start + qi) * a.hq + h * a.gqa + gh;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
          f32x4 v = acc[j][mt] * fw[0];
#pragma unroll
          for (int ww = 1; ww < NW; ++ww)
            v += *reinterpret_cast<const f32x4*>(s_acc + ((ww - 1) * NT * 16 + n) * RS + 16 * mt +
                                                 4 * lg) * fw[ww];
          v *= inv;
          if (live) {
            if (slot < 0) {
              f16x4 hv = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
              *reinterpret_cast<f16x4*>(a.o + orow * D + 16 * mt + 4 * lg) = hv;
            } else {
              *reinterpret_cast<f32x4*>(a.part_o + ((int64_t)slot * a.rows_max + n) * D + 16 * mt +
                                        4 * lg) = v;
            }
          }
        }
        if (live && lg == 0) {
          const float lse2 = L > 0.f ? M + __log2f(L) : -INFINITY;
          if (slot < 0) {
            if (a.lse != nullptr) a.lse[orow] = lse2 * kLn2;
          } else {
            a.part_lse[(int64_t)slot * a.rows_max + n] = lse2;
          }
        }
      }
    }
    __syncthreads();
  }
}

// Merge the partials of segments cut across workers: one workgroup per
// segment, one thread per (row, dim).  Mirrors phase 2 of the reference
// (paged_attn.py:128-149) in the same exp2 domain.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int32_t* plan = a.plan;
  const int32_t* groups = plan + plan[kPlanOffGroups];
  const int32_t* comb = plan + plan[kPlanOffCombines] + 4 * blockIdx.x;
  const int seg = comb[0], first = comb[1], n_slots = comb[2];
  const int g = seg / a.hkv, h = seg - g * a.hkv;
  const int row_start = groups[4 * g + 0];
  const int n_rows = groups[4 * g + 1] * a.gqa;
  for (int idx = threadIdx.x; idx < n_rows * D; idx += blockDim.x) {
    const int n = idx / D, d = idx - n * D;
    float M = -INFINITY;
    for (int s = 0; s < n_slots; ++s) M = fmaxf(M, a.part_lse[(int64_t)(first + s) * a.rows_max + n]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float wsum = 0.f, acc = 0.f;
    for (int s = 0; s < n_slots; ++s) {
      const int64_t ps = (int64_t)(first + s) * a.rows_max + n;
      const float wgt = exp2f(a.part_lse[ps] - M_use);
      wsum += wgt;
      acc += wgt * a.part_o[ps * D + d];
    }
    const int qi = n / a.gqa, gh = n - qi * a.gqa;
    const int64_t orow = (int64_t)(row_start + qi) * a.hq + h * a.gqa + gh;
    a.o[orow * D + d] = (f16)(acc / wsum);
    if (d == 0 && a.lse != nullptr) a.lse[orow] = (M + __log2f(wsum)) * kLn2;
  }
}

template <int NT>
constexpr size_t lds_bytes() {
  return sizeof(float) * ((NW - 1) * NT * 16 * RS + 2 * NW * NT * 16);
}

template <int NT>
int launch_nt(const AttnArgs& args, int grid, int n_combine, hipStream_t stream) {
  static bool attr_set = false;  // per-process: raise the dynamic-LDS limit once
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_attn_kernel<NT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds_bytes<NT>());
    if (e != hipSuccess)
      return fail(NSD_ERR_HIP, "paged_attention: LDS attribute: %s", hipGetErrorString(e));
    attr_set = true;
  }
  if (grid > 0) {
    hipLaunchKernelGGL(paged_attn_kernel<NT>, dim3(grid), dim3(NW * kWave), lds_bytes<NT>(),
                       stream, args);
    int rc = launch_status("paged_attention");
    if (rc) return rc;
  }
  if (n_combine > 0) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_combine), dim3(256), 0, stream, args);
    return launch_status("paged_attention combine");
  }
  return NSD_OK;
}

template <int NT>
int occupancy_nt(int* blocks) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(
             blocks, reinterpret_cast<const void*>(&paged_attn_kernel<NT>), NW * kWave,
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

extern "C" int nsd_paged_attention(const void* q, void* o, float* lse, const void* k_cache,
                                   const void* v_cache, int64_t num_blocks, int num_layers,
                                   int layer, int num_q_heads, int num_kv_heads, int head_dim,
                                   int block_size, const int32_t* block_table, int64_t bt_stride,
                                   const int32_t* plan_host, const int32_t* plan_dev,
                                   void* workspace, int64_t workspace_bytes, float softmax_scale,
                                   int32_t* status, void* stream) {
  if (head_dim != D) return fail(NSD_ERR_UNSUPPORTED, "paged_attention: head_dim=%d (only 128)", head_dim);
  if (block_size != BS)
    return fail(NSD_ERR_UNSUPPORTED, "paged_attention: block_size=%d (only 16)", block_size);
  if (!plan_host || !plan_dev) return fail(NSD_ERR_INVALID, "paged_attention: null plan");
  if (plan_host[kPlanMagic] != kPlanMagicValue || plan_host[kPlanVersion] != 1)
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
  if (plan_host[kPlanRows] == 0 || grid == 0) return NSD_OK;
  if (!q || !o || !k_cache || !v_cache || !block_table)
    return fail(NSD_ERR_INVALID, "paged_attention: null pointer");
  if (!aligned16(q) || !aligned16(o) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(NSD_ERR_INVALID, "paged_attention: q/o/caches must be 16-byte aligned");
  if (rows_max < 1 || rows_max > kMaxGroupRows || grid % 8 != 0)
    return fail(NSD_ERR_INVALID, "paged_attention: corrupt plan header");
  const int64_t n_slots = plan_host[kPlanSlots];
  const int64_t need = n_slots * rows_max * (int64_t)(D + 1) * 4;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
    return fail(NSD_ERR_WORKSPACE, "paged_attention: workspace %lld bytes < %lld needed",
                (long long)workspace_bytes, (long long)need);

  AttnArgs args;
  args.q = static_cast<const f16*>(q);
  args.o = static_cast<f16*>(o);
  args.lse = lse;
  args.k_cache = static_cast<const f16*>(k_cache);
  args.v_cache = static_cast<const f16*>(v_cache);
  args.bt = block_table;
  args.bt_stride = bt_stride;
  args.plan = plan_dev;
  args.part_o = static_cast<float*>(workspace);
  args.part_lse = static_cast<float*>(workspace) + n_slots * rows_max * D;
  args.status = status;
  args.num_blocks = num_blocks;
  args.blk_stride = (int64_t)num_layers * num_kv_heads * BS * D;
  args.num_layers = num_layers;
  args.layer = layer;
  args.hq = num_q_heads;
  args.hkv = num_kv_heads;
  args.gqa = num_q_heads / num_kv_heads;
  args.rows_max = rows_max;
  args.scale_log2 = softmax_scale * 1.4426950408889634f;

  hipStream_t st = as_stream(stream);
  const int nt = (rows_max + 15) / 16;
  switch (nt) {
    case 1: return launch_nt<1>(args, grid, n_combine, st);
    case 2: return launch_nt<2>(args, grid, n_combine, st);
    case 3: return launch_nt<3>(args, grid, n_combine, st);
    default: return launch_nt<4>(args, grid, n_combine, st);
  }
}
