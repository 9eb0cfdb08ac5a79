// Host-only part of the C ABI: error plumbing, version, and the attention
// work planner (no HIP calls, so it also runs on machines without a GPU).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <string>
#include <vector>

#include "nsd_common.h"

namespace nsd {

namespace {
thread_local std::string g_last_error;
// Cost model of the planner, in 16-token blocks of streaming: a piece costs
// its blocks plus a fixed kPieceCostBlocks for what it adds to the stream
// (the ring items that bring its query rows, the output or partial it
// writes).  A worker opens another piece only if at least kMinPieceBlocks of
// its budget remain for it.
constexpr int64_t kMinPieceBlocks = 4;
constexpr int64_t kPieceCostBlocks = 3;
// Workgroups launch in index order, two per CU: the first half of the grid
// takes one slot on every CU before the second half arrives, and a CU's
// earlier workgroup streams a few percent faster than its later one
// (per-workgroup timelines).  The first half's ranges are cut 1.5% longer,
// the second half's 1.5% shorter (per mille of the cost cap); the plan stays
// a function of the forward's rows alone.
constexpr int64_t kFirstHalfPerMille = 1015;
constexpr int64_t kSecondHalfPerMille = 985;
}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

}  // namespace nsd

using namespace nsd;

extern "C" int nsd_version(void) { return 100; }

extern "C" const char* nsd_last_error(void) { return g_last_error.c_str(); }

static int64_t round_up8(int64_t x) { return (x + 7) / 8 * 8; }

extern "C" int64_t nsd_attn_plan_bound(int64_t n_rows, int num_kv_heads, int n_workers) {
  if (n_rows < 0 || num_kv_heads <= 0 || n_workers <= 0) return -1;
  const int64_t segs = n_rows * num_kv_heads;
  const int64_t nw = round_up8(n_workers);
  // piece records: at most min(32, pieces) per worker, at a fixed stride
  const int64_t stride = std::min<int64_t>(kMaxWorkerPieces, nw + segs);
  return NSD_PLAN_HEADER_WORDS + 4 * n_rows + kWorkerWords * nw + kPieceWords * nw * stride +
         kPieceWords * segs;
}

extern "C" int nsd_attn_plan_build(const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                   int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                   int64_t bt_rows, int64_t bt_stride, int n_workers,
                                   int max_group_rows, int32_t* plan, int64_t plan_capacity,
                                   int64_t* plan_words, int64_t* workspace_bytes) {
  if (n_rows < 0) return fail(NSD_ERR_INVALID, "plan: n_rows=%lld < 0", (long long)n_rows);
  if (n_rows > 0 && (seq_ids == nullptr || seq_lens == nullptr))
    return fail(NSD_ERR_INVALID, "plan: null seq_ids/seq_lens");
  if (plan == nullptr || plan_words == nullptr || workspace_bytes == nullptr)
    return fail(NSD_ERR_INVALID, "plan: null output pointer");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(NSD_ERR_INVALID, "plan: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  if (head_dim != kHeadDim) return fail(NSD_ERR_UNSUPPORTED, "plan: head_dim=%d (only 128)", head_dim);
  if (block_size != kBlockTokens)
    return fail(NSD_ERR_UNSUPPORTED, "plan: block_size=%d (only 16)", block_size);
  if (n_workers <= 0) return fail(NSD_ERR_INVALID, "plan: n_workers=%d", n_workers);
  if (bt_rows <= 0 || bt_stride <= 0)
    return fail(NSD_ERR_INVALID, "plan: block table shape [%lld, %lld]", (long long)bt_rows,
                (long long)bt_stride);
  const int gqa = num_q_heads / num_kv_heads;
  if (gqa > kMaxGroupRows)
    return fail(NSD_ERR_UNSUPPORTED, "plan: GQA group %d > %d", gqa, kMaxGroupRows);
  if (max_group_rows < 0 || max_group_rows > kMaxGroupRows)
    return fail(NSD_ERR_INVALID, "plan: max_group_rows=%d outside [0, %d]", max_group_rows,
                kMaxGroupRows);
  const int64_t max_q = std::max(1, (max_group_rows == 0 ? kMaxGroupRows : max_group_rows) / gqa);
  const int64_t max_len = bt_stride * block_size;

  // 1. verify groups: runs of rows with one seq_id and seq_len rising by one.
  std::vector<int32_t> groups;  // {row_start, q_len, seq_id, ctx}
  int rows_max = 0;
  for (int64_t r = 0; r < n_rows;) {
    const int64_t sid = seq_ids[r], sl = seq_lens[r];
    if (sid < 0 || sid >= bt_rows)
      return fail(NSD_ERR_INVALID, "plan: row %lld seq_id=%lld outside [0, %lld)", (long long)r,
                  (long long)sid, (long long)bt_rows);
    if (sl < 1 || sl > max_len)
      return fail(NSD_ERR_INVALID, "plan: row %lld seq_len=%lld outside [1, %lld]", (long long)r,
                  (long long)sl, (long long)max_len);
    int64_t q = 1;
    while (r + q < n_rows && q < max_q && seq_ids[r + q] == sid && seq_lens[r + q] == sl + q) ++q;
    groups.insert(groups.end(), {(int32_t)r, (int32_t)q, (int32_t)sid, (int32_t)(sl - 1)});
    rows_max = std::max<int>(rows_max, (int)(q * gqa));
    r += q;
  }
  const int64_t n_groups = (int64_t)groups.size() / 4;
  const int64_t n_segs = n_groups * num_kv_heads;

  // 2. block counts per segment (segment = group * Hkv + kv head).
  std::vector<int64_t> seg_start(n_segs + 1, 0);
  for (int64_t s = 0; s < n_segs; ++s) {
    const int32_t* g = &groups[4 * (s / num_kv_heads)];
    const int64_t tokens = (int64_t)g[3] + g[1];
    seg_start[s + 1] = seg_start[s] + (tokens + kBlockTokens - 1) / kBlockTokens;
  }
  const int64_t total = seg_start[n_segs];

  // 3. contiguous block ranges per worker of near-equal cost (the cost model
  //    above, weighted by dispatch half).  The target cost is the smallest one that fits the stream into
  //    the workers; it also keeps every segment under kMaxSlotsPerSegment
  //    pieces, every worker under kMaxWorkerPieces pieces and
  //    kMaxWorkerBlocks blocks.
  int64_t max_seg = 0;
  for (int64_t s = 0; s < n_segs; ++s) max_seg = std::max(max_seg, seg_start[s + 1] - seg_start[s]);
  const int64_t cmin = kPieceCostBlocks + std::max<int64_t>(
      kMinPieceBlocks, (max_seg + kMaxSlotsPerSegment - 3) / (kMaxSlotsPerSegment - 2));
  // Greedy cut of the stream for a per-worker cost cap; returns the workers used
  // and, if `cuts` is given, each worker's piece boundaries.
  const int64_t first_half = std::max<int64_t>(1, n_workers) / 2;
  auto cut_stream = [&](int64_t cap, std::vector<int64_t>* cuts) {
    int64_t used = 0, pos = 0, seg_i = 0;
    while (pos < total) {
      int64_t budget = cap * (used < first_half ? kFirstHalfPerMille : kSecondHalfPerMille) / 1000;
      int64_t room = kMaxWorkerBlocks;
      int opened = 0;
      if (cuts) cuts->push_back(-1);  // worker marker
      while (pos < total && opened < kMaxWorkerPieces && room > 0) {
        while (seg_start[seg_i + 1] <= pos) ++seg_i;
        if (opened > 0 && budget < kPieceCostBlocks + kMinPieceBlocks) break;
        const int64_t take = std::min(room, std::max<int64_t>(
            1, std::min(budget - kPieceCostBlocks, seg_start[seg_i + 1] - pos)));
        if (cuts) cuts->insert(cuts->end(), {pos, pos + take});
        pos += take;
        room -= take;
        budget -= kPieceCostBlocks + take;
        ++opened;
        if (budget <= 0) break;
      }
      ++used;
    }
    return used;
  };
  const int64_t want = std::max<int64_t>(1, n_workers);
  int64_t lo = cmin, hi = std::max(cmin, total + n_segs * (kPieceCostBlocks + 1));
  if (total > 0 && cut_stream(lo, nullptr) > want) {
    while (lo + 1 < hi) {  // smallest cap that fits in `want` workers
      const int64_t mid = (lo + hi) / 2;
      if (cut_stream(mid, nullptr) <= want) hi = mid; else lo = mid;
    }
    lo = hi;
  }
  std::vector<int64_t> cuts;
  const int64_t active = total > 0 ? cut_stream(lo, &cuts) : 0;
  const int64_t grid = total > 0 ? round_up8(active) : 0;
  std::vector<int32_t> wstart(grid + 1, 0);
  std::vector<int32_t> pieces;  // kPieceWords per piece, workers' pieces in order
  int64_t seg = 0, w = -1;
  for (size_t c = 0; c < cuts.size();) {
    if (cuts[c] < 0) {  // next worker
      wstart[++w] = (int32_t)(pieces.size() / kPieceWords);
      ++c;
      continue;
    }
    const int64_t a = cuts[c], b = cuts[c + 1];
    c += 2;
    while (seg_start[seg + 1] <= a) ++seg;
    const int32_t* g = &groups[4 * (seg / num_kv_heads)];
    pieces.insert(pieces.end(), {(int32_t)(seg % num_kv_heads), (int32_t)(a - seg_start[seg]),
                                 (int32_t)(b - seg_start[seg]), -1, g[0], g[1], g[2], g[3],
                                 -1, 0, 0, 0});
  }
  for (int64_t v = w + 1; v < grid; ++v) wstart[v] = (int32_t)(pieces.size() / kPieceWords);
  wstart[grid] = (int32_t)(pieces.size() / kPieceWords);
  const int64_t n_pieces = (int64_t)pieces.size() / kPieceWords;

  // 4. partial slots for segments cut into several pieces (pieces of one
  //    segment are adjacent because workers walk the block stream in order).
  std::vector<int32_t> combines;  // kPieceWords per record
  int64_t n_slots = 0;
  auto same_seg = [&](int64_t i, int64_t j) {
    const int32_t* x = &pieces[kPieceWords * i];
    const int32_t* y = &pieces[kPieceWords * j];
    return x[kPieceHead] == y[kPieceHead] && x[kPieceRowStart] == y[kPieceRowStart];
  };
  for (int64_t i = 0; i < n_pieces;) {
    int64_t j = i + 1;
    while (j < n_pieces && same_seg(i, j)) ++j;
    if (j - i > kMaxSlotsPerSegment)
      return fail(NSD_ERR_INVALID, "plan: segment cut into %lld pieces", (long long)(j - i));
    if (j - i > 1) {
      const int32_t* x = &pieces[kPieceWords * i];
      const int32_t ci = (int32_t)(combines.size() / kPieceWords);
      combines.insert(combines.end(), {x[kPieceHead], (int32_t)n_slots, (int32_t)(j - i),
                                       x[kPieceRowStart], x[kPieceQLen], 0, 0, 0, 0, 0, 0, 0});
      for (int64_t k = i; k < j; ++k) {
        int32_t* y = &pieces[kPieceWords * k];
        y[kPieceSlot] = (int32_t)(n_slots + (k - i));
        y[kPieceComb] = ci;
        y[kPieceCombFirst] = (int32_t)n_slots;
        y[kPieceCombSlots] = (int32_t)(j - i);
      }
      n_slots += j - i;
    }
    i = j;
  }
  const int64_t n_combines = (int64_t)combines.size() / kPieceWords;

  // 5. records at a fixed stride per worker (zero records fill the gaps),
  //    each with the blocks of its worker's earlier pieces; the worker table
  //    holds each worker's record range and an inline copy of its first record.
  int64_t stride = 0, max_blocks = 0;
  for (int64_t v = 0; v < grid; ++v) stride = std::max<int64_t>(stride, wstart[v + 1] - wstart[v]);
  std::vector<int32_t> records(kPieceWords * grid * stride, 0);
  std::vector<int32_t> wtable(kWorkerWords * grid, 0);
  for (int64_t v = 0; v < grid; ++v) {
    int64_t blocks_run = 0;
    for (int64_t i = wstart[v]; i < wstart[v + 1]; ++i) {
      int32_t* r = &records[kPieceWords * (v * stride + (i - wstart[v]))];
      std::copy(&pieces[kPieceWords * i], &pieces[kPieceWords * (i + 1)], r);
      r[kPieceKvBase] = (int32_t)blocks_run;
      blocks_run += r[kPieceBlkEnd] - r[kPieceBlkBegin];
    }
    max_blocks = std::max(max_blocks, blocks_run);
    int32_t* row = &wtable[kWorkerWords * v];
    row[0] = (int32_t)(v * stride);
    row[1] = (int32_t)(v * stride + wstart[v + 1] - wstart[v]);
    if (wstart[v] < wstart[v + 1])
      std::copy(&records[kPieceWords * v * stride], &records[kPieceWords * (v * stride + 1)],
                row + kWorkerFirstPiece);
  }
  const int64_t n_records = grid * stride;

  const int64_t off_groups = NSD_PLAN_HEADER_WORDS;
  const int64_t off_wstart = off_groups + 4 * n_groups;
  const int64_t off_pieces = off_wstart + kWorkerWords * grid;
  const int64_t off_combines = off_pieces + kPieceWords * n_records;
  const int64_t words = off_combines + kPieceWords * n_combines;
  if (words > plan_capacity) {
    *plan_words = words;  // so the caller can retry with a large enough buffer
    return fail(NSD_ERR_WORKSPACE, "plan: needs %lld words, capacity %lld", (long long)words,
                (long long)plan_capacity);
  }
  if (words > INT32_MAX || n_slots > INT32_MAX / kMaxGroupRows)
    return fail(NSD_ERR_INVALID, "plan: too large (%lld words)", (long long)words);

  int32_t* h = plan;
  std::fill(h, h + NSD_PLAN_HEADER_WORDS, 0);
  h[kPlanMagic] = kPlanMagicValue;
  h[kPlanVersion] = kPlanVersionValue;
  h[kPlanRows] = (int32_t)n_rows;
  h[kPlanGroups] = (int32_t)n_groups;
  h[kPlanPieces] = (int32_t)n_records;
  h[kPlanWorkers] = (int32_t)grid;
  h[kPlanCombines] = (int32_t)n_combines;
  h[kPlanSlots] = (int32_t)n_slots;
  h[kPlanRowsMax] = rows_max;
  h[kPlanHq] = num_q_heads;
  h[kPlanHkv] = num_kv_heads;
  h[kPlanOffGroups] = (int32_t)off_groups;
  h[kPlanOffWorkers] = (int32_t)off_wstart;
  h[kPlanOffPieces] = (int32_t)off_pieces;
  h[kPlanOffCombines] = (int32_t)off_combines;
  h[kPlanWords] = (int32_t)words;
  h[kPlanPieceStride] = (int32_t)stride;
  h[kPlanBtRows] = (int32_t)std::min<int64_t>(bt_rows, INT32_MAX);
  h[kPlanBtStride] = (int32_t)std::min<int64_t>(bt_stride, INT32_MAX);
  h[kPlanMaxBlocks] = (int32_t)max_blocks;
  std::copy(groups.begin(), groups.end(), h + off_groups);
  std::copy(wtable.begin(), wtable.end(), h + off_wstart);
  std::copy(records.begin(), records.end(), h + off_pieces);
  std::copy(combines.begin(), combines.end(), h + off_combines);

  *plan_words = words;
  // partial O (fp16) and log-sum-exp (fp32) per slot and row
  const int64_t part_bytes = (n_slots * rows_max * (int64_t)(kHeadDim * 2 + 4) + 255) / 256 * 256;
  *workspace_bytes = n_combines > 0 ? part_bytes : 0;
  return NSD_OK;
}
