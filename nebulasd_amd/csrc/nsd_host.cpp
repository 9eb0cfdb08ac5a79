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

bool plan_keeps_sequences_whole(const int32_t* plan_host) {
  const int n_groups = plan_host[kPlanGroups];
  const int32_t* grp = plan_host + plan_host[kPlanOffGroups];  // [n_groups][4] {row_start, q_len, seq_id, ctx}
  std::vector<int32_t> sids(n_groups);
  for (int g = 0; g < n_groups; ++g) sids[g] = grp[4 * g + 2];
  std::sort(sids.begin(), sids.end());
  return std::adjacent_find(sids.begin(), sids.end()) == sids.end();
}

}  // namespace nsd

using namespace nsd;

extern "C" int nsd_version(void) { return 100; }

extern "C" const char* nsd_last_error(void) { return g_last_error.c_str(); }

static int64_t round_up8(int64_t x) { return (x + 7) / 8 * 8; }

extern "C" int64_t nsd_attn_plan_bound(int64_t n_rows, int num_kv_heads, int n_workers) {
  if (n_rows < 0 || num_kv_heads <= 0 || n_workers <= 0) return -1;
  const int64_t segs = n_rows * num_kv_heads;
  // pieces: n_workers, or one per segment where there are more segments,
  // plus the empty records that even out the XCD lists; a plan that needs
  // more (segments longer than 256 blocks each) reports its size and the
  // caller retries
  const int64_t pieces = round_up8(std::max<int64_t>(n_workers, segs)) + kXcds * kMaxSlotsPerSegment;
  return NSD_PLAN_HEADER_WORDS + 4 * n_rows + kPieceWords * pieces + kPieceWords * segs;
}

extern "C" int nsd_attn_plan_build(const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                   int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                   int64_t bt_rows, int64_t bt_stride, int n_workers,
                                   int max_group_rows, int32_t* plan, int64_t plan_capacity,
                                   int64_t* plan_words, int64_t* workspace_bytes) {
  return nsd_attn_plan_build_claimed(seq_ids, seq_lens, n_rows, num_q_heads, num_kv_heads, head_dim, block_size,
                                     bt_rows, bt_stride, n_workers, 0, max_group_rows, plan, plan_capacity,
                                     plan_words, workspace_bytes);
}

extern "C" int nsd_attn_plan_build_claimed(const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                           int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                           int64_t bt_rows, int64_t bt_stride, int n_workers, int static_slots,
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
  if (static_slots < 0) return fail(NSD_ERR_INVALID, "plan: static_slots=%d", static_slots);
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

  // 3. pieces per segment.  Every segment starts with the fewest pieces of
  //    at most kMaxPieceBlocks blocks; then, while the plan has fewer than
  //    n_workers pieces, one more piece goes to the segment whose pieces are
  //    the longest (ties: the lower segment), as long as its pieces stay at
  //    least kMinPieceBlocks long and it stays within kMaxSlotsPerSegment.
  //    No cut into that many pieces has a shorter longest piece, and with
  //    n_workers = the device's workgroup slots every piece starts at once.
  std::vector<int64_t> seg_pieces(n_segs);
  int64_t n_pieces = 0;
  for (int64_t s = 0; s < n_segs; ++s) {
    const int64_t nb = seg_start[s + 1] - seg_start[s];
    seg_pieces[s] = std::max<int64_t>(1, (nb + kMaxPieceBlocks - 1) / kMaxPieceBlocks);
    if (seg_pieces[s] > kMaxSlotsPerSegment)
      return fail(NSD_ERR_UNSUPPORTED, "plan: a segment of %lld blocks needs more than %d pieces of %d",
                  (long long)nb, kMaxSlotsPerSegment, kMaxPieceBlocks);
    n_pieces += seg_pieces[s];
  }
  {
    // max-heap on blocks per piece, nb_s / n_s, compared without division
    auto shorter = [&](int64_t x, int64_t y) {
      const int64_t ax = (seg_start[x + 1] - seg_start[x]) * seg_pieces[y];
      const int64_t ay = (seg_start[y + 1] - seg_start[y]) * seg_pieces[x];
      return ax != ay ? ax < ay : x > y;
    };
    std::vector<int64_t> heap;
    for (int64_t s = 0; s < n_segs; ++s) heap.push_back(s);
    std::make_heap(heap.begin(), heap.end(), shorter);
    while (n_pieces < n_workers && !heap.empty()) {
      std::pop_heap(heap.begin(), heap.end(), shorter);
      const int64_t s = heap.back();
      heap.pop_back();
      const int64_t nb = seg_start[s + 1] - seg_start[s], n = seg_pieces[s] + 1;
      if (n > kMaxSlotsPerSegment || nb < n * kMinPieceBlocks) continue;  // cut as far as it goes
      seg_pieces[s] = n;
      ++n_pieces;
      heap.push_back(s);
      std::push_heap(heap.begin(), heap.end(), shorter);
    }
  }
  //    Piece k of a segment of nb blocks cut into n starts at k * nb / n
  //    rounded to a multiple of the workgroup's four waves (wave w streams
  //    blocks w, w + 4, ...), so that every piece but the segment's last
  //    gives its waves equal block counts and none waits for another at the
  //    merge; the pieces stay within three blocks of nb / n (ceil(nb / n)
  //    + 3 <= 256 is required, else the cut is the plain one).
  auto piece_blocks = [&](int64_t s, int64_t k) {
    const int64_t nb = seg_start[s + 1] - seg_start[s], n = seg_pieces[s];
    if (nb > (kMaxPieceBlocks - kWavesPerPiece) * n) return std::make_pair(k * nb / n, (k + 1) * nb / n);
    auto start = [&](int64_t j) {
      return j >= n ? nb : (j * nb / n + kWavesPerPiece / 2) / kWavesPerPiece * kWavesPerPiece;
    };
    return std::make_pair(start(k), start(k + 1));
  };

  // 4. pieces to XCDs (workgroup i runs on XCD i % 8): longest first (ties:
  //    segment, then piece order), each to the XCD with the fewest blocks
  //    among those holding fewer than ceil(pieces / 8), so the XCDs get
  //    near-equal work and list lengths that differ by at most one.  Each
  //    XCD's list is then longest first, as the hardware dispatches it, and
  //    laid out per CU below.
  std::vector<std::pair<int64_t, int64_t>> all;  // (segment, piece index)
  all.reserve(n_pieces);
  for (int64_t s = 0; s < n_segs; ++s)
    for (int64_t k = 0; k < seg_pieces[s]; ++k) all.push_back({s, k});
  std::stable_sort(all.begin(), all.end(), [&](const std::pair<int64_t, int64_t>& x,
                                              const std::pair<int64_t, int64_t>& y) {
    const auto bx = piece_blocks(x.first, x.second), by = piece_blocks(y.first, y.second);
    return bx.second - bx.first > by.second - by.first;
  });
  //    With static_slots > 0 and more pieces than that, only the
  //    static_slots (rounded down to a multiple of 8) longest go to the XCD
  //    lists; the rest, longest first, are claimed at run time by the
  //    workgroups that start as slots free up, whichever XCD they run on.
  const int64_t n_static_pieces =
      static_slots >= kXcds && n_pieces > static_slots ? static_slots / kXcds * kXcds : n_pieces;
  const size_t cap = (size_t)((n_static_pieces + kXcds - 1) / kXcds);
  std::vector<std::vector<std::pair<int64_t, int64_t>>> lists(kXcds);
  std::vector<int64_t> load(kXcds, 0);
  for (int64_t i = 0; i < n_static_pieces; ++i) {
    const auto& pc = all[i];
    int x = -1;
    for (int c = 0; c < kXcds; ++c)
      if (lists[c].size() < cap && (x < 0 || load[c] < load[x])) x = c;
    const auto b = piece_blocks(pc.first, pc.second);
    load[x] += b.second - b.first;
    lists[x].push_back(pc);
  }
  //    The attention runs two workgroups per CU, and a launch whose static
  //    workgroups all start at once puts positions j and j + C of an XCD's
  //    list on one CU (C = the XCD's CUs, static_slots / 16): a CU streams
  //    its two pieces at one combined rate, so it ends when their sum is
  //    done.  Lists that need a second workgroup on some CUs are therefore
  //    laid out so that every such CU runs a long piece first and a short
  //    one beside it: the longest C pieces take the first positions, and the
  //    CUs that also get one of the rest are those with the shortest first
  //    pieces, the longest of them paired with the shortest of the rest.
  if (static_slots >= 2 * kXcds) {
    const size_t C = (size_t)(static_slots / kXcds / 2);
    for (auto& lst : lists) {
      if (lst.size() <= C || lst.size() > 2 * C) continue;
      const size_t m = lst.size() - C;  // CUs that run two pieces
      std::vector<std::pair<int64_t, int64_t>> o(lst.size());
      for (size_t i = 0; i < C - m; ++i) o[m + i] = lst[i];
      for (size_t i = 0; i < m; ++i) {
        o[i] = lst[C - m + i];
        o[C + i] = lst[lst.size() - 1 - i];
      }
      lst.swap(o);
    }
  }
  const std::vector<std::pair<int64_t, int64_t>> claimed(all.begin() + n_static_pieces, all.end());
  const size_t longest = n_pieces > 0 ? cap : 0;
  const int64_t target = n_pieces > 0 ? (total + n_pieces - 1) / n_pieces : 0;

  // 5. partial slots for segments cut into several pieces, in segment order.
  std::vector<int32_t> combines;  // kPieceWords per record
  std::vector<int64_t> seg_slot(n_segs, -1), seg_comb(n_segs, -1);
  int64_t n_slots = 0;
  for (int64_t s = 0; s < n_segs; ++s) {
    if (seg_pieces[s] < 2) continue;
    const int32_t* g = &groups[4 * (s / num_kv_heads)];
    seg_comb[s] = (int64_t)combines.size() / kPieceWords;
    seg_slot[s] = n_slots;
    combines.insert(combines.end(), {(int32_t)(s % num_kv_heads), (int32_t)n_slots, (int32_t)seg_pieces[s],
                                     g[0], g[1], 0, 0, 0, 0, 0, 0, 0});
    n_slots += seg_pieces[s];
  }
  const int64_t n_combines = (int64_t)combines.size() / kPieceWords;

  // 6. records: first the static ones in dispatch order (position 8j + x
  //    holds the j-th piece of XCD x's list, or an empty record where that
  //    list is shorter), then the claimed ones in claim order.  Half again
  //    as many workgroups as claimed records follow the static ones (each
  //    claims one record or finds none left), so that an XCD whose slots
  //    free up early can take more than its share.
  const int64_t n_static = total > 0 ? kXcds * (int64_t)longest : 0;
  const int64_t n_claimed = (int64_t)claimed.size();
  const int64_t claim_wgs = round_up8((3 * n_claimed + 1) / 2);
  const int64_t grid = n_static + claim_wgs;
  const int64_t n_records = n_static + n_claimed;
  std::vector<int32_t> records(kPieceWords * n_records, 0);
  int64_t max_blocks = 0;
  auto fill = [&](int32_t* r, int64_t s, int64_t k) {
    const auto b = piece_blocks(s, k);
    const int32_t* g = &groups[4 * (s / num_kv_heads)];
    const bool split = seg_pieces[s] > 1;
    const int32_t rec[kPieceWords] = {
        (int32_t)(s % num_kv_heads), (int32_t)b.first, (int32_t)b.second,
        split ? (int32_t)(seg_slot[s] + k) : -1, g[0], g[1], g[2], g[3],
        split ? (int32_t)seg_comb[s] : -1, split ? (int32_t)seg_slot[s] : 0,
        split ? (int32_t)seg_pieces[s] : 0, (int32_t)s};
    std::copy(rec, rec + kPieceWords, r);
    max_blocks = std::max(max_blocks, b.second - b.first);
  };
  for (int64_t j = 0; j < (int64_t)longest; ++j) {
    for (int x = 0; x < kXcds; ++x) {
      int32_t* r = &records[kPieceWords * (kXcds * j + x)];
      if (j >= (int64_t)lists[x].size()) {
        r[kPieceSlot] = -1;
        r[kPieceComb] = -1;
        r[kPieceSeg] = -1;
        continue;
      }
      fill(r, lists[x][j].first, lists[x][j].second);
    }
  }
  for (int64_t i = 0; i < n_claimed; ++i)
    fill(&records[kPieceWords * (n_static + i)], claimed[i].first, claimed[i].second);

  const int64_t off_groups = NSD_PLAN_HEADER_WORDS;
  const int64_t off_pieces = off_groups + 4 * n_groups;
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
  h[kPlanSizedFor] = n_workers;
  h[kPlanOffPieces] = (int32_t)off_pieces;
  h[kPlanOffCombines] = (int32_t)off_combines;
  h[kPlanWords] = (int32_t)words;
  h[kPlanPieceBlocks] = (int32_t)target;
  h[kPlanBtRows] = (int32_t)std::min<int64_t>(bt_rows, INT32_MAX);
  h[kPlanBtStride] = (int32_t)std::min<int64_t>(bt_stride, INT32_MAX);
  h[kPlanMaxBlocks] = (int32_t)max_blocks;
  h[kPlanStatic] = (int32_t)n_static;
  h[kPlanClaimed] = (int32_t)n_claimed;
  std::copy(groups.begin(), groups.end(), h + off_groups);
  std::copy(records.begin(), records.end(), h + off_pieces);
  std::copy(combines.begin(), combines.end(), h + off_combines);

  *plan_words = words;
  *workspace_bytes = n_combines > 0 || n_claimed > 0 ? plan_workspace_bytes(n_slots, rows_max) : 0;
  return NSD_OK;
}
