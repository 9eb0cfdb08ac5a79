// Internal host-side helpers shared by the C ABI translation units.
#pragma once

#include <stdint.h>

#include "nsd_attn.h"

namespace nsd {

// Records `fmt` (printf-style) as this thread's last error and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The FFN's up/gate projection + SiLU-and-mul through the split-k GEMM's
// gated unit (nsd_gemm.hip), for shapes whose units fill the device (one
// unit per 48 output columns, <= 112 rows); *served is false (and nothing is
// launched) for the others.  Arguments as nsd_up_gate_silu_and_mul.
int up_gate_silu_gated(const void* x, const void* up_gate, void* y, int64_t n_rows, int64_t hidden, int64_t inter,
                       void* stream, bool* served);

// Plan word layout (int32), shared by the planner and the attention launch.
enum PlanHeader {
  kPlanMagic = 0,      // 0x4E534450
  kPlanVersion,        // kPlanVersionValue
  kPlanRows,           // decode/verify rows covered
  kPlanGroups,         // verify groups
  kPlanPieces,         // piece records (one workgroup each; empty records pad the XCD lists)
  kPlanWorkers,        // launch grid: equal to kPlanPieces, a multiple of 8
  kPlanCombines,       // segments cut into >1 piece
  kPlanSlots,          // partial slots
  kPlanRowsMax,        // max query rows per (group, kv head)
  kPlanHq,
  kPlanHkv,
  kPlanOffGroups,      // word offset of groups [n_groups][4] {row_start, q_len, seq_id, ctx}
  kPlanSizedFor,       // the n_workers (pieces asked for) the plan was cut for
  kPlanOffPieces,      // word offset of pieces [n_pieces][kPieceWords]
  kPlanOffCombines,    // word offset of combines [n_combines][kPieceWords]
  kPlanWords,          // total words
  kPlanPieceBlocks,    // mean blocks per piece, rounded up
  kPlanBtRows,         // block-table rows every piece's seq_id was checked against
  kPlanBtStride,       // block-table row length every piece's block range was checked against
  kPlanMaxBlocks,      // most 16-token blocks in one piece
  kPlanStatic,         // workgroups 0 .. kPlanStatic-1 stream records of the same index
  kPlanClaimed,        // records kPlanStatic .. +kPlanClaimed-1, claimed at run time by the
                       // later workgroups in order (kPlanWorkers - kPlanStatic of them)
};
static_assert(kPlanMaxBlocks < NSD_PLAN_HEADER_WORDS, "plan header size");

// A piece: blocks [blk_begin, blk_end) of one (group, kv head) segment, with
// the group's description inlined so a workgroup needs one record.  A record
// with q_len 0 is empty (it pads an XCD's list; its workgroup exits at once).
enum PieceField {
  kPieceHead = 0,   // kv head
  kPieceBlkBegin,   // first 16-token block
  kPieceBlkEnd,     // one past the last block
  kPieceSlot,       // partial slot, or -1 when the piece is the whole segment
  kPieceRowStart,   // first decode row of the group
  kPieceQLen,       // rows in the group (0: empty record)
  kPieceSeqId,      // block-table row
  kPieceCtx,        // tokens before the group's first new token
  kPieceComb,       // combine record of the segment, or -1
  kPieceCombFirst,  // first partial slot of the segment
  kPieceCombSlots,  // partial slots of the segment
  kPieceSeg,        // segment index (group * Hkv + kv head)
  kPieceWords,
};
// A combine record: {kv head, first slot, slot count, row start, q_len, 0, 0, 0}.
enum CombineField { kCombHead = 0, kCombFirst, kCombSlots, kCombRowStart, kCombQLen };

constexpr int32_t kPlanMagicValue = 0x4E534450;
constexpr int32_t kPlanVersionValue = 9;
constexpr int kHeadDim = 128;
constexpr int kBlockTokens = 16;
constexpr int kMaxGroupRows = 48;       // query rows of one segment: three 16-row tiles in one wave
constexpr int kMaxSlotsPerSegment = 128;
constexpr int kMaxPieceBlocks = 256;    // blocks of one piece (four waves, one block id per lane)
// Shortest piece a cut makes: two blocks per wave, whose loads are both in
// flight from the piece's start, so a shorter cut saves no latency and only
// adds the merge of the segment's pieces.
constexpr int kMinPieceBlocks = 8;
constexpr int kWavesPerPiece = 4;       // waves of an attention workgroup (wave w: blocks w, w + 4, ...)
constexpr int kXcds = 8;                // workgroup i of a launch runs on XCD i % 8

// Whether a plan keeps every sequence's rows in one verify group, as the
// fused prologue + attention launch needs (then no workgroup reads a new K/V
// row that another one writes in the same launch).  plan_host is a checked
// plan's header and tables.
bool plan_keeps_sequences_whole(const int32_t* plan_host);

// Attention workspace: the claim counter of plans with claimed records
// (zero between calls; its 256 bytes are reserved in every layout, so no
// other plan's partials land there), then the partials of the split
// segments, normalised O (fp16) and log2-sum-exp (fp32) per slot and row.
constexpr int64_t kClaimBytes = 256;
inline int64_t plan_workspace_bytes(int64_t n_slots, int64_t rows_max) {
  return kClaimBytes + (n_slots * rows_max * (int64_t)(kHeadDim * 2 + 4) + 255) / 256 * 256;
}

}  // namespace nsd
