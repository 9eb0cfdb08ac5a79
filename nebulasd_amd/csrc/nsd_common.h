// Internal host-side helpers shared by the C ABI translation units.
#pragma once

#include <stdint.h>

#include "nsd_attn.h"

namespace nsd {

// Records `fmt` (printf-style) as this thread's last error and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Plan word layout (int32), shared by the planner and the attention launch.
enum PlanHeader {
  kPlanMagic = 0,      // 0x4E534450
  kPlanVersion,        // 2
  kPlanRows,           // decode/verify rows covered
  kPlanGroups,         // verify groups
  kPlanPieces,         // (segment, block range) pieces
  kPlanWorkers,        // launch grid (multiple of 8)
  kPlanCombines,       // segments cut into >1 piece
  kPlanSlots,          // partial slots
  kPlanRowsMax,        // max query rows per (group, kv head)
  kPlanHq,
  kPlanHkv,
  kPlanOffGroups,      // word offset of groups [n_groups][4] {row_start, q_len, seq_id, ctx}
  kPlanOffWorkers,     // word offset of the worker table [n_workers][kWorkerWords]
  kPlanOffPieces,      // word offset of pieces [n_pieces][kPieceWords]
  kPlanOffCombines,    // word offset of combines [n_combines][kPieceWords]
  kPlanWords,          // total words
  kPlanPieceStride,    // piece records per worker: worker w's records start at w * stride
  kPlanRingStages,     // blocks per claimed group the records' group counts assume
};
static_assert(kPlanRingStages < NSD_PLAN_HEADER_WORDS, "plan header size");

// A piece: blocks [blk_begin, blk_end) of one (group, kv head) segment, with
// the group's description inlined so a worker needs one record per piece.
// The workgroup's waves claim a piece's blocks in groups of ring_stages(nt)
// consecutive blocks; kPieceGroupEnd counts the groups of the worker's pieces
// up to and including this one.
enum PieceField {
  kPieceHead = 0,   // kv head
  kPieceBlkBegin,   // first 16-token block
  kPieceBlkEnd,     // one past the last block
  kPieceSlot,       // partial slot, or -1 when the piece is the whole segment
  kPieceRowStart,   // first decode row of the group
  kPieceQLen,       // rows in the group
  kPieceSeqId,      // block-table row
  kPieceCtx,        // tokens before the group's first new token
  kPieceComb,       // combine record of the segment, or -1
  kPieceCombFirst,  // first partial slot of the segment
  kPieceCombSlots,  // partial slots of the segment
  kPieceGroupEnd,   // groups of this worker's pieces 0 .. this one
  kPieceWords,
};
// A worker-table row: {first piece, end piece, <first piece record>, 0, 0}.
// Worker w's records are pieces [w * stride, w * stride + count), so the
// kernel loads them without reading the table first.
constexpr int kWorkerWords = 16;
constexpr int kWorkerFirstPiece = 2;
// A combine record: {kv head, first slot, slot count, row start, q_len, 0, 0, 0}.
enum CombineField { kCombHead = 0, kCombFirst, kCombSlots, kCombRowStart, kCombQLen };

constexpr int32_t kPlanMagicValue = 0x4E534450;
constexpr int32_t kPlanVersionValue = 6;
constexpr int kHeadDim = 128;
constexpr int kBlockTokens = 16;
constexpr int kMaxGroupRows = 64;
constexpr int kMaxSlotsPerSegment = 128;
constexpr int kMaxWorkerPieces = 32;   // pieces one workgroup keeps records of

// Attention kernel shape for groups of up to 16*nt query rows (nt = 1..4):
// K/V ring depth, which is also the size of a claimed group of blocks, and
// waves per workgroup (one workgroup per compute unit).  Every shape now
// streams with eight waves and a one-block ring; the plan still records the
// depth it was built for, so a kernel built for another depth rejects it.
constexpr int ring_stages(int /*nt*/) { return 1; }
constexpr int attn_waves(int /*nt*/) { return 8; }

}  // namespace nsd
