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
  kPlanBtRows,         // block-table rows every piece's seq_id was checked against
  kPlanBtStride,       // block-table row length every piece's block range was checked against
  kPlanMaxBlocks,      // most 16-token blocks one worker streams
};
static_assert(kPlanMaxBlocks < NSD_PLAN_HEADER_WORDS, "plan header size");

// A piece: blocks [blk_begin, blk_end) of one (group, kv head) segment, with
// the group's description inlined so a worker needs one record per piece.
// kPieceKvBase counts the blocks of the worker's earlier pieces: the piece's
// block ids sit at that offset of the worker's id list.
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
  kPieceKvBase,     // blocks of this worker's pieces before this one
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
constexpr int32_t kPlanVersionValue = 7;
constexpr int kHeadDim = 128;
constexpr int kBlockTokens = 16;
constexpr int kMaxGroupRows = 64;
constexpr int kMaxSlotsPerSegment = 128;
constexpr int kMaxWorkerPieces = 4;    // pieces one workgroup streams (their query rows stay in registers)
constexpr int kMaxWorkerBlocks = 1024; // blocks one workgroup streams (its LDS id list)

}  // namespace nsd
