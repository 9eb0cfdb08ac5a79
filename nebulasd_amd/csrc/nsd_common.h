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
  kPlanVersion,        // 1
  kPlanRows,           // decode/verify rows covered
  kPlanGroups,         // verify groups
  kPlanPieces,         // (segment, chunk range) pieces
  kPlanWorkers,        // launch grid (multiple of 8)
  kPlanCombines,       // segments cut into >1 piece
  kPlanSlots,          // partial slots
  kPlanRowsMax,        // max query rows per (group, kv head)
  kPlanHq,
  kPlanHkv,
  kPlanOffGroups,      // word offset of groups [n_groups][4] {row_start, q_len, seq_id, ctx}
  kPlanOffWorkerStart, // word offset of worker piece starts [n_workers+1]
  kPlanOffPieces,      // word offset of pieces [n_pieces][4] {segment, chunk_begin, chunk_end, slot}
  kPlanOffCombines,    // word offset of combines [n_combines][4] {segment, first_slot, n_slots, 0}
  kPlanWords,          // total words
};
static_assert(kPlanWords + 1 == NSD_PLAN_HEADER_WORDS, "plan header size");

constexpr int32_t kPlanMagicValue = 0x4E534450;
constexpr int kHeadDim = 128;
constexpr int kBlockTokens = 16;
constexpr int kChunkTokens = 32;
constexpr int kMaxGroupRows = 64;

}  // namespace nsd
