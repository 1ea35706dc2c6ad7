// Step planner: turns one ragged scheduler step (ehip_step_desc) into the
// packed device descriptor the attention kernels walk. Host-only C++ (no HIP
// calls), so the CPU test suite exercises it through ehip_plan_counts.
//
// The reference threads a decode over (sequence, kv head) units
// (src/kernels/paged_attention.cpp:140-146) and a varlen prefill over
// (sequence, head, 32-query block) units (src/kernels/attention.cpp:166-186).
// On the GPU one unit of work is a (query row, kv head, key split): the g
// query heads of a kv head share one pass over its K/V (the reference's reuse
// rule, src/kernels/internal/attention_common.h:229-235), and a long context
// is cut into splits of whole 64-token tiles whose (max, sum, output)
// partials are merged with a log-sum-exp rescale.
//
// Shared prefixes: blocks are shared only as whole leading blocks of forked
// sequences (BlockPool::Share, src/kvcache/block_pool.cpp:256-266; shared
// blocks are immutable, docs/design/paged-kv-cache.md:487-507), and every row
// of a prefill chunk reads its sequence's table. The planner pairs rows whose
// tables agree on a run of leading full blocks and emits "joint" work items
// for that run: one pass over the shared K/V serves both rows, each of which
// still gets its own split partial.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "ehip.h"

namespace ehip {

// Tuning switches (EHIP_* environment variables), read once when a context is
// created and carried by it, as the reference memoizes its dispatch choice in
// a function-local static (src/kernels/paged_attention.cpp:93, :125): the
// planner and the launch paths never read the environment. The context-free
// planning entry points (ehip_plan_counts / _items / _prefill_items) read it
// per call.
struct Tuning {
  int32_t split_tokens = 0;    // EHIP_SPLIT_TOKENS: fixed base split length (0: per step)
  int64_t target_items = 0;    // EHIP_TARGET_ITEMS: decode work-item target (0: default)
  int32_t tail_split = 0;      // EHIP_TAIL_SPLIT: tail piece length in keys (0: no tail pieces)
  double tail_frac = 0.08;     // EHIP_TAIL_FRAC: share of the step's keys cut into tail pieces
  int8_t split_even = -1;      // EHIP_SPLIT_EVEN=1/0: a row's ranges of near-equal length
                               // always / never (default: when items <= the item target)
  bool joint = true;           // EHIP_NO_JOINT=1: no joint items over shared prefixes
  bool prefill = true;         // EHIP_PREFILL=0: chunk rows stay on the decode kernels
  double prefill_split = 2.0;  // EHIP_PREFILL_SPLIT: key-split threshold in shares (0: none)
  bool decode_valu = false;    // EHIP_DECODE_KERNEL=valu: all-VALU decode kernels
  bool decode_tile16 = false;  // EHIP_DECODE_TILE=16: one 16-key MFMA half per tile
  bool decode_bufs3 = false;   // EHIP_DECODE_BUFS=3: three tiles in registers
  bool decode_persist = true;  // EHIP_DECODE_PERSIST=0: one workgroup per work item
  int32_t decode_slots = 0;    // EHIP_DECODE_SLOTS: cap on persistent wavefronts (0: none)
  bool decode_qspread = true;  // EHIP_DECODE_QSPREAD=0: each sub-queue served by one XCD
  int32_t decode_queues = 0;   // EHIP_DECODE_QUEUES: item sub-queues (0: default)
  bool decode_wg = true;       // EHIP_DECODE_WG=0: no workgroup-per-row small fp32 steps
  bool decode_split4 = true;   // EHIP_DECODE_SPLIT4=0: one wavefront per item in small fp32 steps
  bool fused_append = true;    // EHIP_FUSED_APPEND=0: append and attention in two launches
};

// The switches as the environment sets them now.
Tuning ReadTuning();

// One query row: its sequence's table slice and the keys it attends (a decode
// row attends the whole post-append context; row t of a prefill chunk
// attends P + t + 1 keys). Its splits own partial slots
// [split_base*Hkv + hk*nsplit, +nsplit) for kv head hk.
struct RowDesc {
  int32_t table_off;   // first entry of this row's sequence in the CSR ids
  int32_t length;      // keys attended, >= 1
  int32_t split_base;  // prefix sum of nsplit over earlier rows
  int32_t nsplit;      // splits of this row (joint ones first)
};

// One work item = one wavefront: keys [tok_begin, tok_end) of row0 (and, for
// a joint item, of the other rows reading the same blocks over the range:
// row1, -1 otherwise; a group of three or four rows keeps rows 3 and 4 in the
// plan's ItemRowsX array, read only by the kernels that serve such groups),
// for the g query heads of one kv head. `split` is the partial slot index
// inside each row's range (the same for every row of a joint item). The
// range's table slice starts at table_off, so a kernel can fetch the table,
// the queries and the row descriptors in parallel as soon as it has the item.
struct WorkItem {
  int32_t row0;
  int32_t row1;
  int32_t tok_begin;
  int32_t tok_end;
  int32_t hk_split;  // kv_head | split << 12
  int32_t table_off;
  int32_t first_block0;  // block id of token tok_begin (-1: read the table)
  int32_t first_block1;  // block id of token min(tok_begin + 16, tok_end - 1)
  int32_t first_block2;  // block id of token min(tok_begin + 32, tok_end - 1)
  int32_t first_block3;  // block id of token min(tok_begin + 48, tok_end - 1)
};

// Rows 3 and 4 of a joint item (-1 where absent), parallel to the work list
// when the plan has groups of more than two rows.
struct ItemRowsX {
  int32_t row2;
  int32_t row3;
};

// One causal prefill block: query rows q0 .. q0+M-1 of a chunk of `chunk`
// rows (starting at packed row row_base) over `past` cached keys, for the g
// query heads of one kv head (M = PrefillRowsPerItem for the geometry).
// A block whose key range is long relative to the step's prefill work is
// cut into key splits [key_begin, key_end) of whole 32-key tiles; each split
// writes (max, sum, output) partials for its rows that the split merge
// combines (the rows' RowDesc.nsplit counts the splits). An unsplit item
// covers [0, P + q0 + rows) and writes the output directly.
struct PrefillItem {
  int32_t row_base;
  int32_t chunk;
  int32_t past;
  int32_t q0;
  int32_t hk_split;   // kv_head | split << 12
  int32_t table_off;
  int32_t key_begin;
  int32_t key_end;
};

// Rows per joint item: at most 4, and at most 16 / g, so that the item's
// virtual heads (g per row) fill no more than the 16 rows of one MFMA block.
constexpr int kMaxJointRows = 4;
constexpr int JointRowsCap(int64_t group) {
  return group <= 0 ? 1 : (16 / group >= kMaxJointRows ? kMaxJointRows
                                                        : (16 / group < 1 ? 1 : int(16 / group)));
}
// The packed (kv head, split) word of a work item: kv head in bits 0-11,
// split in bits 12-28, and bit 30 set on the item whose key range ends at its
// row's last key (the item that appends the row's new token in the fused
// append + attention launch).
constexpr int kHkBits = 12;
constexpr int kSplitBits = 17;
constexpr int32_t kLastRangeFlag = int32_t{1} << 30;

constexpr int32_t PackHkSplit(int32_t hk, int32_t split) { return hk | (split << kHkBits); }
constexpr int32_t UnpackHk(int32_t v) { return v & ((1 << kHkBits) - 1); }
constexpr int32_t UnpackSplit(int32_t v) { return (v >> kHkBits) & ((1 << kSplitBits) - 1); }
constexpr bool IsLastRange(int32_t v) { return (v & kLastRangeFlag) != 0; }

// Rows of one step landing in one block (INT8/FP8 append): the block, the first
// new row's offset in it, the row count and where its row indices start in
// Plan::q8_rows.
struct Q8Group {
  int32_t block;
  int32_t off0;
  int32_t n;
  int32_t row0;
};

struct Plan {
  std::vector<RowDesc> rows;
  std::vector<WorkItem> items;
  std::vector<ItemRowsX> items_x;   // empty unless joint_rows > 2; else one per item
  std::vector<PrefillItem> prefill;  // chunk rows served by the MFMA prefill kernel
  std::vector<int32_t> groups;      // member rows of each joint group (host side) ...
  std::vector<int32_t> group_start;  // ... group i is groups[group_start[i] .. group_start[i+1])
  std::vector<int32_t> table_ids;   // CSR ids, copied
  std::vector<int64_t> slots;       // slot mapping of appended tokens (may be empty)
  std::vector<int32_t> merge_rows;  // rows with more than one split, ascending
  std::vector<Q8Group> q8_groups;   // scaled-KV append groups (INT8/FP8 with slots)
  std::vector<int32_t> q8_rows;     // row indices of the groups, in offset order
  int64_t partials = 0;             // sum over rows of nsplit * Hkv
  int64_t max_length = 0;           // longest visible length (largest position + 1)
  int32_t split_tokens = 0;         // base split length chosen for this step
  int64_t joint_items = 0;
  int32_t joint_rows = 1;           // rows of the largest joint item (1: none)
  // Keys whose re-reads the joint items save: for each group, its shared
  // prefix times (members - 1).
  int64_t shared_tokens = 0;
  bool any_split = false;           // some decode row has more than one split (merge needed)
  bool all_decode = false;          // every row is its sequence's only new token (T_b == 1)
};

// Geometry validation shared by every entry point. Returns a StatusCode and
// fills *err on failure.
int ValidateGeometry(const ehip_geometry& g, std::string* err);

// Effective block stride in elements (geometry value or Hkv*bs*d).
int64_t BlockStride(const ehip_geometry& g);

// KV element types whose slabs carry per-(block, kv head) scales.
inline bool ScaledKv(int kv_dtype) { return kv_dtype == EHIP_KV_INT8 || kv_dtype == EHIP_KV_FP8; }

// Base split length: sized so that the step yields enough work items to fill
// the chip (a few per SIMD) without drowning in partial-merge traffic.
// Tuning::split_tokens overrides it (rounded to a multiple of 64).
int32_t ChooseSplitTokens(const ehip_geometry& g, int64_t unit_tokens, const Tuning& tune);
// Longest key range of one decode work item.
int32_t MaxSplitTokens(const ehip_geometry& g);
// Split length of one row of `len` keys given the step's base length: the
// base, grown (in whole 64-key units, up to MaxSplitTokens) so the row has at
// most 64 splits while the cap allows.
int32_t RowSplitTokens(const ehip_geometry& g, int32_t base, int32_t len);
// The split length BuildSingleRowPlan gives a row of `length` keys (the
// single-sequence decode's partition), without building the plan.
int32_t SingleRowSplitTokens(const ehip_geometry& g, int64_t length, const Tuning& tune);

// Validates the step (lengths, CSR offsets, every table id and slot in range)
// and builds the plan. Chunks of at least kMinPrefillRows rows go to the MFMA
// prefill kernel when it covers the geometry (prefill_rows > 0: query rows
// per prefill work item; Tuning::prefill = false keeps every row on the
// decode kernels); their rows get nsplit = 0.
constexpr int32_t kMinPrefillRows = 16;
constexpr int32_t kPrefillTile = 32;       // keys per prefill tile
constexpr int32_t kPrefillSlots = 512;     // workgroups resident at once (2 per CU)
constexpr int32_t kMinPrefillSplitTiles = 8;
// head_major: K/V are one contiguous [Hkv, L, d] cache read through an
// identity table (block_stride = bs * d, kv heads L * d apart), so the slab
// rule block_stride >= Hkv * bs * d does not apply.
int BuildPlan(const ehip_geometry& g, const ehip_step_desc& s, const Tuning& tune, Plan* plan,
              std::string* err, int prefill_rows = 0, bool head_major = false);

// Plan for one row reading a device-resident table (single-sequence paged
// decode): one row of `length` keys, table offset 0.
int BuildSingleRowPlan(const ehip_geometry& g, int64_t length, int64_t num_blocks,
                       const Tuning& tune, Plan* plan, std::string* err);

}  // namespace ehip
