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
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "ehip.h"

namespace ehip {

// One query row: its sequence's table slice and the number of keys it
// attends (a decode row attends the whole post-append context; row t of a
// prefill chunk attends P + t + 1 keys).
struct RowDesc {
  int32_t table_off;   // first entry of this row's sequence in the CSR ids
  int32_t length;      // keys attended, >= 1
  int32_t split_base;  // prefix sum of nsplit over earlier rows
  int32_t split_len;   // tokens per split (multiple of 64, <= 64 * bs)
};

// One work item = one wavefront: keys [split*split_len, min(length,
// (split+1)*split_len)) of row `row`, for all g query heads of kv head
// `kv_head`.
struct WorkItem {
  int32_t row;
  int32_t kv_head;
  int32_t split;
  int32_t nsplit;
};

struct Plan {
  std::vector<RowDesc> rows;
  std::vector<WorkItem> items;
  std::vector<int32_t> table_ids;   // CSR ids, copied
  std::vector<int64_t> slots;       // slot mapping of appended tokens (may be empty)
  int64_t partials = 0;             // sum over rows of nsplit * Hkv
  int32_t split_tokens = 0;         // base split length chosen for this step
};

// Geometry validation shared by every entry point. Returns a StatusCode and
// fills *err on failure.
int ValidateGeometry(const ehip_geometry& g, std::string* err);

// Effective block stride in elements (geometry value or Hkv*bs*d).
int64_t BlockStride(const ehip_geometry& g);

// Base split length: sized so that the step yields enough work items to fill
// the chip (a few per SIMD) without drowning in partial-merge traffic.
// EHIP_SPLIT_TOKENS overrides it (rounded to a multiple of 64).
int32_t ChooseSplitTokens(const ehip_geometry& g, int64_t unit_tokens);

// Validates the step (lengths, CSR offsets, every table id and slot in range)
// and builds the plan. `with_tables` copies the CSR ids; `table_ids_valid`
// false skips the id range check (ids live on the device).
int BuildPlan(const ehip_geometry& g, const ehip_step_desc& s, Plan* plan, std::string* err);

// Plan for rows that all read one device-resident table (single-sequence
// paged decode): one row of `length` keys, table offset 0.
int BuildSingleRowPlan(const ehip_geometry& g, int64_t length, int64_t num_blocks, Plan* plan,
                       std::string* err);

}  // namespace ehip
