// Kernel launch interfaces (host side), shared by the runtime and the kernel
// translation units.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "plan.h"

namespace ehip {

// Device-side error bits (OR-ed into the context's error word).
enum : int32_t {
  kErrSlotRange = 1,   // an append slot outside the slab
  kErrBlockRange = 2,  // a block-table id outside the slab
};

struct DecodeParams {
  const float* q;           // [rows, H, d]
  const void* k_slab;       // [slab_blocks, Hkv, bs, d] f32 or bf16
  const void* v_slab;
  float* out;               // [rows, H, d]
  const RowDesc* rows;
  const WorkItem* items;
  const int32_t* table;     // CSR ids (or a single sequence's table)
  float* part_o;            // [partials, g, d]
  float* part_ml;           // [partials, g, 2]
  int32_t* err;
  int64_t block_stride;     // elements
  int64_t head_stride;      // elements between kv heads of a block (bs * d for slabs; L * d
                            // for a contiguous [Hkv, L, d] cache read as one identity table);
                            // the fp32 kernels honour it, the bf16/INT8 ones assume bs * d
  int64_t slab_blocks;
  int32_t n_items;
  int32_t n_rows;
  const int32_t* merge_rows;  // [n_merge] rows with more than one split
  int32_t n_merge;
  int32_t n_joint;          // joint work items in the plan
  int32_t joint_rows;       // rows of the plan's largest joint item (1: none)
  const ItemRowsX* items_x; // rows 3 and 4 per item when joint_rows > 2, else null
  int32_t heads;
  int32_t kv_heads;
  int32_t group;            // g = H / Hkv
  int32_t d;
  int32_t bs;
  float scale_log2;         // scale * log2(e)
  int64_t max_length;       // longest row (keys attended)
  int32_t has_prefill;      // the step also has MFMA prefill items
  const float* k_scale;     // INT8/FP8 KV: per-(block, kv head) scales [slab_blocks, Hkv]
  const float* v_scale;
  // Fused append (bf16 MFMA decode of an all-decode step): the step's new K/V
  // rows [rows, Hkv, d] fp32 and their slots. The item flagged as its row's
  // last key range stores the row's new bf16 K/V at the slot and uses them for
  // that key. Null: the rows were appended by a separate launch.
  const float* new_k;
  const float* new_v;
  const int64_t* slots;
  uint32_t* queue;          // kItemQueues ticket counters, kQueueStride words apart
                            // (zero at launch; MFMA kernel only)
  uint32_t* queue_done;     // wavefronts finished (zero at launch)
  int32_t queue_spread;     // sub-queue of workgroup b: (b / 8) mod count (else b mod count)
  int32_t queues;           // sub-queues used, 1..kItemQueues
};

// The persistent decode kernel's item queue is split into kItemQueues
// sub-queues: sub-queue q serves the items whose index is q modulo the
// sub-queue count, to the wavefronts whose index is q modulo it. One counter
// takes every ticket of a launch through one memory channel's atomic unit,
// which serialises them (about 12 ns apiece on MI355X); counters in separate
// 256-byte lines draw in parallel. Up to kItemQueues of them; kDefaultQueues
// by default. Fewer sub-queues balance the end of a launch better (each is
// drawn by more wavefronts): C4 with 1536-key items, one process, interleaved
// calls: 388.5 us at 32, 386.7 at 16, 384.2 at 8, 384.4 at 4, 383.3 at 1.
// Eight keeps most of that and 8x one counter's ticket rate.
constexpr int kItemQueues = 32;
constexpr int kDefaultQueues = 8;
constexpr int kQueueStride = 64;  // words between counters

// The item-queue counters of a context (kItemQueues ticket counters and the
// wavefronts-done counter); each persistent decode launch leaves them zero,
// so launches on the context's stream, eager or replayed from a captured
// graph, need no clearing between them.
struct QueueState {
  uint32_t* d_counters;
  uint32_t* d_done;
};

struct PrefillParams {
  const float* q;           // [rows, H, d]
  const void* k_slab;       // bf16 slabs
  const void* v_slab;
  float* out;               // [rows, H, d]
  const PrefillItem* items;
  const int32_t* table;
  const RowDesc* rows;      // split slots of the rows of key-split items
  float* part_o;            // [partials, g, d]
  float* part_ml;           // [partials, g, 2]
  int32_t* err;
  int64_t block_stride;
  int64_t slab_blocks;
  int32_t n_items;
  int32_t heads;
  int32_t kv_heads;
  int32_t group;
  int32_t d;
  int32_t bs;
  float scale_log2;
};

// Causal prefill chunks on MFMA (bf16 K/V, d = 128, g in {4, 8}, bs >= 16):
// one 4-wavefront workgroup per (chunk, kv head, M query rows). Returns
// false (nothing launched) for shapes it does not cover.
bool LaunchPrefillMfma(const PrefillParams& p, hipStream_t stream, hipError_t* err);
// Query rows per prefill work item for this geometry, or 0 when the MFMA
// prefill kernel does not cover it (bf16 K/V, d = 128, g in {4, 8}, bs >= 16,
// slabs below 4 GiB).
int PrefillRowsPerItem(int kv_dtype, int d, int group, int bs, int64_t slab_bytes);

// Launch the decode kernel family for the given plan (one wavefront per work
// item; picks the specialised (dtype, d, g) kernel or the generic one), then,
// if any row was split, the merge of the split partials. The kernel boundary
// between the two publishes the partials: no device-wide fences or counters.
hipError_t LaunchDecode(const DecodeParams& p, int kv_dtype, const Tuning& tune, QueueState* queue,
                        hipStream_t stream);

// Whether the matrix-core decode kernel covers p for this KV type (bf16: d
// 64/128, g 1/2/4/8; fp32: d 64, g 1/2/4/7/8; bs >= 16, 16-byte aligned
// operands, not forced to the VALU kernel by Tuning::decode_valu). Only it
// performs the fused append.
bool DecodeMfmaCovers(const DecodeParams& p, int kv_dtype, const Tuning& tune);
// bf16- or fp32-KV decode with QK^T on MFMA; returns false (nothing launched)
// when DecodeMfmaCovers does not hold.
bool LaunchDecodeMfma(const DecodeParams& p, int kv_dtype, const Tuning& tune, QueueState* queue,
                      hipStream_t stream, hipError_t* err);
// INT8 or FP8 (E4M3) KV decode (paged_decode_q8.hip); false when the shape
// is not covered.
bool LaunchDecodeQ8(const DecodeParams& p, bool fp8, hipStream_t stream, hipError_t* err);

// KvScatter: rows [T, Hkv, d] fp32 into slabs (fp32 copy or bf16 RNE).
hipError_t LaunchKvScatter(const float* src_k, const float* src_v, const int64_t* slots,
                           int64_t t_dim, int32_t kv_heads, int32_t d, int32_t bs,
                           int64_t slab_blocks, void* k_slab, void* v_slab, int kv_dtype,
                           int32_t* err, hipStream_t stream);

hipError_t LaunchKvGather(const float* k_slab, const float* v_slab, const int32_t* table,
                          int32_t bs, int64_t length, int32_t kv_heads, int32_t d,
                          int64_t slab_blocks, float* out_k, float* out_v, int32_t* err,
                          hipStream_t stream);

// INT8 or FP8 (E4M3) append with per-(block, kv head) scales, one wavefront
// per (append group, kv head).
hipError_t LaunchAppendQ8(const float* src_k, const float* src_v, const Q8Group* groups,
                          int64_t n_groups, const int32_t* rows, int kv_heads, int d, int bs,
                          int64_t slab_blocks, void* k_slab, void* v_slab, float* k_scale,
                          float* v_scale, bool fp8, int32_t* err, hipStream_t stream);

// Fused RoPE + KV append of one step's rows (q rotated in place; rotated K and
// V scattered at the rows' slots; row r at position rows[r].length - 1).
hipError_t LaunchRopeKvAppend(float* q, const float* src_k, const float* src_v,
                              const RowDesc* rows, const float* cos_t, const float* sin_t,
                              const int64_t* slots, int64_t n_rows, int heads, int kv_heads,
                              int d, int bs, int64_t slab_blocks, void* k_slab, void* v_slab,
                              int kv_dtype, int32_t* err, hipStream_t stream);

// Allocation-free single-sequence decode (decode_static.hip): the one-row
// plan and its split partials live in a per-device static scratch array of
// kStaticScratchBytes. InitStaticScratch fetches the array's address on the
// current device and creates the device's ordering event (once per device;
// called at context creation).
constexpr size_t kStaticScratchBytes = size_t{4} << 20;
hipError_t InitStaticScratch(int device);
// Scratch bytes a row cut into nsplit key splits needs (plan + partials).
size_t StaticScratchNeed(int64_t nsplit, int kv_heads, int group, int d);
// Writes the plan of one row of `length` keys, cut into nsplit splits of
// split_len keys, into the device's scratch and runs the fp32 decode (and the
// split merge) on it; base carries everything else (q, slabs, table, out,
// geometry). Eager calls on one device run in call order, whichever context
// or stream makes them (each waits for the previous call's end). A call on a
// capturing stream is not ordered that way. hipErrorNotInitialized if the
// device's address was not fetched, hipErrorInvalidValue if the plan does not
// fit.
hipError_t LaunchSingleRowStatic(const DecodeParams& base, int device, int32_t length,
                                 int32_t split_len, int32_t nsplit, const Tuning& tune,
                                 QueueState* queue, hipStream_t stream);

// Packed linear layer (packed_gemm.hip): y[m, n] = x[m, k] W^T (+ bias) over
// the reference's panel layout [ceil(n/16), k, 16].
struct GemmParams {
  const float* x;       // [m, k]
  uint16_t* xp;         // x's three bf16 planes [3][m_pad][k_pad] (workspace)
  const void* wp;       // packed weight
  const float* bias;    // [n] or null
  float* y;             // [m, n]
  float* part;          // [splits, m, n] partial sums (splits > 1)
  int64_t m, k, n;
  int64_t m_pad, k_pad;  // m, k rounded up to whole 64 x 64 tiles
  int64_t panels;       // ceil(n / 16)
  int32_t group_panels;  // panels per workgroup (the weight type's tile width)
  int64_t k_split;      // k per split (a multiple of 32)
  int32_t splits;
  int32_t x_vec;        // x rows are 16-byte aligned (k % 4 == 0, aligned base)
};
// Tiles and k splits for a call (cus: the device's CU count).
void PlanPackedGemm(int64_t m, int64_t k, int64_t n, int weight_dtype, int cus, GemmParams* p);
// Workspace bytes of x's planes for the planned call.
size_t PackedGemmPlaneBytes(const GemmParams& p);
hipError_t LaunchPackedGemm(const GemmParams& p, int weight_dtype, hipStream_t stream);
hipError_t LaunchPackWeightPanels(const void* w, int weight_dtype, int64_t n, int64_t k, void* wp,
                                  hipStream_t stream);

hipError_t LaunchFillNormal(void* dst, int64_t n, int dtype, float mean, float stddev,
                            uint64_t seed, hipStream_t stream);

}  // namespace ehip
