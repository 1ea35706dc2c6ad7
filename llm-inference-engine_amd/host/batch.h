// Step assembly and the per-layer batched attention of one engine step.
//
// BatchAssembler flattens the scheduled sequences of a step like the
// reference's engine::BatchAssembler (src/engine/batch.h:56-142,
// batch.cpp:37-84): concatenated token ids, absolute positions (cache length
// + t), cu_seqlens [B+1], the caches. On top of that it does what the
// reference defers to each sequence's layer-0 append: it grows every cache by
// its T_b tokens up front (all-or-nothing over the whole step: on exhaustion
// the caches grown so far are truncated back) and packs the step descriptor
// the device path consumes: query lengths, post-append context lengths, the
// CSR of block tables and the slot mapping.
//
// BatchedAttention replaces the per-sequence loops of
// model::OptimizedModel::BatchedAttention (src/model/optimized_model.cpp:
// 370-467): one descriptor upload per step, then per layer one KV-append
// launch and one attention launch for every decode row and prefill chunk.
#pragma once

#include <cstdint>
#include <span>
#include <vector>

#include "block_pool.h"
#include "ehip.h"
#include "paged_kv_cache.h"
#include "status.h"

namespace ehip::host {

struct BatchSeqInput {
  // Tokens this sequence feeds this step (prefill chunk or one decode token).
  std::span<const int32_t> token_ids;
  PagedKvCache* cache = nullptr;
};

struct BatchInputs {
  std::vector<int32_t> token_ids;        // [ΣT_b]
  std::vector<int32_t> positions;        // [ΣT_b] absolute positions
  std::vector<int32_t> cu_seqlens;       // [B+1]
  std::vector<PagedKvCache*> caches;     // [B]
  std::vector<int32_t> query_lens;       // [B]   T_b
  std::vector<int64_t> context_lens;     // [B]   L_b after the append
  std::vector<int32_t> table_offsets;    // [B+1] CSR offsets
  std::vector<int32_t> table_ids;        // block ids, sequence-major
  std::vector<int64_t> slot_mapping;     // [ΣT_b]

  int64_t num_seqs() const { return static_cast<int64_t>(caches.size()); }
  int64_t num_tokens() const { return static_cast<int64_t>(token_ids.size()); }
  // View of the packed step for ehip_step_upload / ehip_plan_counts; valid
  // while this object is unchanged.
  ehip_step_desc desc() const;
};

class BatchAssembler {
 public:
  // Any T_b >= 1 (prefill chunks).
  Status AssemblePrefill(std::span<const BatchSeqInput> seqs);
  // T_b == 1 for every sequence.
  Status AssembleDecode(std::span<const BatchSeqInput> seqs);
  // Decode rows and prefill chunks in one step (the device path runs both in
  // one launch).
  Status AssembleMixed(std::span<const BatchSeqInput> seqs);

  const BatchInputs& inputs() const { return inputs_; }
  // Bytes reserved by the staging vectors; stable once the high-water step has
  // been seen (steady-state steps allocate nothing).
  size_t staging_bytes() const;

 private:
  enum class Mode { kPrefill, kDecode, kMixed };
  Status Flatten(std::span<const BatchSeqInput> seqs, Mode mode);
  void Clear();
  BatchInputs inputs_;
};

class BatchedAttention {
 public:
  // Geometry comes from the pool (device-resident); heads = H query heads.
  BatchedAttention(ehip_ctx* ctx, const BlockPool* pool, int heads);

  // Once per step, after assembly. Every cache must live on this pool.
  Status Upload(const BatchInputs& inputs);
  // One layer: append the step's new K/V rows (d_k_new, d_v_new [ΣT_b, Hkv, d]
  // fp32) into the layer's slabs, then attention for every row: d_q and d_out
  // [ΣT_b, H, d] fp32. Layers come in order 0..L-1 once per step.
  Status ForwardLayer(int layer, const float* d_q, const float* d_k_new, const float* d_v_new,
                      float* d_out);
  // The same with RoPE fused into the append: d_q is rotated in place and the
  // new K rows on their way into the slabs, at each row's absolute position
  // (the rows' context position), as OptimizedModel's layer forward does with
  // kernels::RopeApplyF32 before the append (src/model/optimized_model.cpp:284-291).
  // d_cos/d_sin are the [positions, d/2] fp32 tables (Rope::cos()/sin()).
  struct RopeTables {
    const float* d_cos = nullptr;
    const float* d_sin = nullptr;
    int64_t positions = 0;
  };
  Status ForwardLayerRope(int layer, float* d_q, const float* d_k_new, const float* d_v_new,
                          const RopeTables& rope, float* d_out);

  const ehip_geometry& geometry() const { return geom_; }
  float scale() const { return geom_.scale; }

 private:
  ehip_ctx* ctx_;
  const BlockPool* pool_;
  ehip_geometry geom_{};
  Status CheckLayer(int layer) const;
  Status Attend(int layer, const float* d_q, float* d_out);

  bool uploaded_ = false;
  bool has_slots_ = false;
  int next_layer_ = 0;
};

}  // namespace ehip::host
