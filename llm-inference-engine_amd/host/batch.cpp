#include "batch.h"

#include "device_buffer.h"
#include "kernels.h"

namespace ehip::host {
namespace {

template <class T>
size_t VectorBytes(const std::vector<T>& v) {
  return v.capacity() * sizeof(T);
}

}  // namespace

ehip_step_desc BatchInputs::desc() const {
  ehip_step_desc s{};
  s.num_seqs = static_cast<int32_t>(caches.size());
  s.h_query_lens = query_lens.data();
  s.h_context_lens = context_lens.data();
  s.h_table_offsets = table_offsets.data();
  s.h_table_ids = table_ids.data();
  s.h_slot_mapping = slot_mapping.empty() ? nullptr : slot_mapping.data();
  return s;
}

void BatchAssembler::Clear() {
  inputs_.token_ids.clear();
  inputs_.positions.clear();
  inputs_.cu_seqlens.clear();
  inputs_.caches.clear();
  inputs_.query_lens.clear();
  inputs_.context_lens.clear();
  inputs_.table_offsets.clear();
  inputs_.table_ids.clear();
  inputs_.slot_mapping.clear();
}

Status BatchAssembler::Flatten(std::span<const BatchSeqInput> seqs, Mode mode) {
  Clear();
  // Validate every descriptor before growing any cache.
  int64_t total = 0;
  for (size_t b = 0; b < seqs.size(); ++b) {
    const BatchSeqInput& s = seqs[b];
    if (s.cache == nullptr)
      return Error(StatusCode::kInvalidArgument,
                   Format("BatchAssembler: sequence %zu has a null cache", b));
    const int64_t t = static_cast<int64_t>(s.token_ids.size());
    if (t < 1)
      return Error(StatusCode::kInvalidArgument,
                   Format("BatchAssembler: sequence %zu has empty token_ids", b));
    if (mode == Mode::kDecode && t != 1)
      return Error(StatusCode::kInvalidArgument,
                   Format("BatchAssembler: decode sequence %zu must contribute exactly one token "
                          "(got %lld)",
                          b, static_cast<long long>(t)));
    if (s.cache->pool() != seqs[0].cache->pool())
      return Error(StatusCode::kInvalidArgument,
                   Format("BatchAssembler: sequence %zu lives on another block pool", b));
    for (size_t a = 0; a < b; ++a)
      if (seqs[a].cache == s.cache)
        return Error(StatusCode::kInvalidArgument,
                     Format("BatchAssembler: sequences %zu and %zu share one cache", a, b));
    total += t;
  }
  if (total > INT32_MAX)
    return Error(StatusCode::kInvalidArgument, "BatchAssembler: step exceeds 2^31 tokens");

  inputs_.cu_seqlens.push_back(0);
  inputs_.table_offsets.push_back(0);
  for (size_t b = 0; b < seqs.size(); ++b) {
    const BatchSeqInput& s = seqs[b];
    const int64_t t = static_cast<int64_t>(s.token_ids.size());
    const int64_t base = s.cache->length();
    StatusOr<const std::vector<int64_t>*> slots = s.cache->Grow(t);
    if (!slots.ok()) {
      // All-or-nothing over the step: undo the growth of earlier sequences.
      for (size_t a = 0; a < b; ++a)
        (void)inputs_.caches[a]->truncate(inputs_.context_lens[a] - inputs_.query_lens[a]);
      Clear();
      return slots.status();
    }
    for (int64_t i = 0; i < t; ++i) {
      inputs_.token_ids.push_back(s.token_ids[static_cast<size_t>(i)]);
      inputs_.positions.push_back(static_cast<int32_t>(base + i));
    }
    inputs_.slot_mapping.insert(inputs_.slot_mapping.end(), (*slots)->begin(), (*slots)->end());
    inputs_.cu_seqlens.push_back(inputs_.cu_seqlens.back() + static_cast<int32_t>(t));
    inputs_.caches.push_back(s.cache);
    inputs_.query_lens.push_back(static_cast<int32_t>(t));
    inputs_.context_lens.push_back(s.cache->length());
    const std::vector<int32_t>& ids = s.cache->block_table().blocks();
    inputs_.table_ids.insert(inputs_.table_ids.end(), ids.begin(), ids.end());
    inputs_.table_offsets.push_back(static_cast<int32_t>(inputs_.table_ids.size()));
  }
  return Status::Ok();
}

Status BatchAssembler::AssemblePrefill(std::span<const BatchSeqInput> seqs) {
  return Flatten(seqs, Mode::kPrefill);
}

Status BatchAssembler::AssembleDecode(std::span<const BatchSeqInput> seqs) {
  return Flatten(seqs, Mode::kDecode);
}

Status BatchAssembler::AssembleMixed(std::span<const BatchSeqInput> seqs) {
  return Flatten(seqs, Mode::kMixed);
}

size_t BatchAssembler::staging_bytes() const {
  return VectorBytes(inputs_.token_ids) + VectorBytes(inputs_.positions) +
         VectorBytes(inputs_.cu_seqlens) + VectorBytes(inputs_.caches) +
         VectorBytes(inputs_.query_lens) + VectorBytes(inputs_.context_lens) +
         VectorBytes(inputs_.table_offsets) + VectorBytes(inputs_.table_ids) +
         VectorBytes(inputs_.slot_mapping);
}

BatchedAttention::BatchedAttention(ehip_ctx* ctx, const BlockPool* pool, int heads)
    : ctx_(ctx), pool_(pool) {
  const CacheGeometry& g = pool->geometry();
  geom_.heads = heads;
  geom_.kv_heads = g.num_kv_heads;
  geom_.head_dim = g.head_dim;
  geom_.block_size = pool->block_size();
  geom_.kv_dtype = static_cast<int32_t>(g.dtype);
  geom_.slab_blocks = pool->num_blocks();
  geom_.block_stride = pool->block_stride();
  geom_.scale = kernels::AttentionScale(g.head_dim);
}

Status BatchedAttention::Upload(const BatchInputs& in) {
  uploaded_ = false;
  if (!pool_->device_resident())
    return Error(StatusCode::kFailedPrecondition,
                 "BatchedAttention: the pool's slabs are not in HBM");
  for (size_t b = 0; b < in.caches.size(); ++b)
    if (in.caches[b]->pool() != pool_)
      return Error(StatusCode::kInvalidArgument,
                   Format("BatchedAttention: sequence %zu lives on another block pool", b));
  const ehip_step_desc s = in.desc();
  if (Status st = FromRc(ctx_, ehip_step_upload(ctx_, &geom_, &s)); !st.ok()) return st;
  uploaded_ = true;
  has_slots_ = !in.slot_mapping.empty();
  next_layer_ = 0;
  return Status::Ok();
}

Status BatchedAttention::CheckLayer(int layer) const {
  if (!uploaded_)
    return Error(StatusCode::kFailedPrecondition, "BatchedAttention: no step uploaded");
  if (layer != next_layer_)
    return Error(StatusCode::kInvalidArgument,
                 Format("BatchedAttention: expected layer %d next, got %d", next_layer_, layer));
  return Status::Ok();
}

Status BatchedAttention::Attend(int layer, const float* d_q, float* d_out) {
  if (Status s = FromRc(ctx_, ehip_step_attention(ctx_, d_q, pool_->k_slab(layer),
                                                  pool_->v_slab(layer), d_out));
      !s.ok())
    return s;
  next_layer_ = (layer + 1) % pool_->geometry().num_layers;
  return Status::Ok();
}

Status BatchedAttention::ForwardLayer(int layer, const float* d_q, const float* d_k_new,
                                      const float* d_v_new, float* d_out) {
  if (Status s = CheckLayer(layer); !s.ok()) return s;
  if (has_slots_)
    if (Status s = FromRc(ctx_, ehip_step_kv_append(ctx_, d_k_new, d_v_new, pool_->k_slab(layer),
                                                    pool_->v_slab(layer)));
        !s.ok())
      return s;
  return Attend(layer, d_q, d_out);
}

Status BatchedAttention::ForwardLayerRope(int layer, float* d_q, const float* d_k_new,
                                          const float* d_v_new, const RopeTables& rope,
                                          float* d_out) {
  if (Status s = CheckLayer(layer); !s.ok()) return s;
  if (!has_slots_)
    return Error(StatusCode::kFailedPrecondition,
                 "BatchedAttention: RoPE needs the step's slot mapping");
  if (Status s = FromRc(ctx_, ehip_step_rope_kv_append(ctx_, d_q, d_k_new, d_v_new, rope.d_cos,
                                                       rope.d_sin, rope.positions,
                                                       pool_->k_slab(layer),
                                                       pool_->v_slab(layer)));
      !s.ok())
    return s;
  return Attend(layer, d_q, d_out);
}

}  // namespace ehip::host
