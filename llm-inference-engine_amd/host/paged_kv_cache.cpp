#include "paged_kv_cache.h"

#include <utility>

#include "check.h"
#include "kernels.h"

namespace ehip::host {

PagedKvCache::PagedKvCache(BlockPool* pool, ehip_ctx* ctx) : pool_(pool), ctx_(ctx), table_(pool) {
  EHIP_CHECK(pool_ != nullptr, "a paged cache needs a pool");
}

int64_t PagedKvCache::capacity() const {
  return (table_.num_blocks() + pool_->free_blocks()) * pool_->block_size();
}

Status PagedKvCache::RequireDevice(const char* what) const {
  if (pool_->device_resident() && ctx_ != nullptr) return Status::Ok();
  return Error(StatusCode::kFailedPrecondition,
               Format("%s runs on the device: the pool must be in HBM and a context given", what));
}

Status PagedKvCache::append(int layer, const float* d_k, const float* d_v, int64_t t_dim) {
  const CacheGeometry& g = pool_->geometry();
  if (!layer_in_range(layer))
    return Error(StatusCode::kInvalidArgument,
                 Format("append: the cache has layers 0..%d, not %d", g.num_layers - 1, layer));
  if (d_k == nullptr || d_v == nullptr || t_dim < 1)
    return Error(StatusCode::kInvalidArgument,
                 Format("append: needs K and V rows of at least one token (T=%lld)",
                        static_cast<long long>(t_dim)));
  if (Status s = RequireDevice("append"); !s.ok()) return s;
  if (layer != fwd_.layers_written)
    return Error(StatusCode::kInvalidArgument,
                 Format("append: layer %d arrived while this forward expects layer %d (each "
                        "forward writes layers 0, 1, ... once each)",
                        layer, fwd_.layers_written));
  if (layer == 0) {
    // A new forward: grow the table (all-or-nothing) and publish its slots.
    StatusOr<std::vector<int64_t>> grown = table_.AppendTokens(t_dim);
    if (!grown.ok()) {
      fwd_ = Forward{};
      return grown.status();
    }
    fwd_.slots = std::move(*grown);
    table_dirty_ = true;
    if (Status s = d_slots_.Upload(ctx_, fwd_.slots.data(),
                                   t_dim * static_cast<int64_t>(sizeof(int64_t)));
        !s.ok())
      return s;
  } else if (t_dim != static_cast<int64_t>(fwd_.slots.size())) {
    return Error(StatusCode::kInvalidArgument,
                 Format("append: layer %d brings %lld tokens but this forward appends %zu",
                        layer, static_cast<long long>(t_dim), fwd_.slots.size()));
  }
  const auto* slots = static_cast<const int64_t*>(d_slots_.get());
  const int bs = pool_->block_size();
  Status s = g.dtype == KvDtype::kBFloat16
                 ? kernels::KvScatterBf16(ctx_, d_k, d_v, slots, t_dim, g.num_kv_heads, g.head_dim,
                                          bs, pool_->num_blocks(),
                                          static_cast<uint16_t*>(pool_->k_slab(layer)),
                                          static_cast<uint16_t*>(pool_->v_slab(layer)))
                 : kernels::KvScatterF32(ctx_, d_k, d_v, slots, t_dim, g.num_kv_heads, g.head_dim,
                                         bs, pool_->num_blocks(),
                                         static_cast<float*>(pool_->k_slab(layer)),
                                         static_cast<float*>(pool_->v_slab(layer)));
  if (!s.ok()) return s;
  if (++fwd_.layers_written == g.num_layers) fwd_.layers_written = 0;  // forward complete
  return Status::Ok();
}

int64_t PagedKvCache::visible_length(int layer) const {
  const bool pending = fwd_.layers_written > 0 && layer >= fwd_.layers_written;
  return table_.num_tokens() - (pending ? static_cast<int64_t>(fwd_.slots.size()) : 0);
}

Status PagedKvCache::SyncDeviceTable() const {
  if (!table_dirty_) return Status::Ok();
  const std::vector<int32_t>& ids = table_.blocks();
  const int64_t bytes = static_cast<int64_t>(ids.size() * sizeof(int32_t));
  if (Status s = d_table_.Reserve(ctx_, bytes > 0 ? bytes : 4); !s.ok()) return s;
  if (bytes > 0)
    if (Status s = FromRc(ctx_, ehip_copy_to_device(ctx_, d_table_.get(), ids.data(), bytes));
        !s.ok())
      return s;
  table_dirty_ = false;
  return Status::Ok();
}

Status PagedKvCache::view(int layer, float* d_out_k, float* d_out_v) const {
  if (!layer_in_range(layer))
    return Error(StatusCode::kInvalidArgument, Format("view: no layer %d", layer));
  if (Status s = RequireDevice("view"); !s.ok()) return s;
  const CacheGeometry& g = pool_->geometry();
  if (g.dtype != KvDtype::kFloat32)
    return Error(StatusCode::kUnimplemented, "view: the contiguous gather reads f32 slabs");
  const int64_t len = visible_length(layer);
  if (len == 0) return Status::Ok();
  if (Status s = SyncDeviceTable(); !s.ok()) return s;
  return kernels::KvGatherF32(ctx_, static_cast<const float*>(pool_->k_slab(layer)),
                              static_cast<const float*>(pool_->v_slab(layer)),
                              static_cast<const int32_t*>(d_table_.get()), pool_->block_size(),
                              len, g.num_kv_heads, g.head_dim, pool_->num_blocks(), d_out_k,
                              d_out_v);
}

StatusOr<PagedKvView> PagedKvCache::paged_view(int layer) const {
  if (!layer_in_range(layer))
    return Error(StatusCode::kInvalidArgument, Format("paged_view: no layer %d", layer));
  PagedKvView v;
  if (pool_->device_resident() && ctx_ != nullptr) {
    if (Status s = SyncDeviceTable(); !s.ok()) return s;
    v.d_block_table = static_cast<const int32_t*>(d_table_.get());
  }
  v.k_slab = pool_->k_slab(layer);
  v.v_slab = pool_->v_slab(layer);
  v.block_table = table_.blocks().data();
  v.num_blocks = table_.num_blocks();
  v.block_size = pool_->block_size();
  v.length = table_.num_tokens();
  v.block_stride = pool_->block_stride();
  v.slab_blocks = pool_->num_blocks();
  v.dtype = pool_->geometry().dtype;
  return v;
}

Status PagedKvCache::truncate(int64_t new_length) {
  if (Status s = table_.Truncate(new_length); !s.ok()) return s;
  fwd_ = Forward{};
  table_dirty_ = true;
  return Status::Ok();
}

StatusOr<const std::vector<int64_t>*> PagedKvCache::Grow(int64_t t_dim) {
  if (fwd_.layers_written != 0)
    return Error(StatusCode::kFailedPrecondition,
                 Format("Grow: a layer-by-layer forward is open (%d layers written)",
                        fwd_.layers_written));
  StatusOr<std::vector<int64_t>> grown = table_.AppendTokens(t_dim);
  if (!grown.ok()) return grown.status();
  fwd_.slots = std::move(*grown);
  table_dirty_ = true;
  return &fwd_.slots;
}

Status PagedKvCache::ForkFrom(const PagedKvCache& parent, int64_t tokens) {
  if (Status s = table_.ForkFrom(parent.table_, tokens); !s.ok()) return s;
  table_dirty_ = true;
  return Status::Ok();
}

}  // namespace ehip::host
