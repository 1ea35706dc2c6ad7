// PagedKvCache: one sequence's KV cache over a device-resident BlockPool.
//
// The per-forward layer protocol of the reference's kvcache::PagedKvCache
// (src/kvcache/paged_cache.h:47-129): a forward appends its T new tokens to
// every layer, in layer order, once per layer. The first layer's append grows
// the block table by T tokens; the later layers write the same slots. Until a
// layer has been written in the current forward, it does not see the new
// tokens (visible_length). paged_view(layer) exposes the slab pointers, the
// table, its length and the block stride; view(layer) gathers a contiguous
// [Hkv, len, d] copy.
//
// K/V rows arrive as device pointers ([T, Hkv, d] fp32, token-major) and are
// written by the device scatter kernel; bf16 slabs store RNE-narrowed bits.
// The batched step path (BatchAssembler) grows every sequence of a step once
// through Grow(), and the step's own append kernel writes all layers.
#pragma once

#include <cstdint>
#include <vector>

#include "block_pool.h"
#include "block_table.h"
#include "device_buffer.h"
#include "ehip.h"
#include "status.h"

namespace ehip::host {

// kvcache::PagedKvView (src/kvcache/kv_cache.h:72-80) plus the device copy of
// the table, the slab dtype and the slab's block count.
struct PagedKvView {
  const void* k_slab = nullptr;
  const void* v_slab = nullptr;
  const int32_t* block_table = nullptr;    // host ids, logical order
  const int32_t* d_block_table = nullptr;  // the same ids in HBM
  int64_t num_blocks = 0;
  int block_size = 0;
  int64_t length = 0;
  int64_t block_stride = 0;  // elements per block id
  int64_t slab_blocks = 0;
  KvDtype dtype = KvDtype::kFloat32;
};

class PagedKvCache {
 public:
  // `pool` must outlive the cache; `ctx` may be null only for bookkeeping on a
  // host pool (no append/view/paged_view device work).
  PagedKvCache(BlockPool* pool, ehip_ctx* ctx);
  PagedKvCache(PagedKvCache&&) noexcept = default;
  PagedKvCache(const PagedKvCache&) = delete;
  PagedKvCache& operator=(const PagedKvCache&) = delete;

  CacheGeometry geometry() const { return pool_->geometry(); }
  int64_t length() const { return table_.num_tokens(); }
  // Tokens this sequence could hold: its blocks plus every free block.
  int64_t capacity() const;

  // d_k, d_v: device [t_dim, Hkv, d] fp32. Errors: layer out of range or out
  // of order, t_dim < 1 or different from layer 0's, null rows, host-resident
  // pool (FailedPrecondition), pool exhaustion at layer 0 (ResourceExhausted,
  // nothing grown).
  Status append(int layer, const float* d_k, const float* d_v, int64_t t_dim);
  // Contiguous fp32 [Hkv, visible_length(layer), d] into device buffers.
  Status view(int layer, float* d_out_k, float* d_out_v) const;
  int64_t visible_length(int layer) const;
  StatusOr<PagedKvView> paged_view(int layer) const;
  Status truncate(int64_t new_length);
  void reset() { (void)truncate(0); }

  // Step path: layer-0 growth of one forward without writing any slab.
  // Returns the new tokens' slots (valid until the next Grow/append).
  StatusOr<const std::vector<int64_t>*> Grow(int64_t t_dim);
  // Prefix sharing: adopt the leading `tokens` (whole blocks) of `parent`.
  Status ForkFrom(const PagedKvCache& parent, int64_t tokens);

  const BlockTable& block_table() const { return table_; }
  BlockPool* pool() const { return pool_; }

 private:
  int num_layers() const { return pool_->geometry().num_layers; }
  bool layer_in_range(int layer) const { return layer >= 0 && layer < num_layers(); }
  Status RequireDevice(const char* what) const;
  Status SyncDeviceTable() const;
  // The forward in progress: the slots its layer-0 append took, and how many
  // layers (from layer 0 up) it has written. layers_written == 0: no forward
  // is open (a finished forward closes itself).
  struct Forward {
    std::vector<int64_t> slots;
    int layers_written = 0;
  };

  BlockPool* pool_;
  ehip_ctx* ctx_;
  BlockTable table_;
  Forward fwd_;
  DeviceBuffer d_slots_;
  mutable DeviceBuffer d_table_;
  mutable bool table_dirty_ = true;
};

}  // namespace ehip::host
