// BlockPool: the paged KV cache's block allocator over per-layer K/V slabs.
//
// Interface and observable behaviour follow the reference's kvcache::BlockPool
// (src/kvcache/block_pool.h:62-199; semantics in
// docs/design/paged-kv-cache.md): 2·L slabs of [num_blocks, Hkv, bs, d],
// 256-byte aligned and zero-filled; allocation is last-freed-first with the
// first allocation returning block 0; blocks carry reference counts
// (Share/Release; sharing a free block, releasing a free one or naming a
// block outside the pool aborts); occupancy statistics; the capacity
// arithmetic the engine sizes a pool with.
//
// This pool is built for HBM: every slab of every layer lives in one arena
// (one device allocation, slab i at i·slab_stride), and the free blocks form
// an intrusive chain through a per-block link array rather than a separate
// stack. AllocateRun takes several blocks all-or-nothing for a table's
// growth. Slabs may be bf16 (stored with the reference's Fp32ToBf16Bits
// rounding); the reference pool is fp32-only. Create returns the pool on the
// heap (unique_ptr), because tables keep a raw pointer to it.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

#include "slab_allocator.h"
#include "status.h"

namespace ehip::host {

enum class KvDtype : int32_t { kFloat32 = EHIP_KV_F32, kBFloat16 = EHIP_KV_BF16 };

inline int64_t ItemSize(KvDtype t) { return t == KvDtype::kBFloat16 ? 2 : 4; }

// kvcache::CacheGeometry (src/kvcache/kv_cache.h:45-52).
struct CacheGeometry {
  int num_layers = 0;
  int num_kv_heads = 0;  // Hkv
  int head_dim = 0;      // d
  KvDtype dtype = KvDtype::kFloat32;
};

// kvcache::BlockPoolStats (src/kvcache/block_pool.h:52-60): used + free == total.
struct BlockPoolStats {
  int64_t total = 0;
  int64_t used = 0;
  int64_t free = 0;
  double utilization = 0.0;  // used / total
  int64_t peak_used = 0;     // most blocks ever held at once since Create
  int64_t exhaustions = 0;   // allocation requests refused for lack of blocks
  int block_size = 0;
};

class BlockPool {
 public:
  static constexpr std::size_t kSlabAlignment = 256;

  // 2 · L · Hkv · bs · d · itemsize; InvalidArgument on a bad geometry,
  // block size or overflow.
  static StatusOr<int64_t> BytesPerBlock(const CacheGeometry& geom, int block_size);
  // floor(budget / BytesPerBlock); ResourceExhausted below one block,
  // InvalidArgument for a non-positive budget.
  static StatusOr<int64_t> NumBlocksForBudget(const CacheGeometry& geom, int block_size,
                                              int64_t kv_budget_bytes);

  // Takes the slab arena from `allocator` (non-null; not owned, must outlive
  // the pool). block_size in {8, 16, 32, 64}; num_blocks in [1, 2^31) (block
  // ids are int32).
  static StatusOr<std::unique_ptr<BlockPool>> Create(CacheGeometry geom, int block_size,
                                                     int64_t num_blocks,
                                                     SlabAllocator* allocator);

  BlockPool(const BlockPool&) = delete;
  BlockPool& operator=(const BlockPool&) = delete;
  ~BlockPool();

  // One block, refcount 1; ResourceExhausted when none is free.
  StatusOr<int32_t> Allocate();
  // n >= 0 blocks appended to *out (each refcount 1, in the order Allocate
  // would return them), or none at all and ResourceExhausted.
  Status AllocateRun(int64_t n, std::vector<int32_t>* out);
  // refcount + 1; aborts on a block outside the pool or a free block.
  void Share(int32_t block);
  // refcount - 1; at 0 the block becomes the next one handed out. Aborts on a
  // block outside the pool or a free block.
  void Release(int32_t block);

  int32_t refcount(int32_t block) const;
  BlockPoolStats stats() const;
  int64_t free_blocks() const;
  // Blocks a sequence of cur tokens must add to hold add more:
  // ceil((cur + add) / bs) - ceil(cur / bs). Aborts on negative counts.
  int64_t blocks_needed(int64_t cur_tokens, int64_t add_tokens) const;

  // Slab base pointers (device memory for an HBM allocator).
  void* k_slab(int layer) const;
  void* v_slab(int layer) const;
  int64_t block_stride() const { return int64_t{geom_.num_kv_heads} * block_size_ * geom_.head_dim; }
  int64_t head_stride() const { return int64_t{block_size_} * geom_.head_dim; }
  int64_t row_stride() const { return geom_.head_dim; }

  const CacheGeometry& geometry() const { return geom_; }
  int block_size() const { return block_size_; }
  int64_t num_blocks() const { return num_blocks_; }
  int64_t slab_bytes() const { return slab_bytes_; }
  int64_t total_bytes() const { return slab_bytes_ * 2 * geom_.num_layers; }
  bool device_resident() const { return allocator_->device(); }

 private:
  static constexpr int32_t kNoBlock = -1;

  BlockPool(CacheGeometry geom, int block_size, int64_t num_blocks, int64_t slab_bytes,
            SlabAllocator* allocator);
  void* slab(int index) const;
  void CheckHeld(int32_t block, const char* op) const;  // mu_ held
  int32_t PopFree();                                    // mu_ held, chain non-empty
  void PushFree(int32_t block);                         // mu_ held

  const CacheGeometry geom_;
  const int block_size_;
  const int64_t num_blocks_;
  const int64_t slab_bytes_;
  const int64_t slab_stride_;  // slab_bytes_ rounded up to kSlabAlignment
  SlabAllocator* const allocator_;
  void* arena_ = nullptr;

  mutable std::mutex mu_;
  // Per block: holders (0 = free) and, for a free block, the next free block.
  std::vector<int32_t> holders_;
  std::vector<int32_t> next_free_;
  int32_t free_head_ = kNoBlock;
  int64_t free_count_ = 0;
  int64_t high_water_ = 0;
  int64_t refused_ = 0;
};

}  // namespace ehip::host
