// BlockPool: the paged KV cache's block allocator over per-layer K/V slabs.
//
// Same interface and semantics as the reference's kvcache::BlockPool
// (src/kvcache/block_pool.h:62-199, .cpp:28-339): 2·L slabs of
// [num_blocks, Hkv, bs, d], 256-byte aligned and zero-filled; a LIFO free
// list seeded so the first Allocate returns block 0; refcounts with Share /
// Release (sharing a free block or releasing one twice aborts); occupancy
// stats; the capacity arithmetic the engine sizes the pool with. Two
// differences: the slabs may be bf16 (the reference pool is fp32-only,
// block_pool.cpp:41-46; bf16 storage follows its Fp32ToBf16Bits rounding), and
// Create returns a heap-pinned pool (unique_ptr) instead of a move-once value,
// because a BlockTable holds a raw pointer to its pool.
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

// kvcache::BlockPoolStats (block_pool.h:52-60): used + free == total.
struct BlockPoolStats {
  int64_t total = 0;
  int64_t used = 0;
  int64_t free = 0;
  double utilization = 0.0;  // used / total
  int64_t peak_used = 0;     // high-water mark of used since Create
  int64_t exhaustions = 0;   // Allocate() calls that found the free list empty
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

  // Allocates the 2·L slabs from `allocator` (non-null; the pool does not own
  // it and it must outlive the pool). block_size ∈ {8,16,32,64}; num_blocks in
  // [1, 2^31) because block ids are int32.
  static StatusOr<std::unique_ptr<BlockPool>> Create(CacheGeometry geom, int block_size,
                                                     int64_t num_blocks,
                                                     SlabAllocator* allocator);

  BlockPool(const BlockPool&) = delete;
  BlockPool& operator=(const BlockPool&) = delete;
  ~BlockPool();

  // Pops the free list (LIFO), refcount 1. ResourceExhausted when empty.
  StatusOr<int32_t> Allocate();
  // refcount += 1; aborts on an out-of-range or free block.
  void Share(int32_t block);
  // refcount -= 1, 1 -> 0 returns the block to the free list; aborts on an
  // out-of-range or free block (double free).
  void Release(int32_t block);

  int32_t refcount(int32_t block) const;
  BlockPoolStats stats() const;
  int64_t free_blocks() const;
  // ceil((cur+add)/bs) - ceil(cur/bs); aborts on negative arguments.
  int64_t blocks_needed(int64_t cur_tokens, int64_t add_tokens) const;

  // Slab base pointers (device memory for an HBM allocator).
  void* k_slab(int layer) const;
  void* v_slab(int layer) const;
  int64_t block_stride() const { return block_stride_; }  // Hkv·bs·d elements
  int64_t head_stride() const { return head_stride_; }    // bs·d
  int64_t row_stride() const { return row_stride_; }      // d

  const CacheGeometry& geometry() const { return geom_; }
  int block_size() const { return block_size_; }
  int64_t num_blocks() const { return num_blocks_; }
  int64_t slab_bytes() const { return slab_bytes_; }
  int64_t total_bytes() const { return slab_bytes_ * 2 * geom_.num_layers; }
  bool device_resident() const { return allocator_->device(); }

 private:
  BlockPool(CacheGeometry geom, int block_size, int64_t num_blocks, int64_t slab_bytes,
            SlabAllocator* allocator);
  bool in_range(int32_t block) const { return block >= 0 && block < num_blocks_; }

  CacheGeometry geom_;
  int block_size_;
  int64_t num_blocks_;
  int64_t slab_bytes_;
  int64_t block_stride_;
  int64_t head_stride_;
  int64_t row_stride_;
  SlabAllocator* allocator_;
  std::vector<void*> k_slabs_;
  std::vector<void*> v_slabs_;

  mutable std::mutex mu_;
  std::vector<int32_t> refcount_;
  std::vector<int32_t> free_list_;  // top = back
  int64_t used_ = 0;
  int64_t peak_used_ = 0;
  int64_t exhaustions_ = 0;
};

}  // namespace ehip::host
