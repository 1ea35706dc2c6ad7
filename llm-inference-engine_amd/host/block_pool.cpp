#include "block_pool.h"

#include <cstdio>

#include "check.h"

namespace ehip::host {
namespace {

bool ValidBlockSize(int bs) { return bs == 8 || bs == 16 || bs == 32 || bs == 64; }

Status ValidateGeometry(const CacheGeometry& g) {
  if (g.num_layers < 1 || g.num_kv_heads < 1 || g.head_dim < 1)
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockPool: geometry must be positive, got num_layers=%d, "
                        "num_kv_heads=%d, head_dim=%d",
                        g.num_layers, g.num_kv_heads, g.head_dim));
  if (g.dtype != KvDtype::kFloat32 && g.dtype != KvDtype::kBFloat16)
    return Error(StatusCode::kUnimplemented, "BlockPool: K/V slabs are f32 or bf16");
  return Status::Ok();
}

Status MulChecked(int64_t* acc, int64_t f) {
  if (__builtin_mul_overflow(*acc, f, acc))
    return Error(StatusCode::kInvalidArgument, "BlockPool: size overflows int64");
  return Status::Ok();
}

}  // namespace

StatusOr<int64_t> BlockPool::BytesPerBlock(const CacheGeometry& g, int bs) {
  if (Status s = ValidateGeometry(g); !s.ok()) return s;
  if (!ValidBlockSize(bs))
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockPool: block_size must be one of {8, 16, 32, 64}, got %d", bs));
  int64_t bytes = 2;
  for (int64_t f : {int64_t{g.num_layers}, int64_t{g.num_kv_heads}, int64_t{bs},
                    int64_t{g.head_dim}, ItemSize(g.dtype)})
    if (Status s = MulChecked(&bytes, f); !s.ok()) return s;
  return bytes;
}

StatusOr<int64_t> BlockPool::NumBlocksForBudget(const CacheGeometry& g, int bs,
                                                int64_t budget) {
  if (budget <= 0)
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockPool: kv_budget_bytes must be positive, got %lld",
                        static_cast<long long>(budget)));
  StatusOr<int64_t> per = BytesPerBlock(g, bs);
  if (!per.ok()) return per.status();
  const int64_t n = budget / *per;
  if (n < 1)
    return Error(StatusCode::kResourceExhausted,
                 Format("BlockPool: KV budget %lld bytes is below one block (%lld bytes/block)",
                        static_cast<long long>(budget), static_cast<long long>(*per)));
  return n;
}

BlockPool::BlockPool(CacheGeometry geom, int bs, int64_t num_blocks, int64_t slab_bytes,
                     SlabAllocator* allocator)
    : geom_(geom),
      block_size_(bs),
      num_blocks_(num_blocks),
      slab_bytes_(slab_bytes),
      block_stride_(int64_t{geom.num_kv_heads} * bs * geom.head_dim),
      head_stride_(int64_t{bs} * geom.head_dim),
      row_stride_(geom.head_dim),
      allocator_(allocator),
      refcount_(static_cast<size_t>(num_blocks), 0) {
  // Descending, so the top of the stack (the back) is block 0.
  free_list_.reserve(static_cast<size_t>(num_blocks));
  for (int64_t b = num_blocks - 1; b >= 0; --b) free_list_.push_back(static_cast<int32_t>(b));
}

BlockPool::~BlockPool() {
  for (void* p : k_slabs_) allocator_->Free(p);
  for (void* p : v_slabs_) allocator_->Free(p);
}

StatusOr<std::unique_ptr<BlockPool>> BlockPool::Create(CacheGeometry geom, int bs,
                                                       int64_t num_blocks,
                                                       SlabAllocator* allocator) {
  if (Status s = ValidateGeometry(geom); !s.ok()) return s;
  if (!ValidBlockSize(bs))
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockPool::Create: block_size must be one of {8, 16, 32, 64}, got %d",
                        bs));
  if (num_blocks < 1 || num_blocks > INT32_MAX)
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockPool::Create: num_blocks must be in [1, 2^31), got %lld",
                        static_cast<long long>(num_blocks)));
  if (allocator == nullptr)
    return Error(StatusCode::kInvalidArgument, "BlockPool::Create: allocator must not be null");
  int64_t slab_bytes = num_blocks;
  for (int64_t f : {int64_t{geom.num_kv_heads}, int64_t{bs}, int64_t{geom.head_dim},
                    ItemSize(geom.dtype)})
    if (Status s = MulChecked(&slab_bytes, f); !s.ok()) return s;

  std::unique_ptr<BlockPool> pool(new BlockPool(geom, bs, num_blocks, slab_bytes, allocator));
  for (int slab = 0; slab < 2 * geom.num_layers; ++slab) {
    Status st;
    void* p = allocator->Allocate(static_cast<size_t>(slab_bytes), kSlabAlignment, &st);
    if (p == nullptr) return st;  // the pool's destructor frees the slabs taken so far
    (slab % 2 == 0 ? pool->k_slabs_ : pool->v_slabs_).push_back(p);
  }
  std::fprintf(stderr,
               "[ehip] BlockPool: %lld blocks x %d tokens (%lld bytes/block, %lld bytes total, %s) "
               "for %d layers, Hkv=%d, d=%d\n",
               static_cast<long long>(num_blocks), bs,
               static_cast<long long>(pool->total_bytes() / num_blocks),
               static_cast<long long>(pool->total_bytes()), allocator->device() ? "HBM" : "host",
               geom.num_layers, geom.num_kv_heads, geom.head_dim);
  return pool;
}

StatusOr<int32_t> BlockPool::Allocate() {
  std::lock_guard<std::mutex> lock(mu_);
  if (free_list_.empty()) {
    ++exhaustions_;
    return Error(StatusCode::kResourceExhausted,
                 Format("BlockPool::Allocate: no free blocks (%lld of %lld in use)",
                        static_cast<long long>(used_), static_cast<long long>(num_blocks_)));
  }
  const int32_t b = free_list_.back();
  free_list_.pop_back();
  refcount_[static_cast<size_t>(b)] = 1;
  if (++used_ > peak_used_) peak_used_ = used_;
  return b;
}

void BlockPool::Share(int32_t block) {
  std::lock_guard<std::mutex> lock(mu_);
  EHIP_CHECK(in_range(block), "BlockPool::Share: block %d out of range [0, %lld)", block,
             static_cast<long long>(num_blocks_));
  int32_t& rc = refcount_[static_cast<size_t>(block)];
  EHIP_CHECK(rc > 0, "BlockPool::Share: block %d is free (refcount 0)", block);
  ++rc;
}

void BlockPool::Release(int32_t block) {
  std::lock_guard<std::mutex> lock(mu_);
  EHIP_CHECK(in_range(block), "BlockPool::Release: block %d out of range [0, %lld)", block,
             static_cast<long long>(num_blocks_));
  int32_t& rc = refcount_[static_cast<size_t>(block)];
  EHIP_CHECK(rc > 0, "BlockPool::Release: block %d released twice (refcount 0)", block);
  if (--rc == 0) {
    free_list_.push_back(block);
    --used_;
  }
}

int32_t BlockPool::refcount(int32_t block) const {
  std::lock_guard<std::mutex> lock(mu_);
  EHIP_CHECK(in_range(block), "BlockPool::refcount: block %d out of range [0, %lld)", block,
             static_cast<long long>(num_blocks_));
  return refcount_[static_cast<size_t>(block)];
}

BlockPoolStats BlockPool::stats() const {
  std::lock_guard<std::mutex> lock(mu_);
  BlockPoolStats s;
  s.total = num_blocks_;
  s.used = used_;
  s.free = static_cast<int64_t>(free_list_.size());
  s.utilization = num_blocks_ > 0 ? static_cast<double>(used_) / static_cast<double>(num_blocks_)
                                  : 0.0;
  s.peak_used = peak_used_;
  s.exhaustions = exhaustions_;
  s.block_size = block_size_;
  return s;
}

int64_t BlockPool::free_blocks() const {
  std::lock_guard<std::mutex> lock(mu_);
  return static_cast<int64_t>(free_list_.size());
}

int64_t BlockPool::blocks_needed(int64_t cur, int64_t add) const {
  EHIP_CHECK(cur >= 0 && add >= 0, "BlockPool::blocks_needed: negative token count (%lld, %lld)",
             static_cast<long long>(cur), static_cast<long long>(add));
  const int64_t bs = block_size_;
  return (cur + add + bs - 1) / bs - (cur + bs - 1) / bs;
}

void* BlockPool::k_slab(int layer) const {
  EHIP_CHECK(layer >= 0 && layer < geom_.num_layers, "BlockPool::k_slab: layer %d", layer);
  return k_slabs_[static_cast<size_t>(layer)];
}

void* BlockPool::v_slab(int layer) const {
  EHIP_CHECK(layer >= 0 && layer < geom_.num_layers, "BlockPool::v_slab: layer %d", layer);
  return v_slabs_[static_cast<size_t>(layer)];
}

}  // namespace ehip::host
