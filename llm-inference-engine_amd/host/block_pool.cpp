#include "block_pool.h"

#include "check.h"

namespace ehip::host {
namespace {

bool ValidBlockSize(int bs) { return bs == 8 || bs == 16 || bs == 32 || bs == 64; }

Status CheckGeometry(const CacheGeometry& g, int bs) {
  if (g.num_layers < 1 || g.num_kv_heads < 1 || g.head_dim < 1)
    return Error(StatusCode::kInvalidArgument,
                 Format("KV geometry needs layers, kv heads and head_dim >= 1 "
                        "(have %d / %d / %d)",
                        g.num_layers, g.num_kv_heads, g.head_dim));
  if (g.dtype != KvDtype::kFloat32 && g.dtype != KvDtype::kBFloat16)
    return Error(StatusCode::kUnimplemented, "KV slabs hold f32 or bf16 elements only");
  if (!ValidBlockSize(bs))
    return Error(StatusCode::kInvalidArgument,
                 Format("tokens per block must be 8, 16, 32 or 64 (have %d)", bs));
  return Status::Ok();
}

// Product of the factors, or InvalidArgument when it leaves int64.
StatusOr<int64_t> Product(std::initializer_list<int64_t> factors) {
  int64_t p = 1;
  for (int64_t f : factors)
    if (__builtin_mul_overflow(p, f, &p))
      return Error(StatusCode::kInvalidArgument, "KV pool size does not fit in 64 bits");
  return p;
}

int64_t RoundUp(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

StatusOr<int64_t> BlockPool::BytesPerBlock(const CacheGeometry& g, int bs) {
  if (Status s = CheckGeometry(g, bs); !s.ok()) return s;
  return Product({2, g.num_layers, g.num_kv_heads, bs, g.head_dim, ItemSize(g.dtype)});
}

StatusOr<int64_t> BlockPool::NumBlocksForBudget(const CacheGeometry& g, int bs,
                                                int64_t budget) {
  if (budget <= 0)
    return Error(StatusCode::kInvalidArgument,
                 Format("a KV byte budget must be positive (have %lld)",
                        static_cast<long long>(budget)));
  StatusOr<int64_t> per_block = BytesPerBlock(g, bs);
  if (!per_block.ok()) return per_block.status();
  if (budget < *per_block)
    return Error(StatusCode::kResourceExhausted,
                 Format("%lld bytes cannot hold a single %lld-byte block (all layers, K and V)",
                        static_cast<long long>(budget), static_cast<long long>(*per_block)));
  return budget / *per_block;
}

BlockPool::BlockPool(CacheGeometry geom, int bs, int64_t num_blocks, int64_t slab_bytes,
                     SlabAllocator* allocator)
    : geom_(geom),
      block_size_(bs),
      num_blocks_(num_blocks),
      slab_bytes_(slab_bytes),
      slab_stride_(RoundUp(slab_bytes, static_cast<int64_t>(kSlabAlignment))),
      allocator_(allocator),
      holders_(static_cast<size_t>(num_blocks), 0),
      next_free_(static_cast<size_t>(num_blocks)) {
  // Chain every block in ascending order: block 0 is handed out first.
  for (int64_t b = 0; b < num_blocks; ++b)
    next_free_[static_cast<size_t>(b)] = b + 1 < num_blocks ? static_cast<int32_t>(b + 1) : kNoBlock;
  free_head_ = 0;
  free_count_ = num_blocks;
}

BlockPool::~BlockPool() {
  if (arena_) allocator_->Free(arena_);
}

StatusOr<std::unique_ptr<BlockPool>> BlockPool::Create(CacheGeometry geom, int bs,
                                                       int64_t num_blocks,
                                                       SlabAllocator* allocator) {
  if (Status s = CheckGeometry(geom, bs); !s.ok()) return s;
  if (num_blocks < 1 || num_blocks > INT32_MAX)
    return Error(StatusCode::kInvalidArgument,
                 Format("a pool holds between 1 and 2^31 - 1 blocks (asked for %lld)",
                        static_cast<long long>(num_blocks)));
  if (allocator == nullptr)
    return Error(StatusCode::kInvalidArgument, "a pool needs a slab allocator");
  StatusOr<int64_t> slab =
      Product({num_blocks, geom.num_kv_heads, bs, geom.head_dim, ItemSize(geom.dtype)});
  if (!slab.ok()) return slab.status();
  std::unique_ptr<BlockPool> pool(new BlockPool(geom, bs, num_blocks, *slab, allocator));
  StatusOr<int64_t> arena = Product({pool->slab_stride_, 2, geom.num_layers});
  if (!arena.ok()) return arena.status();
  Status st;
  pool->arena_ = allocator->Allocate(static_cast<size_t>(*arena), kSlabAlignment, &st);
  if (pool->arena_ == nullptr) return st;
  return pool;
}

void BlockPool::CheckHeld(int32_t block, const char* op) const {
  EHIP_CHECK(block >= 0 && block < num_blocks_, "%s: no block %d in a pool of %lld", op, block,
             static_cast<long long>(num_blocks_));
  EHIP_CHECK(holders_[static_cast<size_t>(block)] > 0, "%s: block %d has no holder", op, block);
}

int32_t BlockPool::PopFree() {
  const int32_t b = free_head_;
  free_head_ = next_free_[static_cast<size_t>(b)];
  --free_count_;
  holders_[static_cast<size_t>(b)] = 1;
  const int64_t used = num_blocks_ - free_count_;
  if (used > high_water_) high_water_ = used;
  return b;
}

void BlockPool::PushFree(int32_t block) {
  next_free_[static_cast<size_t>(block)] = free_head_;
  free_head_ = block;
  ++free_count_;
}

StatusOr<int32_t> BlockPool::Allocate() {
  std::lock_guard<std::mutex> lock(mu_);
  if (free_count_ == 0) {
    ++refused_;
    return Error(StatusCode::kResourceExhausted,
                 Format("KV pool is full: all %lld blocks are held",
                        static_cast<long long>(num_blocks_)));
  }
  return PopFree();
}

Status BlockPool::AllocateRun(int64_t n, std::vector<int32_t>* out) {
  EHIP_CHECK(n >= 0 && out != nullptr, "AllocateRun: bad request (n=%lld)",
             static_cast<long long>(n));
  std::lock_guard<std::mutex> lock(mu_);
  if (n > free_count_) {
    ++refused_;
    return Error(StatusCode::kResourceExhausted,
                 Format("KV pool cannot supply %lld blocks: %lld of %lld are free",
                        static_cast<long long>(n), static_cast<long long>(free_count_),
                        static_cast<long long>(num_blocks_)));
  }
  out->reserve(out->size() + static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) out->push_back(PopFree());
  return Status::Ok();
}

void BlockPool::Share(int32_t block) {
  std::lock_guard<std::mutex> lock(mu_);
  CheckHeld(block, "Share");
  ++holders_[static_cast<size_t>(block)];
}

void BlockPool::Release(int32_t block) {
  std::lock_guard<std::mutex> lock(mu_);
  CheckHeld(block, "Release");
  if (--holders_[static_cast<size_t>(block)] == 0) PushFree(block);
}

int32_t BlockPool::refcount(int32_t block) const {
  std::lock_guard<std::mutex> lock(mu_);
  EHIP_CHECK(block >= 0 && block < num_blocks_, "refcount: no block %d in a pool of %lld", block,
             static_cast<long long>(num_blocks_));
  return holders_[static_cast<size_t>(block)];
}

BlockPoolStats BlockPool::stats() const {
  std::lock_guard<std::mutex> lock(mu_);
  BlockPoolStats s;
  s.total = num_blocks_;
  s.free = free_count_;
  s.used = num_blocks_ - free_count_;
  s.utilization = static_cast<double>(s.used) / static_cast<double>(num_blocks_);
  s.peak_used = high_water_;
  s.exhaustions = refused_;
  s.block_size = block_size_;
  return s;
}

int64_t BlockPool::free_blocks() const {
  std::lock_guard<std::mutex> lock(mu_);
  return free_count_;
}

int64_t BlockPool::blocks_needed(int64_t cur, int64_t add) const {
  EHIP_CHECK(cur >= 0 && add >= 0, "blocks_needed: token counts must be >= 0 (%lld, %lld)",
             static_cast<long long>(cur), static_cast<long long>(add));
  const auto blocks_for = [this](int64_t tokens) { return (tokens + block_size_ - 1) / block_size_; };
  return blocks_for(cur + add) - blocks_for(cur);
}

void* BlockPool::slab(int index) const {
  return static_cast<char*>(arena_) + static_cast<int64_t>(index) * slab_stride_;
}

void* BlockPool::k_slab(int layer) const {
  EHIP_CHECK(layer >= 0 && layer < geom_.num_layers, "k_slab: no layer %d", layer);
  return slab(2 * layer);
}

void* BlockPool::v_slab(int layer) const {
  EHIP_CHECK(layer >= 0 && layer < geom_.num_layers, "v_slab: no layer %d", layer);
  return slab(2 * layer + 1);
}

}  // namespace ehip::host
