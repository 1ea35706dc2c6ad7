#include "block_table.h"

#include <utility>

#include "check.h"

namespace ehip::host {

BlockTable::BlockTable(BlockPool* pool) : pool_(pool) {
  EHIP_CHECK(pool_ != nullptr, "BlockTable: pool must not be null");
}

BlockTable::~BlockTable() { FreeAll(); }

BlockTable::BlockTable(BlockTable&& other) noexcept
    : pool_(other.pool_), blocks_(std::move(other.blocks_)), num_tokens_(other.num_tokens_) {
  other.blocks_.clear();
  other.num_tokens_ = 0;
}

StatusOr<std::vector<int64_t>> BlockTable::AppendTokens(int64_t count) {
  if (count <= 0)
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockTable::AppendTokens: count must be positive, got %lld",
                        static_cast<long long>(count)));
  const int64_t bs = pool_->block_size();
  const int64_t need = pool_->blocks_needed(num_tokens_, count);
  std::vector<int32_t> fresh;
  fresh.reserve(static_cast<size_t>(need));
  while (static_cast<int64_t>(fresh.size()) < need) {
    StatusOr<int32_t> b = pool_->Allocate();
    if (!b.ok()) {
      for (int32_t taken : fresh) pool_->Release(taken);
      return Error(StatusCode::kResourceExhausted,
                   Format("BlockTable::AppendTokens: pool exhausted growing %lld tokens by %lld "
                          "(needed %lld new blocks, %lld free)",
                          static_cast<long long>(num_tokens_), static_cast<long long>(count),
                          static_cast<long long>(need),
                          static_cast<long long>(pool_->free_blocks())));
    }
    fresh.push_back(*b);
  }
  blocks_.insert(blocks_.end(), fresh.begin(), fresh.end());
  std::vector<int64_t> slots(static_cast<size_t>(count));
  for (int64_t i = 0; i < count; ++i) {
    const int64_t pos = num_tokens_ + i;
    slots[static_cast<size_t>(i)] = int64_t{blocks_[static_cast<size_t>(pos / bs)]} * bs + pos % bs;
  }
  num_tokens_ += count;
  return slots;
}

Status BlockTable::Truncate(int64_t new_len) {
  if (new_len < 0 || new_len > num_tokens_)
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockTable::Truncate: new_len %lld out of range [0, %lld]",
                        static_cast<long long>(new_len), static_cast<long long>(num_tokens_)));
  const int64_t bs = pool_->block_size();
  const int64_t keep = (new_len + bs - 1) / bs;
  // A kept partial tail block is written by the next append; a shared one
  // would need copy-on-write, which this table does not do.
  if (new_len % bs != 0 && pool_->refcount(blocks_[static_cast<size_t>(keep - 1)]) > 1)
    return Error(StatusCode::kFailedPrecondition,
                 Format("BlockTable::Truncate: new_len %lld leaves shared block %d as a partial "
                        "tail (copy-on-write is not supported)",
                        static_cast<long long>(new_len), blocks_[static_cast<size_t>(keep - 1)]));
  while (num_blocks() > keep) {
    pool_->Release(blocks_.back());
    blocks_.pop_back();
  }
  num_tokens_ = new_len;
  return Status::Ok();
}

void BlockTable::FreeAll() {
  for (int32_t b : blocks_) pool_->Release(b);
  blocks_.clear();
  num_tokens_ = 0;
}

int64_t BlockTable::slot(int64_t pos) const {
  EHIP_CHECK(pos >= 0 && pos < num_tokens_, "BlockTable::slot: pos %lld out of range [0, %lld)",
             static_cast<long long>(pos), static_cast<long long>(num_tokens_));
  const int64_t bs = pool_->block_size();
  return int64_t{blocks_[static_cast<size_t>(pos / bs)]} * bs + pos % bs;
}

Status BlockTable::ForkFrom(const BlockTable& other, int64_t tokens) {
  if (other.pool_ != pool_)
    return Error(StatusCode::kInvalidArgument, "BlockTable::ForkFrom: tables on different pools");
  if (num_tokens_ != 0 || !blocks_.empty())
    return Error(StatusCode::kFailedPrecondition, "BlockTable::ForkFrom: table is not empty");
  const int64_t bs = pool_->block_size();
  if (tokens < 0 || tokens % bs != 0 || tokens > other.num_tokens_ ||
      tokens / bs > other.num_blocks())
    return Error(StatusCode::kInvalidArgument,
                 Format("BlockTable::ForkFrom: %lld tokens is not a run of full blocks of the "
                        "source (%lld tokens, bs %lld)",
                        static_cast<long long>(tokens), static_cast<long long>(other.num_tokens_),
                        static_cast<long long>(bs)));
  const int64_t n = tokens / bs;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t b = other.blocks_[static_cast<size_t>(i)];
    pool_->Share(b);
    blocks_.push_back(b);
  }
  num_tokens_ = tokens;
  return Status::Ok();
}

}  // namespace ehip::host
