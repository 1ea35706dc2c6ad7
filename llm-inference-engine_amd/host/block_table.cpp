#include "block_table.h"

#include <utility>

#include "check.h"

namespace ehip::host {

BlockTable::BlockTable(BlockPool* pool) : pool_(pool) {
  EHIP_CHECK(pool_ != nullptr, "a block table needs a pool");
}

BlockTable::~BlockTable() { FreeAll(); }

BlockTable::BlockTable(BlockTable&& other) noexcept
    : pool_(other.pool_), ids_(std::exchange(other.ids_, {})),
      tokens_(std::exchange(other.tokens_, 0)) {}

StatusOr<std::vector<int64_t>> BlockTable::AppendTokens(int64_t count) {
  if (count < 1)
    return Error(StatusCode::kInvalidArgument,
                 Format("a table grows by at least one token (asked for %lld)",
                        static_cast<long long>(count)));
  // The pool hands out every block the growth needs, or none.
  if (Status s = pool_->AllocateRun(pool_->blocks_needed(tokens_, count), &ids_); !s.ok())
    return s;
  std::vector<int64_t> slots(static_cast<size_t>(count));
  for (int64_t i = 0; i < count; ++i) slots[static_cast<size_t>(i)] = SlotOf(tokens_ + i);
  tokens_ += count;
  return slots;
}

void BlockTable::DropBlocksFrom(int64_t keep) {
  for (int64_t i = num_blocks() - 1; i >= keep; --i) pool_->Release(ids_[static_cast<size_t>(i)]);
  ids_.resize(static_cast<size_t>(keep));
}

Status BlockTable::Truncate(int64_t new_len) {
  if (new_len < 0 || new_len > tokens_)
    return Error(StatusCode::kInvalidArgument,
                 Format("cannot truncate a %lld-token table to %lld tokens",
                        static_cast<long long>(tokens_), static_cast<long long>(new_len)));
  const int64_t bs = pool_->block_size();
  const int64_t keep = (new_len + bs - 1) / bs;
  const bool partial_tail = new_len % bs != 0;
  if (partial_tail) {
    const int32_t tail = ids_[static_cast<size_t>(keep - 1)];
    if (pool_->refcount(tail) > 1)
      return Error(StatusCode::kFailedPrecondition,
                   Format("truncating to %lld tokens would make shared block %d writable; "
                          "shared blocks are copied on write by nobody here",
                          static_cast<long long>(new_len), tail));
  }
  DropBlocksFrom(keep);
  tokens_ = new_len;
  return Status::Ok();
}

void BlockTable::FreeAll() {
  // Front to back, so the pool hands the last block out first again.
  for (int32_t id : ids_) pool_->Release(id);
  ids_.clear();
  tokens_ = 0;
}

int64_t BlockTable::slot(int64_t pos) const {
  EHIP_CHECK(pos >= 0 && pos < tokens_, "slot: position %lld is not in a %lld-token table",
             static_cast<long long>(pos), static_cast<long long>(tokens_));
  return SlotOf(pos);
}

Status BlockTable::ForkFrom(const BlockTable& other, int64_t tokens) {
  if (other.pool_ != pool_)
    return Error(StatusCode::kInvalidArgument, "a fork must stay on its parent's pool");
  if (tokens_ != 0 || !ids_.empty())
    return Error(StatusCode::kFailedPrecondition, "only an empty table can fork a prefix");
  const int64_t bs = pool_->block_size();
  if (tokens < 0 || tokens % bs != 0 || tokens > other.tokens_)
    return Error(StatusCode::kInvalidArgument,
                 Format("a forked prefix is whole blocks of the parent: %lld tokens of a "
                        "%lld-token parent with %lld-token blocks",
                        static_cast<long long>(tokens), static_cast<long long>(other.tokens_),
                        static_cast<long long>(bs)));
  ids_.assign(other.ids_.begin(), other.ids_.begin() + tokens / bs);
  for (int32_t id : ids_) pool_->Share(id);
  tokens_ = tokens;
  return Status::Ok();
}

}  // namespace ehip::host
