// BlockTable: one sequence's logical -> physical block map over a BlockPool.
//
// Behaviour of the reference's kvcache::BlockTable (src/kvcache/block_table.h:
// 41-106): growing by `count` tokens is all-or-nothing and yields the new
// positions' slots, slot(pos) = ids[pos / bs] * bs + pos % bs; truncation keeps
// a partial tail block and gives back the wholly emptied blocks, last one
// first; destruction gives back every block. blocks() is the contiguous int32
// id array the attention kernels read.
//
// Prefix sharing (the pool's Share): ForkFrom adopts the leading full blocks
// of another table. An adopted block is never written again here, because a
// table only ever writes past its last full block; a truncation that would
// leave a shared block as the partial (writable) tail is refused, since
// copy-on-write is deferred (src/kvcache/block_table.h:76).
#pragma once

#include <cstdint>
#include <vector>

#include "block_pool.h"
#include "status.h"

namespace ehip::host {

class BlockTable {
 public:
  explicit BlockTable(BlockPool* pool);  // pool non-null, outlives the table
  ~BlockTable();
  BlockTable(BlockTable&& other) noexcept;
  BlockTable& operator=(BlockTable&&) = delete;
  BlockTable(const BlockTable&) = delete;
  BlockTable& operator=(const BlockTable&) = delete;

  // Slots of `count` new positions; count < 1 -> InvalidArgument; not enough
  // free blocks -> ResourceExhausted, with table and pool unchanged.
  StatusOr<std::vector<int64_t>> AppendTokens(int64_t count);
  // Shortens the sequence to new_len in [0, num_tokens] (InvalidArgument
  // otherwise; FailedPrecondition if a shared block would become the tail).
  Status Truncate(int64_t new_len);
  void FreeAll();
  // Slot of position pos; aborts unless 0 <= pos < num_tokens.
  int64_t slot(int64_t pos) const;

  // Adopts the first `tokens` positions of `other` (whole blocks only) by
  // sharing their blocks. This table must be empty (FailedPrecondition) and
  // on the same pool; tokens must be a run of full blocks of `other`
  // (InvalidArgument).
  Status ForkFrom(const BlockTable& other, int64_t tokens);

  int64_t num_tokens() const { return tokens_; }
  int64_t num_blocks() const { return static_cast<int64_t>(ids_.size()); }
  const std::vector<int32_t>& blocks() const { return ids_; }
  int block_size() const { return pool_->block_size(); }
  BlockPool* pool() const { return pool_; }

 private:
  int64_t SlotOf(int64_t pos) const {
    const int64_t bs = pool_->block_size();
    return int64_t{ids_[static_cast<size_t>(pos / bs)]} * bs + pos % bs;
  }
  // Gives back ids_[keep..] to the pool, last block first.
  void DropBlocksFrom(int64_t keep);

  BlockPool* pool_;
  std::vector<int32_t> ids_;
  int64_t tokens_ = 0;
};

}  // namespace ehip::host
