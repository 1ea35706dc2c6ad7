// BlockTable: one sequence's logical -> physical block map over a BlockPool.
//
// Semantics of the reference's kvcache::BlockTable (src/kvcache/block_table.h:
// 41-106, .cpp:28-103): AppendTokens(count) is all-or-nothing and returns the
// slot mapping of the new positions, slot(pos) = blocks[pos/bs]·bs + pos%bs;
// Truncate keeps the partial tail block and releases wholly emptied blocks
// tail-first; FreeAll releases every block (RAII). blocks() is the
// contiguous int32 id array the attention kernels read.
//
// For prefix sharing (the reference's BlockPool::Share, block_pool.cpp:256-266)
// ForkFrom adopts the leading full blocks of another table: each adopted block
// is Share()d, and shared blocks are never written again, because appends only
// ever write past the last full block.
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

  // Grows the sequence by `count` tokens; returns their slots. count <= 0 ->
  // InvalidArgument; pool exhaustion -> ResourceExhausted with table and pool
  // unchanged.
  StatusOr<std::vector<int64_t>> AppendTokens(int64_t count);
  // Drops tokens past new_len in [0, num_tokens]; InvalidArgument otherwise.
  Status Truncate(int64_t new_len);
  void FreeAll();
  // Slot of committed position pos (aborts outside [0, num_tokens)).
  int64_t slot(int64_t pos) const;

  // Adopts the first `tokens` tokens of `other` (a whole number of full
  // blocks) by sharing their blocks; this table must be empty and on the same
  // pool. InvalidArgument / FailedPrecondition otherwise.
  Status ForkFrom(const BlockTable& other, int64_t tokens);

  int64_t num_tokens() const { return num_tokens_; }
  int64_t num_blocks() const { return static_cast<int64_t>(blocks_.size()); }
  const std::vector<int32_t>& blocks() const { return blocks_; }
  int block_size() const { return pool_->block_size(); }
  BlockPool* pool() const { return pool_; }

 private:
  BlockPool* pool_;
  std::vector<int32_t> blocks_;
  int64_t num_tokens_ = 0;
};

}  // namespace ehip::host
