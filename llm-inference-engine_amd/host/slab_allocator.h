// Where a BlockPool's per-layer K/V slabs live. The reference takes a
// memory::Allocator (src/memory/allocator.h:66-95; BlockPool::Create,
// src/kvcache/block_pool.h:96-98); here the production allocator hands out
// HBM through the C ABI (ehip_malloc: 256-byte aligned, zero-filled) and a
// host allocator keeps the bookkeeping testable without a GPU.
#pragma once

#include <cstddef>

#include "ehip.h"
#include "status.h"

namespace ehip::host {

class SlabAllocator {
 public:
  virtual ~SlabAllocator() = default;
  // Zero-filled, at least `align`-byte aligned; nullptr plus *status on failure.
  virtual void* Allocate(std::size_t bytes, std::size_t align, Status* status) = 0;
  virtual void Free(void* p) = 0;
  // True when the memory is device (HBM) memory.
  virtual bool device() const = 0;
};

class HostSlabAllocator final : public SlabAllocator {
 public:
  void* Allocate(std::size_t bytes, std::size_t align, Status* status) override;
  void Free(void* p) override;
  bool device() const override { return false; }
};

class HbmSlabAllocator final : public SlabAllocator {
 public:
  explicit HbmSlabAllocator(ehip_ctx* ctx) : ctx_(ctx) {}
  void* Allocate(std::size_t bytes, std::size_t align, Status* status) override;
  void Free(void* p) override;
  bool device() const override { return true; }

 private:
  ehip_ctx* ctx_;
};

}  // namespace ehip::host
