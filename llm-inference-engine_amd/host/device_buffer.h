// Owning handle for one HBM allocation made through the C ABI.
#pragma once

#include <cstdint>
#include <utility>

#include "ehip.h"
#include "status.h"

namespace ehip::host {

// Converts a C-ABI return code into a Status carrying the context's last error.
Status FromRc(const ehip_ctx* ctx, int rc);

class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  ~DeviceBuffer() { Reset(); }
  DeviceBuffer(DeviceBuffer&& o) noexcept : ctx_(o.ctx_), ptr_(o.ptr_), bytes_(o.bytes_) {
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      Reset();
      ctx_ = o.ctx_;
      ptr_ = std::exchange(o.ptr_, nullptr);
      bytes_ = std::exchange(o.bytes_, 0);
    }
    return *this;
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;

  // Grows (never shrinks) to at least `bytes`; contents are not preserved.
  Status Reserve(ehip_ctx* ctx, int64_t bytes);
  // Reserve + synchronous host-to-device copy.
  Status Upload(ehip_ctx* ctx, const void* src, int64_t bytes);
  void Reset();
  void* get() const { return ptr_; }
  int64_t bytes() const { return bytes_; }

 private:
  ehip_ctx* ctx_ = nullptr;
  void* ptr_ = nullptr;
  int64_t bytes_ = 0;
};

}  // namespace ehip::host
