#include "device_buffer.h"

namespace ehip::host {

Status FromRc(const ehip_ctx* ctx, int rc) {
  if (rc == EHIP_OK) return Status::Ok();
  char msg[512] = {0};
  if (ctx != nullptr) ehip_last_error(ctx, msg, sizeof msg);
  return Error(static_cast<StatusCode>(rc), msg);
}

Status DeviceBuffer::Reserve(ehip_ctx* ctx, int64_t bytes) {
  if (ptr_ != nullptr && ctx == ctx_ && bytes <= bytes_) return Status::Ok();
  Reset();
  const int64_t n = bytes < 256 ? 256 : bytes + bytes / 2;  // headroom against regrowth
  void* p = nullptr;
  if (Status s = FromRc(ctx, ehip_malloc(ctx, n, &p)); !s.ok()) return s;
  ctx_ = ctx;
  ptr_ = p;
  bytes_ = n;
  return Status::Ok();
}

Status DeviceBuffer::Upload(ehip_ctx* ctx, const void* src, int64_t bytes) {
  if (Status s = Reserve(ctx, bytes); !s.ok()) return s;
  return FromRc(ctx, ehip_copy_to_device(ctx, ptr_, src, bytes));
}

void DeviceBuffer::Reset() {
  if (ptr_ != nullptr) (void)ehip_free(ctx_, ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

}  // namespace ehip::host
