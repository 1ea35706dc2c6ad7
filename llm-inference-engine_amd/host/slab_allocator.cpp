#include "slab_allocator.h"

#include <cstdlib>
#include <cstring>

namespace ehip::host {

void* HostSlabAllocator::Allocate(std::size_t bytes, std::size_t align, Status* status) {
  const std::size_t n = ((bytes == 0 ? 1 : bytes) + align - 1) / align * align;
  void* p = std::aligned_alloc(align, n);
  if (p == nullptr) {
    *status = Error(StatusCode::kOutOfMemory, Format("host slab of %zu bytes", bytes));
    return nullptr;
  }
  std::memset(p, 0, n);
  *status = Status::Ok();
  return p;
}

void HostSlabAllocator::Free(void* p) { std::free(p); }

void* HbmSlabAllocator::Allocate(std::size_t bytes, std::size_t align, Status* status) {
  if (align > 256) {
    *status = Error(StatusCode::kInvalidArgument,
                    Format("HBM slabs are 256-byte aligned; %zu requested", align));
    return nullptr;
  }
  void* p = nullptr;
  const int rc = ehip_malloc(ctx_, static_cast<int64_t>(bytes), &p);  // zero-filled
  if (rc != EHIP_OK) {
    char msg[512];
    ehip_last_error(ctx_, msg, sizeof msg);
    *status = Error(static_cast<StatusCode>(rc), msg);
    return nullptr;
  }
  *status = Status::Ok();
  return p;
}

void HbmSlabAllocator::Free(void* p) { (void)ehip_free(ctx_, p); }

}  // namespace ehip::host
