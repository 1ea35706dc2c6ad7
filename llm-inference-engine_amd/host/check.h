// Programmer-error checks: print the condition and message, then abort. The
// reference's CHECK (src/core/check.h) has the same posture — a broken caller
// contract (double free, sharing a free block, querying an uncommitted slot)
// is not a recoverable Status.
#pragma once

#include <string>

#include "status.h"

namespace ehip::host {
[[noreturn]] void CheckFail(const char* file, int line, const char* cond, const std::string& msg);
}  // namespace ehip::host

#define EHIP_CHECK(cond, ...)                                                               \
  do {                                                                                      \
    if (__builtin_expect(!(cond), 0))                                                       \
      ::ehip::host::CheckFail(__FILE__, __LINE__, #cond, ::ehip::host::Format(__VA_ARGS__)); \
  } while (0)
