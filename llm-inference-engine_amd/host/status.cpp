#include "status.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "check.h"

namespace ehip::host {

std::string Format(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  va_list ap2;
  va_copy(ap2, ap);
  const int n = std::vsnprintf(nullptr, 0, fmt, ap);
  va_end(ap);
  std::string out(n > 0 ? static_cast<size_t>(n) : 0, '\0');
  if (n > 0) std::vsnprintf(out.data(), out.size() + 1, fmt, ap2);
  va_end(ap2);
  return out;
}

void CheckFail(const char* file, int line, const char* cond, const std::string& msg) {
  std::fprintf(stderr, "CHECK failed at %s:%d: %s: %s\n", file, line, cond, msg.c_str());
  std::fflush(stderr);
  std::abort();
}

}  // namespace ehip::host
