// Host-side helpers shared by the C-ABI translation units: the thread-local error message,
// alignment and buffer-overlap checks.
#pragma once
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/lowbit_hip.h"

namespace lb {
namespace abi {

inline std::string &last_error() {
  thread_local std::string message;
  return message;
}

inline lb_status fail(lb_status status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  last_error() = buf;
  return status;
}

inline lb_status ok() {
  last_error().clear();
  return LB_OK;
}

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

struct Range {
  uintptr_t lo = 0, hi = 0;  // [lo, hi)
  const char *name = "";
};

inline Range range_of(const void *p, size_t bytes, const char *name) {
  Range r;
  r.lo = reinterpret_cast<uintptr_t>(p);
  r.hi = r.lo + bytes;
  r.name = name;
  return r;
}

inline bool overlaps(const Range &a, const Range &b) {
  return a.lo != a.hi && b.lo != b.hi && a.lo < b.hi && b.lo < a.hi;
}

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace abi
}  // namespace lb
