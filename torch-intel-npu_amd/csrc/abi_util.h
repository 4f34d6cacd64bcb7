// Host-side helpers shared by the C-ABI translation units: the thread-local error message,
// alignment and buffer-overlap checks.
#pragma once
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
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

// Process-wide failure state, the counterpart of the reference's failed context
// (npunlock-probe/torch-device/backend.cpp:58-60, 280-292): once a launch reports a device error,
// or a caller reports a failed synchronisation through lb_mark_failed, every entry point that
// enqueues work refuses with LB_DEVICE_FAILED until the process restarts.
struct FailedState {
  std::atomic<bool> failed{false};
  std::mutex mutex;
  std::string reason;
};

inline FailedState &failed_state() {
  static FailedState state;
  return state;
}

inline void mark_failed(const char *reason) {
  FailedState &st = failed_state();
  std::lock_guard<std::mutex> lock(st.mutex);
  if (!st.failed.load(std::memory_order_relaxed)) st.reason = reason ? reason : "unspecified";
  st.failed.store(true, std::memory_order_release);
}

inline lb_status refuse_if_failed(const char *what) {
  FailedState &st = failed_state();
  if (!st.failed.load(std::memory_order_acquire)) return LB_OK;
  std::lock_guard<std::mutex> lock(st.mutex);
  return fail(LB_DEVICE_FAILED, "%s: the device failed earlier (%s); restart the process before using its buffers",
              what, st.reason.c_str());
}

// Status of the launches just enqueued: a launch error marks the library failed.
inline lb_status launch_status(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ok();
  char reason[256];
  snprintf(reason, sizeof reason, "%s: %s", what, hipGetErrorString(e));
  mark_failed(reason);
  return fail(LB_DEVICE_FAILED, "%s", reason);
}

}  // namespace abi
}  // namespace lb
