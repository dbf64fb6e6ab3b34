// Host-side helpers shared by the C-ABI entry points of libq6moe.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "../../include/q6moe.h"

namespace q6moe {

void set_error(const std::string& msg);

// Record a HIP error (if any) after a launch; returns 0 or Q6MOE_ERR_HIP.
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

#define Q6MOE_REQUIRE(cond, msg)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::q6moe::set_error(msg);                   \
      return Q6MOE_ERR_INVALID;                  \
    }                                            \
  } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Runs f() the first time it is reached on the current device. Kernel
// attributes (hipFuncSetAttribute) belong to a device, so each device of the
// process sets its own; ``done`` holds one bit per device id (0-63). Two
// threads may both run f() for one device, which only sets an attribute twice.
template <typename F>
inline void once_per_device(std::atomic<uint64_t>& done, F&& f) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return;
  f();
  done.fetch_or(bit, std::memory_order_release);
}

}  // namespace q6moe
