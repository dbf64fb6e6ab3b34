// Host-side helpers shared by the C-ABI entry points of libq6moe.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
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

}  // namespace q6moe
