// SPDX-License-Identifier: Apache-2.0
// Host-side helpers shared by the C-ABI entry points: status codes, the thread-local error message and
// argument checks. Every entry point validates its arguments, launches on the caller's stream and
// returns 0 or a negative status; it never allocates and never synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/exl3_mi355x.h"

namespace exl3 {

void set_error(const char* fmt, ...);

#define EXL3_REQUIRE(cond, code, ...) \
  do {                                \
    if (!(cond)) {                    \
      ::exl3::set_error(__VA_ARGS__); \
      return (code);                  \
    }                                 \
  } while (0)

#define EXL3_LAUNCH_CHECK(what)                                                             \
  do {                                                                                      \
    hipError_t _e = hipGetLastError();                                                      \
    if (_e != hipSuccess) {                                                                 \
      ::exl3::set_error("%s: launch failed: %s", (what), hipGetErrorString(_e));            \
      return EXL3_ERR_HIP;                                                                  \
    }                                                                                       \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// True when the byte ranges [a, a + an) and [b, b + bn) share a byte (a NULL pointer overlaps nothing).
inline bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
  if (!a || !b || an == 0 || bn == 0) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + bn && b0 < a0 + an;
}

// Device address of codebook cb's 65,536-entry fp16 lookup table on the current device (nullptr on failure).
const uint16_t* codebook_table(int cb);

}  // namespace exl3
