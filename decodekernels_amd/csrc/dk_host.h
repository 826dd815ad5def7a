// Host-side helpers shared by the C-ABI entry points: argument-error
// reporting and small integer utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

namespace dk {

// Records a description of an argument error for dk_last_error() and returns
// hipErrorInvalidValue, so a validation branch reads `return fail("...")`.
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Clears the thread's last error message.
void clear_error();

inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned_to(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

}  // namespace dk
