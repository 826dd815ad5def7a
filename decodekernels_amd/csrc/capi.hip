// C-ABI utilities: per-thread argument-error message, error strings, version.
#include <string>

#include "../../include/decodekernels_amd.h"
#include "dk_host.h"

namespace dk {

namespace {
thread_local std::string g_last_error;
}

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return static_cast<int>(hipErrorInvalidValue);
}

void clear_error() { g_last_error.clear(); }

}  // namespace dk

extern "C" const char* dk_last_error(void) { return dk::g_last_error.c_str(); }

extern "C" const char* dk_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

// The package version (pyproject.toml's [project] version, checked by
// tests/test_packaging.py) and the target.
extern "C" const char* dk_version(void) { return "decodekernels_amd 0.2.0 (gfx950)"; }
