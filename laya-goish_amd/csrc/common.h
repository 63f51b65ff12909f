// Shared host-side plumbing: status codes carried by exceptions inside the library,
// converted to LG_ERR_* + a thread-local message at the C ABI (capi.cpp).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "lg.h"

namespace lg {

// Word 3 of a raw buffer resource on gfx9 (32-bit data format, no swizzle); reads beyond
// num_records return zero.
constexpr int kBufferFlags = 0x00020000;

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Error(code, buf);
}

inline void hip_check(hipError_t e, const char *what, const char *file, int line) {
  if (e != hipSuccess)
    fail(LG_ERR_DEVICE, "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
}
#define HIP_CHECK(x) ::lg::hip_check((x), #x, __FILE__, __LINE__)

// Launch-bounds check helper: every kernel launcher validates its shapes on the host.
#define LG_REQUIRE(cond, ...)                       \
  do {                                              \
    if (!(cond)) ::lg::fail(LG_ERR_INVALID, __VA_ARGS__); \
  } while (0)

}  // namespace lg
