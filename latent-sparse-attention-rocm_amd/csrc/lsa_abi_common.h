// Host-side helpers shared by the extern "C" entry points: thread-local last error,
// argument checks (run before any HIP call, so they are testable without a GPU) and
// element-type / span dispatch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "lsa_rocm.h"

namespace lsa {

int fail(int code, const char* fmt, ...);
void clear_error();

// Test hooks of the fused decode (thread-local, set by lsa_debug_decode).
struct DecodeDebug {
  int skip_publish;  // select workgroups never publish the record
  int spin_limit;    // polls before a reader gives up; 0 = the default
};
const DecodeDebug& decode_debug();

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

}  // namespace lsa

#define LSA_REQUIRE(cond, code, ...)                 \
  do {                                               \
    if (!(cond)) return ::lsa::fail(code, __VA_ARGS__); \
  } while (0)

#define LSA_LAUNCHED(what)                                                                     \
  do {                                                                                         \
    hipError_t err_ = hipGetLastError();                                                       \
    if (err_ != hipSuccess) return ::lsa::fail(LSA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err_)); \
  } while (0)

// Propagates a nonzero status of a host-side check.
#define LSA_TRY(expr)              \
  do {                             \
    int rc_ = (expr);              \
    if (rc_ != LSA_OK) return rc_; \
  } while (0)

// Query / key element type dispatch: binds QT.
#define LSA_DISPATCH_QT(dtype, ...)                       \
  switch (dtype) {                                        \
    case LSA_F32: { using QT = float; __VA_ARGS__; } break;          \
    case LSA_BF16: { using QT = ::lsa::bf16_t; __VA_ARGS__; } break; \
    default: { using QT = _Float16; __VA_ARGS__; } break;            \
  }

// Canonical-score span (D / 16) dispatch: binds SPAN.
#define LSA_DISPATCH_SPAN(span, ...)                      \
  switch (span) {                                         \
    case 1: { constexpr int SPAN = 1; __VA_ARGS__; } break;   \
    case 2: { constexpr int SPAN = 2; __VA_ARGS__; } break;   \
    case 4: { constexpr int SPAN = 4; __VA_ARGS__; } break;   \
    case 8: { constexpr int SPAN = 8; __VA_ARGS__; } break;   \
    default: { constexpr int SPAN = 16; __VA_ARGS__; } break; \
  }
