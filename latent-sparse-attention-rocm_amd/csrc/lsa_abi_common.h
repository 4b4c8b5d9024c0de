// Host-side helpers shared by the extern "C" entry points: thread-local last error,
// argument checks (run before any HIP call, so they are testable without a GPU) and
// element-type / span dispatch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "lsa_rocm.h"
#include "lsa_rocm_testing.h"

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

namespace lsa {

inline int check_tables(int32_t rows, int32_t cap, int64_t row_tables, int64_t group_tables) {
  LSA_REQUIRE(rows >= 1, LSA_ERR_SHAPE, "bucket table needs >= 1 row, got %d", rows);
  LSA_REQUIRE(cap >= 1, LSA_ERR_SHAPE, "bucket cap must be >= 1, got %d", cap);
  LSA_REQUIRE(row_tables >= 0 && group_tables >= 0, LSA_ERR_SHAPE, "table strides must be >= 0");
  return LSA_OK;
}

inline int check_dim(int32_t D) {
  LSA_REQUIRE(D >= 16 && D <= 256 && is_pow2(D), LSA_ERR_SHAPE,
              "index dim must be a power of two in [16, 256], got %d", D);
  return LSA_OK;
}

inline int check_dtype(int dtype) {
  LSA_REQUIRE(dtype == LSA_F32 || dtype == LSA_BF16 || dtype == LSA_F16, LSA_ERR_DTYPE, "unknown dtype %d", dtype);
  return LSA_OK;
}

// The scoring loads a lane's D/16 centroid elements with vector loads and the expansion
// loads member rows as 16-byte vectors when cap % 32 == 0: both need aligned tables.
inline int check_query_aligned(const void* q, int q_dtype, int D) {
  size_t need = (size_t)(D / 16) * (q_dtype == LSA_F32 ? 4 : 2);
  need = need > 16 ? 16 : need;
  LSA_REQUIRE(((uintptr_t)q % need) == 0, LSA_ERR_ALIGN, "query rows must be %zu-byte aligned", need);
  return LSA_OK;
}

inline int check_aligned(const void* centroids, int D, int score_mode, const int32_t* members, int cap) {
  const size_t esize = score_mode == LSA_SCORE_F32 ? 4 : 2;
  size_t need = (size_t)(D / 16) * esize;
  need = need > 16 ? 16 : need;
  LSA_REQUIRE(centroids == nullptr || ((uintptr_t)centroids % need) == 0, LSA_ERR_ALIGN,
              "centroid table must be %zu-byte aligned", need);
  LSA_REQUIRE(members == nullptr || cap % 32 != 0 || ((uintptr_t)members % 16) == 0, LSA_ERR_ALIGN,
              "member table must be 16-byte aligned");
  return LSA_OK;
}

// Checks an optional slot map and copies it into the kernels' by-value form `out` (the
// device SlotMap: table == nullptr when there is none).
template <typename SlotMapT>
inline int check_slots(const char* who, const lsa_slot_map* m, SlotMapT* out) {
  *out = SlotMapT{nullptr, nullptr, 0, 0, 0};
  if (m == nullptr) return LSA_OK;
  LSA_REQUIRE(m->table && m->rows, LSA_ERR_NULL, "%s: slot map with a NULL table or rows", who);
  LSA_REQUIRE(m->width >= 1 && m->n_rows >= 1 && m->stride >= m->width, LSA_ERR_SHAPE,
              "%s: slot map needs n_rows >= 1 and stride >= width >= 1", who);
  *out = SlotMapT{m->table, m->rows, m->stride, m->width, m->n_rows};
  return LSA_OK;
}

}  // namespace lsa

#define LSA_LAUNCHED(what)                                                                    \
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
