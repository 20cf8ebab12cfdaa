// Host-side plumbing shared by the entry points: error state, argument
// checks, tile-configuration choice and the launch helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cdna4q.h"

namespace c4q {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define C4Q_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      ::c4q::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)

// Reports a failed launch (bad configuration, invalid stream, ...).
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Output rows can take 16-byte stores: aligned base, row pitch a multiple of 16.
inline int rows_vec16(const void* d, int64_t ld, int64_t elem_bytes) {
  return aligned16(d) && (ld * elem_bytes) % 16 == 0 ? 1 : 0;
}

}  // namespace c4q
