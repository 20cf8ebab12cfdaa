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

// Output-tile shapes of the tiled kernels. Larger tiles reuse each staged
// operand byte across more MFMAs; smaller ones make more workgroups for
// shapes that would otherwise leave CUs idle.
enum TileCfg { TILE_256x256 = 0, TILE_128x128 = 1, TILE_64x128 = 2 };

inline TileCfg pick_tile(int64_t M, int64_t N) {
  const int64_t cus = 256;
  if (cdiv(M, 256) * cdiv(N, 256) >= 2 * cus) return TILE_256x256;
  if (cdiv(M, 128) * cdiv(N, 128) >= cus) return TILE_128x128;
  return TILE_64x128;
}

}  // namespace c4q
