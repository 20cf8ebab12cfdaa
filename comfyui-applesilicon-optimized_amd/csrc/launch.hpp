// Launch helpers binding the tiled and generic kernels to an entry point.
#pragma once
#include <stdlib.h>

#include "api_common.hpp"
#include "epilogues.hpp"
#include "gemm_tile.hpp"
#include "generic.hpp"

namespace c4q {

// Tile variants of the MFMA kernels: BM x BN output tile, WM x WN waves,
// the LDS budget of one workgroup (160 KB: one workgroup per CU; less
// leaves room for two or three) and the stage depth in K of the 8-bit
// operand policies (64 or 128).
template <int BM_, int BN_, int WM_, int WN_, int LDS_KB_, int KS8_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NT = 64 * WM_ * WN_;
  static constexpr int LDS = LDS_KB_ * 1024;
  static constexpr int KS8 = KS8_;
};

// Ring depth: as many stages as the budget holds next to the epilogue
// strips, at most 4.
template <class T, class Op, bool PAIR>
constexpr int ring_depth() {
  constexpr int stage = T::BM * Op::SA + T::BN * Op::SB;
  constexpr int strips = (T::WM * T::WN) * strip_bytes<T::BN / T::WN / 32, PAIR>();
  constexpr int n = (T::LDS - strips) / stage;
  return n > 4 ? 4 : (n < 2 ? 2 : n);
}
enum TileId : int {
  TILE_256x256_W8 = 0,   // 8 waves (2 per SIMD), 128x64 per wave
  TILE_256x256_W4 = 1,   // 4 waves, 128x128 per wave
  TILE_128x128_W4 = 2,   // 4 waves, 64x64 per wave
  TILE_64x128_W4 = 3,    // 4 waves, 32x64 per wave
  TILE_128x128_W4_K128 = 4,
  TILE_64x128_W4_K128 = 5,
  TILE_256x256_W8_K64 = 6,
  TILE_COUNT = 7,
};

template <class F>
int with_tile(int id, F&& f) {
  switch (id) {
    case TILE_256x256_W8: return f(Tile<256, 256, 2, 4, 160, 128>{});
    case TILE_256x256_W4: return f(Tile<256, 256, 2, 2, 160, 128>{});
    case TILE_128x128_W4: return f(Tile<128, 128, 2, 2, 80, 64>{});
    case TILE_128x128_W4_K128: return f(Tile<128, 128, 2, 2, 80, 128>{});
    case TILE_64x128_W4_K128: return f(Tile<64, 128, 2, 2, 64, 128>{});
    case TILE_256x256_W8_K64: return f(Tile<256, 256, 2, 4, 160, 64>{});
    default: return f(Tile<64, 128, 2, 2, 53, 64>{});
  }
}

// Tile choice by a cost model of the persistent kernel: a tile variant runs
// in ceil(tiles / slots) rounds (slots = CUs x resident workgroups per CU),
// each costing one tile's MACs times the slots it fills, at the variant's
// measured relative per-CU throughput on large shapes (MI355X, 8-bit
// operands: 256x256 w8 1.00, 256x256 w4 0.90, 128x128 0.87, 64x128 0.70).
// A tile id in the environment variable C4Q_TILE (0..6) overrides it, for
// tuning sweeps.
inline int pick_tile(int64_t M, int64_t N) {
  const char* env = getenv("C4Q_TILE");
  if (env && env[0] >= '0' && env[0] < '0' + TILE_COUNT && env[1] == 0) return env[0] - '0';
  struct Cand { int id, bm, bn, per_cu; double eff; };
  static const Cand cands[] = {{TILE_256x256_W8, 256, 256, 1, 1.00},
                               {TILE_128x128_W4_K128, 128, 128, 2, 0.87},
                               {TILE_64x128_W4_K128, 64, 128, 2, 0.70}};
  const double cus = 256;
  int best = TILE_256x256_W8;
  double best_cost = 0;
  for (const Cand& c : cands) {
    const double tiles = (double)(cdiv(M, c.bm) * cdiv(N, c.bn));
    const double slots = cus * c.per_cu;
    const double rounds = (double)(int64_t)((tiles + slots - 1) / slots);
    const double cost = rounds * slots * c.bm * c.bn / c.eff;
    if (c.id == TILE_256x256_W8 || cost < best_cost) {
      best = c.id;
      best_cost = cost;
    }
  }
  return best;
}

// Compute units of the current device (cached per device id).
int device_cus();

// Workgroups of the persistent kernel: one per tile while tiles are fewer
// than the resident slots (CUs x workgroups per CU), else every slot. `occ`
// caches the kernel's workgroups per CU (one cache per launch_tile
// instantiation: kernels of different tiles share a function type, so the
// cache cannot be keyed on that).
template <class K>
int persistent_grid(K kernel, int nt, int64_t tiles, int& occ) {
  if (occ <= 0) {
    int o = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel, nt, 0) != hipSuccess || o < 1) o = 1;
    occ = o;
  }
  const int64_t slots = (int64_t)device_cus() * occ;
  return (int)(tiles < slots ? tiles : slots);
}

template <class T, class Op, bool PAIR, class Epi>
int launch_tile(GemmShape sh, int64_t n_rows_b, const Src2& sa, const Src2& sb, const float* b_scale,
                const Epi& epi, hipStream_t s, const char* what) {
  sh.tiles_m = (int)cdiv(sh.M, T::BM);
  sh.tiles_n = (int)cdiv(n_rows_b, T::BN);
  const int64_t tiles = (int64_t)sh.tiles_m * sh.tiles_n;
  C4Q_REQUIRE(tiles < (1ll << 30), C4Q_ERR_SHAPE, "%s: problem too large (%lld tiles)", what,
              (long long)tiles);
  constexpr int nbuf = ring_depth<T, Op, PAIR>();
  auto kernel = gemm_tile_kernel<Op, T::BM, T::BN, T::WM, T::WN, nbuf, PAIR, Epi>;
  static int occ = 0;
  const int grid = persistent_grid(kernel, T::NT, tiles, occ);
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, s, sh, sa, sb, b_scale, epi);
  return check_launch(what);
}

template <class Op, class Epi>
int launch_generic(int64_t M, int64_t N, int64_t K, const Op& op, const Epi& epi, hipStream_t s,
                   const char* what) {
  const int64_t nbx = cdiv(N, 64);
  const int64_t blocks = nbx * cdiv(M, 4);
  C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
  hipLaunchKernelGGL((gemm_generic_kernel<Op, Epi>), dim3((unsigned)blocks), dim3(256), 0, s, M, N,
                     K, nbx, op, epi);
  return check_launch(what);
}

// The tiled kernels address one tile (at most 256 rows) with 32-bit byte
// offsets inside a buffer resource.
inline bool tile_offsets_fit(int64_t lda_bytes, int64_t ldb_bytes) {
  return lda_bytes <= (1ll << 22) && ldb_bytes <= (1ll << 22);
}

// 8-bit x 8-bit GEMM (int8 or fp8 operands) with epilogue Epi; OpT<KS> is
// the operand policy at stage depth KS.
template <template <int> class OpT, class GenOp, class Epi>
int run_gemm8(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, int64_t M, int64_t N,
              int64_t K, const Epi& epi, hipStream_t s, const char* what) {
  if (M == 0 || N == 0) return C4Q_OK;
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(b) && lda % 16 == 0 &&
                     ldb % 16 == 0 && tile_offsets_fit(lda, ldb);
  if (!tiled) return launch_generic(M, N, K, GenOp::make(a, lda, b, ldb), epi, s, what);
  GemmShape sh{M, N, K, 0, 0};
  const Src2 sa{a, a, lda, M}, sb{b, b, ldb, N};
  return with_tile(pick_tile(M, N), [&](auto t) {
    using T = decltype(t);
    return launch_tile<T, OpT<T::KS8>, false>(sh, N, sa, sb, nullptr, epi, s, what);
  });
}

}  // namespace c4q
