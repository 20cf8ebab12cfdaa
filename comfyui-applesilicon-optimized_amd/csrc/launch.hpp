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
// leaves room for two or three), the stage depth in K of the 8-bit operand
// policies (64 or 128) and the number of K groups (KG > 1: the split-K
// kernel, KG groups of WM x WN waves).
template <int BM_, int BN_, int WM_, int WN_, int LDS_KB_, int KS8_, int KG_ = 1>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, KG = KG_;
  static constexpr int NT = 64 * WM_ * WN_ * KG_;
  static constexpr int LDS = LDS_KB_ * 1024;
  static constexpr int KS8 = KS8_;
};

// Ring depth: as many stages as the budget holds next to the epilogue
// strips, at most 4.
template <class T, class Op, bool PAIR>
constexpr int ring_depth() {
  constexpr int stage = T::KG * (T::BM * Op::SA + T::BN * Op::SB);
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
  TILE_64x64_KG4 = 7,    // split-K: 4 groups of 2 waves, 32x64 per wave
  TILE_COUNT = 8,
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
    case TILE_64x64_KG4: return f(Tile<64, 64, 2, 1, 132, 128, 4>{});
    default: return f(Tile<64, 128, 2, 2, 53, 64>{});
  }
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

// Operand policy of the ping-pong kernel: 8-bit operands stage 64 K, so
// that the ring holds four stages (copies run three stages ahead).
template <class Op> struct PingPongOp { using type = Op; };
template <> struct PingPongOp<OpI8T<128>> { using type = OpI8T<64>; };
template <> struct PingPongOp<OpF8T<128>> { using type = OpF8T<64>; };

// The 8-wave tiles take the ping-pong schedule where the operand policy asks
// for it (W8A16: its 48 KB stage leaves a three-stage ring, and the dequant
// work lengthens the MFMA interval against the memory interval; MI355X,
// FLUX shapes: +1-3%). 8-bit operands keep the one-group schedule, whose
// 128-K stages beat the 64-K stages ping-pong needs (-5-10% with them).
// C4Q_PINGPONG=0 / 1 in the environment forces either, for tuning sweeps.
template <class Op>
inline bool pingpong_on() {
  const char* e = getenv("C4Q_PINGPONG");
  if (e && (e[0] == '0' || e[0] == '1') && e[1] == 0) return e[0] == '1';
  return Op::kPingPong;
}

// K from which fp8 GEMMs on the 256x256 tile take gemm_w4_kernel
// (MI355X, same-process A/B against the 8-wave kernel, bits identical:
// 16384 rows, K = 13824 +11.6 %, K = 8192 +3.6 %, K = 5120 0 to +3 %,
// K = 3072 -3 to -5 %).
constexpr int64_t kW4MinK = 5120;

template <class Op> struct IsF8 : std::false_type {};
template <int KS> struct IsF8<OpF8T<KS>> : std::true_type {};

// fp8 on the 256x256 tile: gemm_w4_kernel (one wave per SIMD, 128-K stages)
// where K is long. C4Q_W4=0 / 1 in the environment forces either, for
// sweeps.
inline bool w4_for_fp8(int64_t K) {
  const char* e = getenv("C4Q_W4");
  if (e && (e[0] == '0' || e[0] == '1') && e[1] == 0) return e[0] == '1';
  return K >= kW4MinK;
}

template <class Op> struct IsW8A16 : std::false_type {};
template <bool B, bool S> struct IsW8A16<OpW8A16<B, S>> : std::true_type {
  static constexpr bool kBF16 = B, kScale = S;
};

// W8A16 on the 256x256 tile: gemm_w4a16_kernel (one wave per SIMD) with
// 1 x 4 waves (C4Q_W4A16=1) or 2 x 2 waves (=2), or the 8-wave ping-pong
// kernel (=0), for sweeps.
inline int w4a16_mode() {
  const char* e = getenv("C4Q_W4A16");
  if (e && e[0] >= '0' && e[0] <= '2' && e[1] == 0) return e[0] - '0';
  return 1;
}

template <class T, class Op, bool PAIR, class Epi>
int launch_tile(const GemmShape& sh, const Src2& sa, const Src2& sb, const float* b_scale,
                const Epi& epi, hipStream_t s, const char* what) {
  // 224 x 256: the W8A16 one-wave-per-SIMD kernel only (W8A16Tiles)
  if constexpr (T::BM == 224) {
    static_assert(IsW8A16<Op>::value && !PAIR && T::BN == 256 && T::WM == 1 && T::WN == 4,
                  "the 224-row tile is W8A16 on 1 x 4 waves");
    auto kernel = gemm_w4a16_kernel<IsW8A16<Op>::kBF16, IsW8A16<Op>::kScale, 1, 4, 3, Epi, 224>;
    static int bocc = 0;
    const int grid = persistent_grid(kernel, 256, sh.count, bocc);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, s, sh, sa, sb, b_scale, epi);
    return check_launch(what);
  } else {
  if constexpr (IsW8A16<Op>::value && !PAIR && T::BM == 256 && T::BN == 256 && T::WM == 2 &&
                T::WN == 4 && T::KG == 1) {
    const int mode = w4a16_mode();
    if (mode != 0) {
      auto kernel = mode == 1 ? gemm_w4a16_kernel<IsW8A16<Op>::kBF16, IsW8A16<Op>::kScale, 1, 4, 3, Epi>
                              : gemm_w4a16_kernel<IsW8A16<Op>::kBF16, IsW8A16<Op>::kScale, 2, 2, 3, Epi>;
      static int aocc = 0;
      const int grid = persistent_grid(kernel, 256, sh.count, aocc);
      hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, s, sh, sa, sb, b_scale, epi);
      return check_launch(what);
    }
  }
  if constexpr (IsF8<Op>::value && !PAIR && T::BM == 256 && T::BN == 256 && T::WM == 2 &&
                T::WN == 4 && T::KG == 1) {
    if (w4_for_fp8(sh.K)) {
      auto kernel = gemm_w4_kernel<OpF8T<128>, 2, false, Epi>;
      static int wocc = 0;
      const int grid = persistent_grid(kernel, 256, sh.count, wocc);
      hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, s, sh, sa, sb, b_scale, epi);
      return check_launch(what);
    }
  }
  if constexpr (T::WM == 2 && T::WN == 4) {
    using POp = typename PingPongOp<Op>::type;
    constexpr int pbuf = ring_depth<T, POp, PAIR>();
    if constexpr (pbuf >= 3) {
      if (pingpong_on<Op>()) {
        auto kernel = gemm_pingpong_kernel<POp, T::BM, T::BN, pbuf, PAIR, Epi>;
        static int pocc = 0;
        const int grid = persistent_grid(kernel, T::NT, sh.count, pocc);
        hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, s, sh, sa, sb, b_scale, epi);
        return check_launch(what);
      }
    }
  }
  constexpr int nbuf = ring_depth<T, Op, PAIR>();
  if constexpr (T::KG > 1) {
    auto kernel = gemm_splitk_kernel<Op, T::BM, T::BN, T::WM, T::WN, T::KG, nbuf, PAIR, Epi>;
    static int kocc = 0;
    const int grid = persistent_grid(kernel, T::NT, sh.count, kocc);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, s, sh, sa, sb, b_scale, epi);
    return check_launch(what);
  } else {
    auto kernel = gemm_tile_kernel<Op, T::BM, T::BN, T::WM, T::WN, nbuf, PAIR, Epi>;
    static int occ = 0;
    const int grid = persistent_grid(kernel, T::NT, sh.count, occ);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, s, sh, sa, sb, b_scale, epi);
    return check_launch(what);
  }
  }
}

// Tile plan of one GEMM: the main tile variant and how many of its tiles
// (in tile_of order) the main launch takes; with a tail variant, the rest of
// the tiles are split into pieces of that variant in a second launch.
struct TilePlan {
  int main_id;
  int64_t main_count;
  int tail_id;              // < 0: no tail launch
};

inline int tile_bm(int id) { return with_tile(id, [](auto t) { return decltype(t)::BM; }); }
inline int tile_bn(int id) { return with_tile(id, [](auto t) { return decltype(t)::BN; }); }

// Cost model of the persistent kernel in CU-time units (one unit: the K MACs
// of one output element at the big tile's per-CU rate). A variant runs its
// tiles in rounds of `slots` (CUs x resident workgroups); a round costs the
// tile area x workgroups per CU / the variant's relative per-CU throughput,
// measured on large shapes (MI355X, 8-bit operands: 256x256 1.00, 128x128
// 0.87, 64x128 0.70). When the big tile's last round would leave CUs idle,
// its whole rounds can run as one launch and the leftover tiles, split into
// pieces of a smaller variant, as a second launch spread over every CU; the
// second launch costs about 3 us more (9e6 / K units at ~6 TOP/s per CU).
// The split-K 64x64 variant (0.30, one workgroup per CU) only takes such
// leftover pieces: as the only tile of a GEMM it loses to 64x128.
// A tile id in the environment variable C4Q_TILE (0..7) forces one launch
// of that variant, for tuning sweeps.
struct TileCand { int id, per_cu; double eff; };

// The cost model over a list of main tiles and a list of tail tiles; bm_of
// and bn_of give a tile id's shape.
inline TilePlan plan_from(const TileCand* cands, int nc, const TileCand* tails, int nt,
                          int (*bm_of)(int), int (*bn_of)(int), int64_t M, int64_t N, int64_t K,
                          int cus) {
  const double gap = 9e6 / (double)(K > 0 ? K : 1);
  TilePlan best{cands[0].id, 0, -1};
  double best_cost = -1;
  for (int ci = 0; ci < nc; ++ci) {
    const TileCand& c = cands[ci];
    const int bm = bm_of(c.id), bn = bn_of(c.id);
    const int64_t tiles = cdiv(M, bm) * cdiv(N, bn);
    const int64_t slots = (int64_t)cus * c.per_cu;
    const double round = (double)c.per_cu * bm * bn / c.eff;
    const double plain = (double)cdiv(tiles, slots) * round;
    if (best_cost < 0 || plain < best_cost) {
      best = {c.id, tiles, -1};
      best_cost = plain;
    }
    const int64_t whole = tiles / slots * slots, rest = tiles - whole;
    if (whole == 0 || rest == 0) continue;
    for (int ti = 0; ti < nt; ++ti) {
      const TileCand& t = tails[ti];
      const int tm = bm_of(t.id), tn = bn_of(t.id);
      if (tm * tn >= bm * bn || bm % tm || bn % tn) continue;
      const int64_t pieces = rest * (bm / tm) * (bn / tn);
      const int64_t tslots = (int64_t)cus * t.per_cu;
      const double cost = (double)(whole / slots) * round +
                          (double)cdiv(pieces, tslots) * t.per_cu * tm * tn / t.eff + gap;
      if (cost < best_cost) {
        best = {c.id, whole, t.id};
        best_cost = cost;
      }
    }
  }
  return best;
}

// A tile id forced by the environment variable `name` (one digit below
// `count`), else -1.
inline int forced_tile(const char* name, int count) {
  const char* env = getenv(name);
  if (env && env[0] >= '0' && env[0] < '0' + count && env[1] == 0) return env[0] - '0';
  return -1;
}

inline TilePlan plan_tiles(int64_t M, int64_t N, int64_t K, int cus) {
  const int id = forced_tile("C4Q_TILE", TILE_COUNT);
  if (id >= 0) return {id, cdiv(M, tile_bm(id)) * cdiv(N, tile_bn(id)), -1};
  static const TileCand cands[] = {{TILE_256x256_W8, 1, 1.00},
                                   {TILE_128x128_W4_K128, 2, 0.87},
                                   {TILE_64x128_W4_K128, 2, 0.70}};
  static const TileCand tails[] = {{TILE_128x128_W4_K128, 2, 0.87},
                                   {TILE_64x128_W4_K128, 2, 0.70},
                                   {TILE_64x64_KG4, 1, 0.30}};
  return plan_from(cands, 3, tails, 3, tile_bm, tile_bn, M, N, K, cus);
}

// The tile set of the general kernels.
struct MainTiles {
  template <class F> static int with(int id, F&& f) { return with_tile(id, f); }
  static int bm(int id) { return tile_bm(id); }
  static int bn(int id) { return tile_bn(id); }
  static TilePlan plan(int64_t M, int64_t N, int64_t K, int cus) { return plan_tiles(M, N, K, cus); }
};

// The tile set of W8A16 GEMMs: the general set plus 224 x 256 (id
// TILE_224x256_W8A16; gemm_w4a16_kernel with 1 x 4 waves of 224 x 64), which
// the cost model takes where 256-row tiles would leave a last round mostly
// idle. Its relative per-CU throughput, 0.92 of the 256 x 256 tile of the
// same kernel, is measured on MI355X (same process, bits identical): two
// full rounds of each at 9216 x 3072, K = 3072 and 12288, take 156.0 against
// 162.9 us and 581.6 against 607.5 us for 7/8 the work per tile.
// The split-K 64x64 tile is also a main candidate here (K >= 1024): with
// few tiles each CU runs one long K chain, and W8A16's in-register dequant
// makes that chain the bound; four wave groups over K cut it. Measured on
// MI355X (K = 3072, against the 64x128 plan): M = 65-256, N = 3072
// 32.9-33.2 -> 21.3-21.5 us; M = 128, K = 12288: 111.4 -> 46.6 us; where its
// pieces need two or more rounds the cost model keeps the larger tiles.
// C4Q_TILE=0..8 forces one launch of one of them, for tuning sweeps.
constexpr int TILE_224x256_W8A16 = TILE_COUNT;
struct W8A16Tiles {
  template <class F> static int with(int id, F&& f) {
    if (id == TILE_224x256_W8A16) return f(Tile<224, 256, 1, 4, 160, 128>{});
    return with_tile(id, f);
  }
  static int bm(int id) { return id == TILE_224x256_W8A16 ? 224 : tile_bm(id); }
  static int bn(int id) { return id == TILE_224x256_W8A16 ? 256 : tile_bn(id); }
  static TilePlan plan(int64_t M, int64_t N, int64_t K, int cus) {
    const int id = forced_tile("C4Q_TILE", TILE_COUNT + 1);
    if (id >= 0) return {id, cdiv(M, bm(id)) * cdiv(N, bn(id)), -1};
    static const TileCand cands[] = {{TILE_256x256_W8, 1, 1.00},
                                     {TILE_224x256_W8A16, 1, 0.92},
                                     {TILE_128x128_W4_K128, 2, 0.87},
                                     {TILE_64x128_W4_K128, 2, 0.70},
                                     {TILE_64x64_KG4, 1, 0.30}};
    static const TileCand tails[] = {{TILE_128x128_W4_K128, 2, 0.87},
                                     {TILE_64x128_W4_K128, 2, 0.70},
                                     {TILE_64x64_KG4, 1, 0.30}};
    TilePlan p = plan_from(cands, K >= 1024 ? 5 : 4, tails, 3, bm, bn, M, N, K, cus);
    // The model prices every round at two workgroups per CU. A 64x128 plan
    // with more tiles than CUs whose 128x128 tiles fit one per CU runs
    // faster on those (MI355X, K = 3072: 1024 x 3072 47.5 -> 43.2 us,
    // 256 x 9216 47.6 -> 43.0 us, 128 x 18432 47.7 -> 44.4 us).
    const int64_t t64 = cdiv(M, 64) * cdiv(N, 128), t128 = cdiv(M, 128) * cdiv(N, 128);
    if (p.main_id == TILE_64x128_W4_K128 && p.tail_id < 0 && t64 > cus && t128 <= cus)
      p = {TILE_128x128_W4_K128, t128, -1};
    return p;
  }
};

// Tiles whose waves each span 128 output columns -- one attention head --
// for epilogues that reduce over a head (IsHeadNorm): 256x256 with 8 waves
// of 64x128 (4 x 2; two waves per SIMD, so one wave's epilogue latency
// hides behind the other's work), 128x128 with 2 waves of 64x128 (two
// workgroups per CU) for leftover tiles, and 256x256 with 4 waves of
// 128x128. C4Q_HEAD_TILE=0/1/2 forces one launch of one of them, for
// tuning sweeps.
enum HeadTileId : int {
  HEAD_TILE_256x256_W8 = 0,
  HEAD_TILE_128x128_W2 = 1,
  HEAD_TILE_256x256_W4 = 2,
  HEAD_TILE_COUNT = 3
};
struct HeadTiles {
  template <class F> static int with(int id, F&& f) {
    if (id == HEAD_TILE_256x256_W8) return f(Tile<256, 256, 4, 2, 160, 128>{});
    if (id == HEAD_TILE_256x256_W4) return f(Tile<256, 256, 2, 2, 160, 128>{});
    return f(Tile<128, 128, 2, 1, 80, 128>{});
  }
  static int bm(int id) { return id == HEAD_TILE_128x128_W2 ? 128 : 256; }
  static int bn(int id) { return id == HEAD_TILE_128x128_W2 ? 128 : 256; }
  static TilePlan plan(int64_t M, int64_t N, int64_t K, int cus) {
    const int id = forced_tile("C4Q_HEAD_TILE", HEAD_TILE_COUNT);
    if (id >= 0) return {id, cdiv(M, bm(id)) * cdiv(N, bn(id)), -1};
    static const TileCand cands[] = {{HEAD_TILE_256x256_W8, 1, 1.00},
                                     {HEAD_TILE_128x128_W2, 2, 0.70}};
    static const TileCand tails[] = {{HEAD_TILE_128x128_W2, 2, 0.70}};
    return plan_from(cands, 2, tails, 1, bm, bn, M, N, K, cus);
  }
};

// The launches of a GEMM's tile plan as (tile id, shape) pairs; returns
// their number (1 or 2). n_rows_b = rows of the B tile space (pair kernels:
// 2 * N_out), N = output columns.
template <class Set = MainTiles>
inline int plan_launches(int64_t M, int64_t n_rows_b, int64_t N, int64_t K, int cus, int ids[2],
                         GemmShape shs[2]) {
  const TilePlan p = Set::plan(M, n_rows_b, K, cus);
  const int bm = Set::bm(p.main_id), bn = Set::bn(p.main_id);
  const int64_t mapped = cdiv(M, bm) * cdiv(n_rows_b, bn);
  GemmShape sh{M, N, K, (int)cdiv(M, bm), (int)cdiv(n_rows_b, bn), 0, (int)p.main_count, 1, 1};
  const char* gm_env = getenv("C4Q_GROUP_M");          // raster band height, for sweeps
  if (gm_env) {
    const int gm = atoi(gm_env);
    if (gm >= 1 && gm <= 64) sh.group_m = gm;
  }
  int n = 0;
  if (sh.count > 0) {
    ids[n] = p.main_id;
    shs[n++] = sh;
  }
  if (p.tail_id >= 0) {
    sh.first = (int)p.main_count;
    sh.sub_m = bm / Set::bm(p.tail_id);
    sh.sub_n = bn / Set::bn(p.tail_id);
    sh.count = (int)((mapped - p.main_count) * sh.sub_m * sh.sub_n);
    ids[n] = p.tail_id;
    shs[n++] = sh;
  }
  return n;
}

// Runs a GEMM through its tile plan. OpFor maps a Tile to its operand policy
// (a callable whose return type is the policy).
template <bool PAIR, class OpFor, class Epi, class Set = MainTiles>
int run_tiles(int64_t M, int64_t n_rows_b, int64_t N, int64_t K, const Src2& sa, const Src2& sb,
              const float* b_scale, const Epi& epi, hipStream_t s, const char* what, OpFor op_for,
              Set = {}) {
  // bound on the tile count of any plan (the smallest tile is 64 x 64)
  C4Q_REQUIRE(cdiv(M, 64) * cdiv(n_rows_b, 64) < (1ll << 27), C4Q_ERR_SHAPE,
              "%s: problem too large (%lld x %lld)", what, (long long)M, (long long)n_rows_b);
  int ids[2];
  GemmShape shs[2];
  const int n = plan_launches<Set>(M, n_rows_b, N, K, device_cus(), ids, shs);
  for (int l = 0; l < n; ++l) {
    const int st = Set::with(ids[l], [&](auto t) {
      using T = decltype(t);
      return launch_tile<T, decltype(op_for(t)), PAIR>(shs[l], sa, sb, b_scale, epi, s, what);
    });
    if (st != C4Q_OK) return st;
  }
  return C4Q_OK;
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
  const Src2 sa{a, a, lda, M}, sb{b, b, ldb, N};
  return run_tiles<false>(M, N, N, K, sa, sb, nullptr, epi, s, what,
                          [](auto t) { return OpT<decltype(t)::KS8>{}; });
}

}  // namespace c4q
