// Host-side checks of the library's own planning and error code under
// AddressSanitizer and UndefinedBehaviorSanitizer (built host-only by
// tests/native/Makefile, run on the CPU by tests/test_host_sanitized.py):
//   * the tile plans of the three tile sets (plan_launches, tile_at: the functions
//     the entry points run before every launch) over a grid of shapes, K
//     values and CU counts, each 32 x 64 output cell computed exactly once;
//   * the error path of the C ABI (set_error / c4q_last_error): formatting,
//     truncation of over-long messages, the ABI version.
// Exit status 0 when every check passes; a sanitizer report aborts.
#include <stdio.h>
#include <string.h>

#include <vector>

#include "launch.hpp"

using namespace c4q;

namespace {

int failures = 0;
int64_t idle_pieces = 0;

void fail(const char* what, int64_t M, int64_t N, int64_t K, int cus) {
  if (failures++ < 20)
    fprintf(stderr, "FAIL %s: M=%lld N=%lld K=%lld cus=%d\n", what, (long long)M, (long long)N,
            (long long)K, cus);
}

template <class Set>
void check_plan(int64_t M, int64_t N, int64_t K, int cus) {
  int ids[2] = {-1, -1};
  GemmShape shs[2];
  const int n = plan_launches<Set>(M, N, N, K, cus, ids, shs);
  if (n < 1 || n > 2) return fail("launch count", M, N, K, cus);
  const int64_t cm = cdiv(M, 32), cn = cdiv(N, 64);     // cells of 32 rows x 64 columns
  std::vector<int> cover((size_t)(cm * cn), 0);
  for (int l = 0; l < n; ++l) {
    const int bm = Set::bm(ids[l]), bn = Set::bn(ids[l]);
    if (bm <= 0 || bn <= 0 || bm % 32 || bn % 64) return fail("tile size", M, N, K, cus);
    if (shs[l].count <= 0) return fail("empty launch", M, N, K, cus);
    // kernel tiles lie in the grid of mapped tiles (a leftover mapped tile
    // split into pieces can leave a piece wholly past the matrix edge: it
    // reads zeros and stores nothing)
    const int64_t tm_max = (int64_t)shs[l].tiles_m * shs[l].sub_m;
    const int64_t tn_max = (int64_t)shs[l].tiles_n * shs[l].sub_n;
    for (int i = 0; i < shs[l].count; ++i) {
      const TileCoord t = tile_at(shs[l], i);
      if (t.tm < 0 || t.tn < 0 || t.tm >= tm_max || t.tn >= tn_max)
        return fail("tile outside the mapped grid", M, N, K, cus);
      if ((int64_t)t.tm * bm >= M || (int64_t)t.tn * bn >= N) ++idle_pieces;
      for (int64_t r = (int64_t)t.tm * bm; r < (int64_t)(t.tm + 1) * bm && r < M; r += 32)
        for (int64_t c = (int64_t)t.tn * bn; c < (int64_t)(t.tn + 1) * bn && c < N; c += 64)
          ++cover[(size_t)((r / 32) * cn + c / 64)];
    }
  }
  for (int v : cover)
    if (v != 1) return fail("cell not computed exactly once", M, N, K, cus);
}

void check_errors() {
  set_error("%s: bad value %d of %lld", "c4q_test", 7, (long long)1 << 40);
  if (strcmp(c4q_last_error(), "c4q_test: bad value 7 of 1099511627776") != 0)
    fail("error message", 0, 0, 0, 0);
  std::vector<char> longmsg(4000, 'x');
  longmsg.back() = 0;
  set_error("%s", longmsg.data());
  const size_t len = strlen(c4q_last_error());
  if (len == 0 || len >= 4000) fail("error truncation", (int64_t)len, 0, 0, 0);
  if (c4q_abi_version() != C4Q_ABI_VERSION) fail("abi version", 0, 0, 0, 0);
}

}  // namespace

int main() {
  const int64_t sizes[] = {1, 17, 64, 100, 255, 256, 257, 640, 1000, 1024, 3072,
                           4608, 5000, 9216, 12288, 16384, 21504};
  const int64_t ks[] = {16, 3072, 13824};
  const int cus_list[] = {1, 8, 80, 256, 304};
  int plans = 0;
  for (int64_t M : sizes)
    for (int64_t N : sizes)
      for (int64_t K : ks)
        for (int cus : cus_list) {
          check_plan<MainTiles>(M, N, K, cus);
          check_plan<HeadTiles>(M, N, K, cus);
          check_plan<W8A16Tiles>(M, N, K, cus);
          plans += 3;
        }
  check_errors();
  printf("%d plans checked, %d failures (%lld leftover pieces wholly past the edge)\n", plans,
         failures, (long long)idle_pieces);
  return failures == 0 ? 0 : 1;
}
