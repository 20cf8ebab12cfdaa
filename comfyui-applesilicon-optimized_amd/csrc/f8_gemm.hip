// FP8 e4m3fn x e4m3fn scaled GEMM (torch._scaled_mm semantics) and the
// W8A16 (bf16/f16 activation x fp8 weight) linear.
#include "launch.hpp"
#include "skinny.hpp"

using namespace c4q;

namespace {

bool valid_dt(int dt) { return dt == C4Q_BF16 || dt == C4Q_F16 || dt == C4Q_F32; }
bool valid_mode(int m) { return m == C4Q_SCALE_NONE || m == C4Q_SCALE_TENSOR || m == C4Q_SCALE_VECTOR; }

template <bool BF16, bool HAS_SCALE, class Epi>
int run_w8a16_tiled(const uint16_t* a, int64_t lda, const uint8_t* w, int64_t ldw,
                    const float* w_scale, int64_t M, int64_t N, int64_t K, const Epi& epi,
                    hipStream_t s, const char* what) {
  const Src2 sa{reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(a), 2 * lda, M};
  const Src2 sb{w, w, ldw, N};
  return run_tiles<false>(M, N, N, K, sa, sb, w_scale, epi, s, what,
                          [](auto) { return OpW8A16<BF16, HAS_SCALE>{}; }, W8A16Tiles{});
}

}  // namespace

extern "C" int c4q_f8_gemm_nt_scaled(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                                     void* d, int d_dtype, int64_t ldd, const float* scale_a,
                                     int scale_a_mode, const float* scale_b, int scale_b_mode,
                                     const float* scale_result, const void* bias, int bias_dtype,
                                     int64_t M, int64_t N, int64_t K, void* stream) {
  const char* what = "c4q_f8_gemm_nt_scaled";
  C4Q_REQUIRE(M >= 0 && N >= 0 && K >= 0, C4Q_ERR_SHAPE, "%s: negative size", what);
  C4Q_REQUIRE(lda >= K && ldb >= K && ldd >= N, C4Q_ERR_SHAPE, "%s: row stride smaller than row",
              what);
  C4Q_REQUIRE(valid_dt(d_dtype), C4Q_ERR_ARG, "%s: bad output dtype %d", what, d_dtype);
  C4Q_REQUIRE(valid_mode(scale_a_mode) && valid_mode(scale_b_mode), C4Q_ERR_ARG,
              "%s: bad scale mode", what);
  C4Q_REQUIRE(scale_a_mode == C4Q_SCALE_NONE || scale_a, C4Q_ERR_ARG, "%s: null scale_a", what);
  C4Q_REQUIRE(scale_b_mode == C4Q_SCALE_NONE || scale_b, C4Q_ERR_ARG, "%s: null scale_b", what);
  C4Q_REQUIRE(!bias || valid_dt(bias_dtype), C4Q_ERR_ARG, "%s: bad bias dtype", what);
  if (M == 0 || N == 0) return C4Q_OK;
  C4Q_REQUIRE(d && (K == 0 || (a && b)), C4Q_ERR_ARG, "%s: null pointer", what);
  auto run = [&](auto out) {
    constexpr int OUT = decltype(out)::value;
    EpiScaled<OUT> epi{{d, ldd, rows_vec16(d, ldd, OUT == DT_F32 ? 4 : 2)}, scale_a, scale_a_mode,
                       scale_b, scale_b_mode, scale_result, bias, bias_dtype, 0, 0, 1.0f};
    return run_gemm8<OpF8Any, GenF8>(a, lda, b, ldb, M, N, K, epi, as_stream(stream), what);
  };
  if (d_dtype == C4Q_F32) return run(std::integral_constant<int, DT_F32>{});
  if (d_dtype == C4Q_F16) return run(std::integral_constant<int, DT_F16>{});
  return run(std::integral_constant<int, DT_BF16>{});
}

namespace {
// Small-M route: 16-row weight blocks, K split over the waves of a
// persistent workgroup (4 chunks of 64 per wave, up to 16 waves), the blocks
// dealt to as many workgroups as fit on the device in one round (balanced
// rounds).
template <bool BF16, bool HAS_SCALE, class Epi>
int run_w8a16_skinny(const uint16_t* a, int64_t lda, const uint8_t* w, int64_t ldw,
                     const float* w_scale, int64_t M, int64_t N, int64_t K, const Epi& epi,
                     hipStream_t s, const char* what) {
  const int64_t nblk = cdiv(N, 16);
  const int64_t nch = cdiv(K, 64);
  auto launch = [&](auto kernel, int cpw, int& occ) {
    const int waves = (int)cdiv(nch, cpw);
    if (occ <= 0) {
      int o = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel, 64 * waves, 0) != hipSuccess || o < 1)
        o = 1;
      occ = o;
    }
    const int64_t slots = (int64_t)device_cus() * occ;
    const int64_t rounds = cdiv(nblk, slots);
    const int64_t grid = cdiv(nblk, rounds);
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * waves), 0, s, a, lda, w, ldw, w_scale,
                       M, N, K, epi);
    return check_launch(what);
  };
  // K <= 3072: at most 12 waves of 4 chunks, 6 blocks per barrier; up to
  // 4096: 16 waves, 4 blocks per barrier (the partial-tile area keeps one
  // workgroup per CU either way). Weight blocks in flight per wave: 2 for
  // M <= 4 with two or more blocks per workgroup, else 1 (the loads of one
  // block per wave across 12 waves already cover the HBM latency; deeper
  // prefetch only pays where each block's arithmetic is short -- MI355X,
  // N = 18432 / 3072, K = 3072). The bias width is a template parameter.
  // M in (16, 32]: two 16-row activation groups per wave (MG = 2), half as
  // many blocks per barrier.
  const int64_t slots = (int64_t)device_cus();
  const bool deep = M <= 4 && cdiv(nblk, slots) >= 2;
  auto pick = [&](auto bias_bits, auto depth) {
    constexpr int BIAS = decltype(bias_bits)::value, D = decltype(depth)::value;
    static int occ12 = 0, occ16 = 0, occ12g = 0, occ16g = 0;
    if (M > 16) {
      if (nch <= 4 * 12)
        return launch(w8a16_skinny_kernel<BF16, HAS_SCALE, 4, 12, 1, 3, BIAS, Epi, 2>, 4, occ12g);
      return launch(w8a16_skinny_kernel<BF16, HAS_SCALE, 4, kSkinnyMaxWaves, 1, 2, BIAS, Epi, 2>, 4,
                    occ16g);
    }
    if (nch <= 4 * 12)
      return launch(w8a16_skinny_kernel<BF16, HAS_SCALE, 4, 12, D, 6, BIAS, Epi>, 4, occ12);
    return launch(w8a16_skinny_kernel<BF16, HAS_SCALE, 4, kSkinnyMaxWaves, D, 4, BIAS, Epi>, 4, occ16);
  };
  auto with_depth = [&](auto bias_bits) {
    return deep ? pick(bias_bits, std::integral_constant<int, 2>{})
                : pick(bias_bits, std::integral_constant<int, 1>{});
  };
  if (!epi.bias) return with_depth(std::integral_constant<int, 0>{});
  if (epi.bias_dt == DT_F32) return with_depth(std::integral_constant<int, 32>{});
  return with_depth(std::integral_constant<int, 16>{});
}

// M in (32, 64] with N up to this many columns runs as two passes of the
// small-M kernel over the two row halves: the weights stream twice (the
// second time mostly from the Infinity Cache), which beats the few tiles
// the tiled route has for such M. Measured on MI355X, K = 3072, graph
// replays with weights rotated past the Infinity Cache, against the tiled
// route: N = 3072 1.42-1.77x, 6144 1.19-1.48x, 9216 1.01-1.29x, 12288
// 1.00-1.21x, 18432 0.80-0.96x (M = 64 ... 33).
constexpr int64_t kSkinnyTwoPassMaxN = 12288;

// EpiW8A16 has no row parameters, so a row range of the output is the same
// functor over an offset output pointer.
template <class Epi>
int run_w8a16(const void* a, int a_dtype, int64_t lda, const uint8_t* w, int64_t ldw,
              const float* w_scale, int64_t M, int64_t N, int64_t K, const Epi& epi, hipStream_t s,
              const char* what) {
  const bool bf16 = a_dtype == C4Q_BF16;
  // The skinny kernel addresses a 16-row weight block and the activation
  // rows with 32-bit buffer offsets.
  // (the small-M kernel reads the bias through the scalar cache: a 4-byte
  // aligned base)
  const bool skinny_ok = K > 0 && K <= kSkinnyMaxK && aligned16(a) &&
                         (epi.bias == nullptr || ((uintptr_t)epi.bias & 3) == 0) &&
                         aligned16(w) && lda % 8 == 0 && ldw % 16 == 0 &&
                         16 * ldw + 64 < (1ll << 31) && kSkinnyMaxM * 2 * lda + 256 < (1ll << 31);
  auto skinny = [&](const uint16_t* a16, int64_t m, const Epi& e) {
    if (bf16)
      return w_scale ? run_w8a16_skinny<true, true>(a16, lda, w, ldw, w_scale, m, N, K, e, s, what)
                     : run_w8a16_skinny<true, false>(a16, lda, w, ldw, w_scale, m, N, K, e, s, what);
    return w_scale ? run_w8a16_skinny<false, true>(a16, lda, w, ldw, w_scale, m, N, K, e, s, what)
                   : run_w8a16_skinny<false, false>(a16, lda, w, ldw, w_scale, m, N, K, e, s, what);
  };
  const uint16_t* a16 = static_cast<const uint16_t*>(a);
  if (skinny_ok && M <= kSkinnyMaxM) return skinny(a16, M, epi);
  if (skinny_ok && M <= 2 * kSkinnyMaxM && N <= kSkinnyTwoPassMaxN) {
    const int64_t h = M / 2;                      // both halves within kSkinnyMaxM rows
    using OutT = typename Epi::OutT;
    Epi hi = epi;
    hi.d = static_cast<uint8_t*>(epi.d) + h * epi.ldd * (int64_t)sizeof(OutT);
    hi.vec = rows_vec16(hi.d, epi.ldd, sizeof(OutT));
    const int st = skinny(a16, h, epi);
    if (st != C4Q_OK) return st;
    return skinny(a16 + h * lda, M - h, hi);
  }
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(w) && lda % 8 == 0 &&
                     ldw % 16 == 0 && tile_offsets_fit(2 * lda, ldw);
  if (!tiled) {
    GenW8A16 op{a16, lda, w, ldw, w_scale, bf16 ? 1 : 0, 1.0f};
    return launch_generic(M, N, K, op, epi, s, what);
  }
  if (bf16) {
    return w_scale ? run_w8a16_tiled<true, true>(a16, lda, w, ldw, w_scale, M, N, K, epi, s, what)
                   : run_w8a16_tiled<true, false>(a16, lda, w, ldw, w_scale, M, N, K, epi, s, what);
  }
  return w_scale ? run_w8a16_tiled<false, true>(a16, lda, w, ldw, w_scale, M, N, K, epi, s, what)
                 : run_w8a16_tiled<false, false>(a16, lda, w, ldw, w_scale, M, N, K, epi, s, what);
}
}  // namespace

extern "C" int c4q_w8a16_gemm_nt(const void* a, int a_dtype, int64_t lda, const uint8_t* w,
                                 int64_t ldw, const float* w_scale, void* d, int d_dtype,
                                 int64_t ldd, const void* bias, int bias_dtype,
                                 const uint16_t* act_table, int64_t M, int64_t N, int64_t K,
                                 void* stream) {
  const char* what = "c4q_w8a16_gemm_nt";
  C4Q_REQUIRE(M >= 0 && N >= 0 && K >= 0, C4Q_ERR_SHAPE, "%s: negative size", what);
  C4Q_REQUIRE(lda >= K && ldw >= K && ldd >= N, C4Q_ERR_SHAPE, "%s: row stride smaller than row",
              what);
  C4Q_REQUIRE(a_dtype == C4Q_BF16 || a_dtype == C4Q_F16, C4Q_ERR_ARG,
              "%s: activation must be bf16 or f16", what);
  C4Q_REQUIRE(valid_dt(d_dtype), C4Q_ERR_ARG, "%s: bad output dtype %d", what, d_dtype);
  C4Q_REQUIRE(!bias || valid_dt(bias_dtype), C4Q_ERR_ARG, "%s: bad bias dtype", what);
  C4Q_REQUIRE(!act_table || d_dtype == C4Q_BF16, C4Q_ERR_UNSUPPORTED,
              "%s: act_table needs a bf16 output", what);
  if (M == 0 || N == 0) return C4Q_OK;
  C4Q_REQUIRE(d && (K == 0 || (a && w)), C4Q_ERR_ARG, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  auto run = [&](auto out) {
    constexpr int OUT = decltype(out)::value;
    EpiW8A16<OUT> epi{{d, ldd, rows_vec16(d, ldd, OUT == DT_F32 ? 4 : 2)}, bias, bias_dtype,
                      act_table};
    return run_w8a16(a, a_dtype, lda, w, ldw, w_scale, M, N, K, epi, s, what);
  };
  if (d_dtype == C4Q_F32) return run(std::integral_constant<int, DT_F32>{});
  if (d_dtype == C4Q_F16) return run(std::integral_constant<int, DT_F16>{});
  return run(std::integral_constant<int, DT_BF16>{});
}
