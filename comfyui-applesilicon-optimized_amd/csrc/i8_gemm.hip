// INT8 W8A8 entry points: raw int32, per-tensor and per-channel fused
// epilogues, and the fused gate/up FFN pair.
#include "launch.hpp"

using namespace c4q;

namespace {

int check_i8_args(const void* a, int64_t lda, const void* b, int64_t ldb, const void* d,
                  int64_t ldd, int64_t M, int64_t N, int64_t K, const char* what) {
  C4Q_REQUIRE(M >= 0 && N >= 0 && K >= 0, C4Q_ERR_SHAPE, "%s: negative size M=%lld N=%lld K=%lld",
              what, (long long)M, (long long)N, (long long)K);
  C4Q_REQUIRE(lda >= K && ldb >= K && ldd >= N, C4Q_ERR_SHAPE,
              "%s: row stride smaller than the row (lda=%lld ldb=%lld ldd=%lld)", what,
              (long long)lda, (long long)ldb, (long long)ldd);
  if (M > 0 && N > 0) {
    C4Q_REQUIRE(d != nullptr, C4Q_ERR_ARG, "%s: null output", what);
    C4Q_REQUIRE(K == 0 || (a != nullptr && b != nullptr), C4Q_ERR_ARG, "%s: null operand", what);
  }
  return C4Q_OK;
}

}  // namespace

extern "C" int c4q_i8_gemm_nt_i32(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                  int32_t* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                  void* stream) {
  const char* what = "c4q_i8_gemm_nt_i32";
  int st = check_i8_args(a, lda, b, ldb, c, ldc, M, N, K, what);
  if (st) return st;
  EpiI32 epi{{c, ldc, rows_vec16(c, ldc, 4)}};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                    uint16_t* d, int64_t ldd, const float* row_scale,
                                    const uint16_t* bias, int64_t M, int64_t N, int64_t K,
                                    void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || row_scale != nullptr, C4Q_ERR_ARG, "%s: null row_scale", what);
  EpiRowScale epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb,
                                       uint16_t* d, int64_t ldd, const float* row_scale,
                                       const float* col_scale, const uint16_t* bias, int64_t M,
                                       int64_t N, int64_t K, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || (row_scale != nullptr && col_scale != nullptr), C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  EpiRowColScale epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, col_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs_f16(const int8_t* a, int64_t lda, const int8_t* b,
                                           int64_t ldb, uint16_t* d, int64_t ldd,
                                           const float* row_scale, const float* col_scale,
                                           const uint16_t* bias, int64_t M, int64_t N, int64_t K,
                                           void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_f16";
  int st = check_i8_args(a, lda, b, ldb, d, ldd, M, N, K, what);
  if (st) return st;
  C4Q_REQUIRE(M == 0 || N == 0 || (row_scale != nullptr && col_scale != nullptr), C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  EpiRowColScaleF16 epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, col_scale, bias};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_gemm_nt_fused_cs_qkv(const int8_t* a, int64_t lda, const int8_t* b,
                                           int64_t ldb, uint16_t* q, uint16_t* k, uint16_t* v,
                                           const float* row_scale, const float* col_scale,
                                           const uint16_t* bias, int64_t M, int64_t K, int64_t H,
                                           int64_t D, void* stream) {
  const char* what = "c4q_i8_gemm_nt_fused_cs_qkv";
  C4Q_REQUIRE(H > 0 && D > 0 && D % 8 == 0, C4Q_ERR_SHAPE,
              "%s: need H > 0 and D > 0 a multiple of 8 (H=%lld D=%lld)", what, (long long)H,
              (long long)D);
  const int64_t N = 3 * H * D;
  C4Q_REQUIRE(N < (1ll << 31) && M < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
  int st = check_i8_args(a, lda, b, ldb, q, N, M, N, K, what);
  if (st) return st;
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(k != nullptr && v != nullptr, C4Q_ERR_ARG, "%s: null K/V output", what);
  C4Q_REQUIRE(row_scale != nullptr && col_scale != nullptr, C4Q_ERR_ARG,
              "%s: null row_scale/col_scale", what);
  const int vec = aligned16(q) && aligned16(k) && aligned16(v);
  const int64_t koff = (int64_t)(reinterpret_cast<intptr_t>(k) - reinterpret_cast<intptr_t>(q));
  const int64_t voff = (int64_t)(reinterpret_cast<intptr_t>(v) - reinterpret_cast<intptr_t>(q));
  EpiRowColScaleQKV epi{{{q, N, vec}, row_scale, col_scale, bias}, koff, voff, M,
                        (uint32_t)(H * D), (uint32_t)D};
  return run_gemm8<OpI8T, GenI8>(reinterpret_cast<const uint8_t*>(a), lda,
                                 reinterpret_cast<const uint8_t*>(b), ldb, M, N, K, epi,
                                 as_stream(stream), what);
}

extern "C" int c4q_i8_ffn_pair(const int8_t* a, int64_t lda, const int8_t* w_gate,
                               const int8_t* w_up, int64_t ldw, uint16_t* d, int64_t ldd,
                               const float* row_scale, const float* gate_scale,
                               const float* up_scale, const uint16_t* table_gate,
                               const uint16_t* table_up, int64_t M, int64_t N_out, int64_t K,
                               void* stream) {
  const char* what = "c4q_i8_ffn_pair";
  int st = check_i8_args(a, lda, w_gate, ldw, d, ldd, M, N_out, K, what);
  if (st) return st;
  if (M == 0 || N_out == 0) return C4Q_OK;
  C4Q_REQUIRE(K == 0 || w_up != nullptr, C4Q_ERR_ARG, "%s: null w_up", what);
  C4Q_REQUIRE(row_scale && gate_scale && up_scale, C4Q_ERR_ARG, "%s: null scale", what);
  hipStream_t s = as_stream(stream);
  EpiPair epi{{d, ldd, rows_vec16(d, ldd, 2)}, row_scale, gate_scale, up_scale, table_gate, table_up};
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(w_gate) &&
                     aligned16(w_up) && lda % 16 == 0 && ldw % 16 == 0 && tile_offsets_fit(lda, ldw);
  if (!tiled) {
    const int64_t nbx = cdiv(N_out, 64);
    const int64_t blocks = nbx * cdiv(M, 4);
    C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
    hipLaunchKernelGGL((pair_generic_kernel<EpiPair>), dim3((unsigned)blocks), dim3(256), 0, s, M,
                       N_out, K, nbx, a, lda, w_gate, w_up, ldw, epi);
    return check_launch(what);
  }
  const Src2 sa{reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(a), lda, M};
  const Src2 sb{reinterpret_cast<const uint8_t*>(w_gate), reinterpret_cast<const uint8_t*>(w_up),
                ldw, N_out};
  return run_tiles<true>(M, 2 * N_out, 2 * N_out, K, sa, sb, nullptr, epi, s, what,
                         [](auto t) { return OpI8T<decltype(t)::KS8>{}; });
}
