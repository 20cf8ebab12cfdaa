// bf16 x bf16 fused FC1/SiTU FFN pair (MOSS on bf16 weights).
#include "launch.hpp"

using namespace c4q;

extern "C" int c4q_bf16_ffn_pair(const uint16_t* a, int64_t lda, const uint16_t* w_hidden,
                                 const uint16_t* w_gate, int64_t ldw, uint16_t* d, int64_t ldd,
                                 const uint16_t* table_hidden, const uint16_t* table_gate,
                                 int64_t M, int64_t N_out, int64_t K, void* stream) {
  const char* what = "c4q_bf16_ffn_pair";
  C4Q_REQUIRE(M >= 0 && N_out >= 0 && K >= 0, C4Q_ERR_SHAPE,
              "%s: negative size M=%lld N_out=%lld K=%lld", what, (long long)M, (long long)N_out,
              (long long)K);
  C4Q_REQUIRE(lda >= K && ldw >= K && ldd >= N_out, C4Q_ERR_SHAPE,
              "%s: row stride smaller than the row (lda=%lld ldw=%lld ldd=%lld)", what,
              (long long)lda, (long long)ldw, (long long)ldd);
  if (M == 0 || N_out == 0) return C4Q_OK;
  C4Q_REQUIRE(d != nullptr, C4Q_ERR_ARG, "%s: null output", what);
  C4Q_REQUIRE(K == 0 || (a != nullptr && w_hidden != nullptr && w_gate != nullptr), C4Q_ERR_ARG,
              "%s: null operand", what);
  hipStream_t s = as_stream(stream);
  EpiPairF epi{{d, ldd, rows_vec16(d, ldd, 2)}, table_hidden, table_gate};
  // 16-byte copies: rows of whole 8-element chunks, 16-byte aligned
  const bool tiled = K > 0 && K % 8 == 0 && aligned16(a) && aligned16(w_hidden) &&
                     aligned16(w_gate) && lda % 8 == 0 && ldw % 8 == 0 &&
                     tile_offsets_fit(lda * 2, ldw * 2);
  if (!tiled) {
    const int64_t nbx = cdiv(N_out, 64);
    const int64_t blocks = nbx * cdiv(M, 4);
    C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large", what);
    hipLaunchKernelGGL((pair_generic_bf16_kernel<EpiPairF>), dim3((unsigned)blocks), dim3(256), 0,
                       s, M, N_out, K, nbx, a, lda, w_hidden, w_gate, ldw, epi);
    return check_launch(what);
  }
  const Src2 sa{reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(a), lda * 2, M};
  const Src2 sb{reinterpret_cast<const uint8_t*>(w_hidden), reinterpret_cast<const uint8_t*>(w_gate),
                ldw * 2, N_out};
  return run_tiles<true>(M, 2 * N_out, 2 * N_out, K, sa, sb, nullptr, epi, s, what,
                         [](auto) { return OpBF16T{}; });
}
