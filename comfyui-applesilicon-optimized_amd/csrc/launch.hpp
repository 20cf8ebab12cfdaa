// Launch helpers binding the tiled and generic kernels to an entry point.
#pragma once
#include "api_common.hpp"
#include "epilogues.hpp"
#include "gemm_tile.hpp"
#include "generic.hpp"

namespace c4q {

template <class Mma, int BM, int BN, class LoadA, class SrcA, class LoadB, class SrcB, class BSt,
          bool PAIR, class Epi>
int launch_tile(GemmShape sh, int64_t n_rows_b, const SrcA& sa, const SrcB& sb, const BSt& bst,
                const Epi& epi, hipStream_t s, const char* what) {
  sh.tiles_m = (int)cdiv(sh.M, BM);
  sh.tiles_n = (int)cdiv(n_rows_b, BN);
  const int64_t blocks = (int64_t)sh.tiles_m * sh.tiles_n;
  C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: problem too large (%lld tiles)", what,
              (long long)blocks);
  hipLaunchKernelGGL((gemm_tile_kernel<Mma, BM, BN, LoadA, SrcA, LoadB, SrcB, BSt, PAIR, Epi>),
                     dim3((unsigned)blocks), dim3(kThreads), 0, s, sh, sa, sb, bst, epi);
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

// 8-bit x 8-bit GEMM (int8 or fp8 operands) with epilogue Epi.
template <class Mma, class GenOp, class Epi>
int run_gemm8(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, int64_t M, int64_t N,
              int64_t K, const Epi& epi, hipStream_t s, const char* what) {
  if (M == 0 || N == 0) return C4Q_OK;
  const bool tiled = K > 0 && K % 16 == 0 && aligned16(a) && aligned16(b) && lda % 16 == 0 &&
                     ldb % 16 == 0;
  if (!tiled) {
    return launch_generic(M, N, K, GenOp::make(a, lda, b, ldb), epi, s, what);
  }
  GemmShape sh{M, N, K, K, K, 0, 0};
  RowsPlain ra{a, lda, M}, rb{b, ldb, N};
  switch (pick_tile(M, N)) {
    case TILE_256x256:
      return launch_tile<Mma, 256, 256, Load8<256, RowsPlain>, RowsPlain, Load8<256, RowsPlain>,
                         RowsPlain, BStorePlain, false>(sh, N, ra, rb, BStorePlain{}, epi, s, what);
    case TILE_128x128:
      return launch_tile<Mma, 128, 128, Load8<128, RowsPlain>, RowsPlain, Load8<128, RowsPlain>,
                         RowsPlain, BStorePlain, false>(sh, N, ra, rb, BStorePlain{}, epi, s, what);
    default:
      return launch_tile<Mma, 64, 128, Load8<64, RowsPlain>, RowsPlain, Load8<128, RowsPlain>,
                         RowsPlain, BStorePlain, false>(sh, N, ra, rb, BStorePlain{}, epi, s, what);
  }
}

}  // namespace c4q
