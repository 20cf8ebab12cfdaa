// Shape-agnostic fallback kernels: any M, N, K, any row stride, any
// alignment. One thread per output element, K walked sequentially. They run
// when a call does not meet the tiled kernels' layout contract (16-byte
// aligned rows, K a multiple of 16) and share the epilogue functors, so the
// stored arithmetic is identical; only the speed differs.
#pragma once
#include "epilogues.hpp"
#include "numerics.hpp"

namespace c4q {

// Operand readers.
struct GenI8 {
  using Acc = int32_t;
  const int8_t* a; int64_t lda; const int8_t* b; int64_t ldb;
  static GenI8 make(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb) {
    return {reinterpret_cast<const int8_t*>(a), lda, reinterpret_cast<const int8_t*>(b), ldb};
  }
  __device__ __forceinline__ int32_t av(int64_t m, int64_t k) const { return a[m * lda + k]; }
  __device__ __forceinline__ int32_t bv(int64_t n, int64_t k) const { return b[n * ldb + k]; }
};
struct GenF8 {
  using Acc = float;
  const uint8_t* a; int64_t lda; const uint8_t* b; int64_t ldb;
  static GenF8 make(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb) {
    return {a, lda, b, ldb};
  }
  __device__ __forceinline__ float av(int64_t m, int64_t k) const { return e4m3_f32(a[m * lda + k]); }
  __device__ __forceinline__ float bv(int64_t n, int64_t k) const { return e4m3_f32(b[n * ldb + k]); }
};
// W8A16: bf16/f16 activation, fp8 weight dequantized to the activation
// type: T(decode(code) * T(scale)) (kitchen formula), or the plain decode.
struct GenW8A16 {
  using Acc = float;
  const uint16_t* a; int64_t lda; const uint8_t* b; int64_t ldb; const float* sp; int bf16;
  float s;
  __device__ __forceinline__ float av(int64_t m, int64_t k) const {
    uint16_t h = a[m * lda + k];
    return bf16 ? bf16_f32(h) : f16_f32(h);
  }
  __device__ __forceinline__ float bv(int64_t n, int64_t k) const {
    float w = e4m3_f32(b[n * ldb + k]);
    if (sp) w = w * s;
    return bf16 ? bf16_f32(bf16_rte(w)) : f16_f32(f16_rte(w));
  }
  __device__ __forceinline__ void prepare() {
    if (sp) s = bf16 ? bf16_f32(bf16_rte(sp[0])) : f16_f32(f16_rte(sp[0]));
  }
};

template <class Op>
__device__ __forceinline__ void gen_prepare(Op&) {}
template <>
__device__ __forceinline__ void gen_prepare<GenW8A16>(GenW8A16& op) { op.prepare(); }

// 1-D grid of cdiv(N,64) x cdiv(M,4) blocks (nbx = cdiv(N,64)); every block
// covers 4 rows x 64 columns.
template <class Op, class Epi>
__global__ void __launch_bounds__(256)
gemm_generic_kernel(int64_t M, int64_t N, int64_t K, int64_t nbx, Op op, Epi epi) {
  const int64_t bx = (int64_t)blockIdx.x % nbx, by = (int64_t)blockIdx.x / nbx;
  const int64_t n = bx * 64 + (threadIdx.x & 63);
  const int64_t m = by * 4 + (threadIdx.x >> 6);
  if (m >= M || n >= N) return;
  gen_prepare(op);
  const Epi ep = epi.prepare();
  typename Op::Acc acc = 0;
  for (int64_t k = 0; k < K; ++k) acc = acc + op.av(m, k) * op.bv(n, k);
  const typename Op::Acc v[4] = {acc, 0, 0, 0};
  store_group(ep, m, n, 1, ep.value4(m, n, v, 1));
}

// FFN pair fallback: gate/up accumulators for output column `col`.
template <class Epi>
__global__ void __launch_bounds__(256)
pair_generic_kernel(int64_t M, int64_t NC, int64_t K, int64_t nbx, const int8_t* a, int64_t lda,
                    const int8_t* g, const int8_t* u, int64_t ldw, Epi epi) {
  const int64_t bx = (int64_t)blockIdx.x % nbx, by = (int64_t)blockIdx.x / nbx;
  const int64_t col = bx * 64 + (threadIdx.x & 63);
  const int64_t m = by * 4 + (threadIdx.x >> 6);
  if (m >= M || col >= NC) return;
  const Epi ep = epi.prepare();
  int32_t ag = 0, au = 0;
  for (int64_t k = 0; k < K; ++k) {
    const int32_t x = a[m * lda + k];
    ag += x * (int32_t)g[col * ldw + k];
    au += x * (int32_t)u[col * ldw + k];
  }
  const int32_t gv[4] = {ag, 0, 0, 0}, uv[4] = {au, 0, 0, 0};
  store_group(ep, m, col, 1, ep.pair4(m, col, gv, uv, 1));
}

// bf16 FFN pair fallback (MOSS bf16 FC1): fp32 sums in K order, each
// product and sum rounded on its own.
template <class Epi>
__global__ void __launch_bounds__(256)
pair_generic_bf16_kernel(int64_t M, int64_t NC, int64_t K, int64_t nbx, const uint16_t* a,
                         int64_t lda, const uint16_t* g, const uint16_t* u, int64_t ldw, Epi epi) {
  const int64_t bx = (int64_t)blockIdx.x % nbx, by = (int64_t)blockIdx.x / nbx;
  const int64_t col = bx * 64 + (threadIdx.x & 63);
  const int64_t m = by * 4 + (threadIdx.x >> 6);
  if (m >= M || col >= NC) return;
  const Epi ep = epi.prepare();
  float ag = 0.0f, au = 0.0f;
  for (int64_t k = 0; k < K; ++k) {
    const float x = bf16_f32(a[m * lda + k]);
    ag = ag + x * bf16_f32(g[col * ldw + k]);
    au = au + x * bf16_f32(u[col * ldw + k]);
  }
  const float gv[4] = {ag, 0.0f, 0.0f, 0.0f}, uv[4] = {au, 0.0f, 0.0f, 0.0f};
  store_group(ep, m, col, 1, ep.pair4(m, col, gv, uv, 1));
}

}  // namespace c4q
