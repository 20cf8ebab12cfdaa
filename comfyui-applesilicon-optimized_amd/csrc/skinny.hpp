// Small-M W8A16 linear (decode-time shapes, M <= 16): HBM-bound on the fp8
// weight stream, so the kernel is built to stream [N, K] fp8 weights at full
// bandwidth rather than to fill MFMA tiles.
//
//   * weight rows are taken in blocks of 16 (one v_mfma_f32_16x16x32 output
//     width); a persistent workgroup walks blocks b, b + G, b + 2G, ...;
//   * its waves split K (wavefront split-K): wave w owns the 64-element
//     chunks [w*CPW, (w+1)*CPW), which spreads the in-register dequantization
//     over every SIMD. Because M <= 16 the activation rows a wave needs are
//     the same for every block, so each wave loads its K-slice of them once
//     (rows >= M read zeros) and keeps it in registers;
//   * per chunk a lane loads one 16-byte run of fp8 codes of weight row
//     n0 + lane%16 at K offset 16 * (lane/16); one MFMA step consumes K values
//     16g + [0, 8) and the next 16g + [8, 16) for lane group g = lane/16 --
//     the same K permutation on both operands, hence the exact dot product;
//   * the weight runs of the next block are loaded (double buffer) before the
//     current block is multiplied, so every wave always has a block's worth
//     of loads in flight; a block's column parameters (bias) are loaded one
//     step before its epilogue, right after the next prefetch;
//   * each wave publishes its partial 16 x 16 tile (row-major) in LDS; after
//     the block barrier the 64 four-column groups of the tile are summed in
//     wave order (a fixed order: the result does not depend on timing) and
//     stored one block late, shared out over the waves, so no wave lags the
//     next barrier by a whole epilogue (the tile area is double-buffered).
// Weights are dequantized in registers exactly like the tiled kernel
// (dequant4: decode, optional kitchen scale, round to the activation type).
#pragma once
#include "gemm_tile.hpp"

namespace c4q {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
}

constexpr int kSkinnyMaxM = 16;
constexpr int kSkinnyMaxWaves = 16;
constexpr int kSkinnyMaxK = 64 * 4 * kSkinnyMaxWaves;  // 4 chunks per wave at most waves

// Clear fp8 codes (4 per word) / 16-bit activations (2 per word) at K
// positions >= K of a 16-element run starting at kb.
__device__ __forceinline__ void mask_codes(i32x4& q, int kb, int64_t K) {
  uint32_t a[4];
  __builtin_memcpy(a, &q, 16);
#pragma unroll
  for (int e = 0; e < 16; ++e)
    if (kb + e >= K) a[e >> 2] &= ~(0xFFu << (8 * (e & 3)));
  __builtin_memcpy(&q, a, 16);
}
__device__ __forceinline__ void mask_halves(i32x4& lo, i32x4& hi, int kb, int64_t K) {
  uint32_t a[8];
  __builtin_memcpy(a, &lo, 16);
  __builtin_memcpy(a + 4, &hi, 16);
#pragma unroll
  for (int e = 0; e < 16; ++e)
    if (kb + e >= K) a[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
  __builtin_memcpy(&lo, a, 16);
  __builtin_memcpy(&hi, a + 4, 16);
}

// CPW 64-element chunks per wave; blockDim.x = 64 * waves with
// waves * CPW >= cdiv(K, 64) and waves <= MAXW; at most 128 VGPRs per wave
// (four waves per SIMD).
template <bool BF16, bool HAS_SCALE, int CPW, int MAXW, class Epi>
__global__ void __launch_bounds__(64 * MAXW, 4)
w8a16_skinny_kernel(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw,
                    const float* w_scale, int64_t M, int64_t N, int64_t K, Epi epi) {
  static_assert(MAXW <= kSkinnyMaxWaves, "too many waves");
  __shared__ f32x4 red[2][MAXW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nch = (int)((K + 63) / 64);
  const int64_t nblk = (N + 15) / 16;
  const float ws = OpW8A16<BF16, HAS_SCALE>::prep_scale(w_scale);
  const Epi ep = epi.prepare();

  // Output group handled by this thread in the store phase: groups are the
  // 64 (row, 4-column) pieces of a 16 x 16 block, dealt over the waves.
  const int grp = lane * nwaves + wave;               // 0 .. 64*nwaves-1
  const bool has_grp = grp < 64;
  const int em = grp >> 2, ecq = (grp & 3) * 4;

  auto load_w = [&](int64_t blk, i32x4 (&q)[CPW]) {
    const int64_t n0 = blk * 16;
    const int64_t rows = N - n0 < 16 ? N - n0 : 16;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + n0 * ldw, rows * ldw);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave * CPW + j;
      q[j] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, c < nch ? (int)(r * ldw) + c * 64 + 16 * g : kOOB, 0, 0);
    }
  };
  // The first block's weights go out before the activation slice, so the two
  // latencies overlap.
  const int64_t G = gridDim.x;
  i32x4 q0[CPW], q1[CPW];
  int64_t blk = blockIdx.x;
  load_w(blk, q0);

  // this wave's K-slice of activation row r, kept in registers
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(reinterpret_cast<const uint8_t*>(x), M * ldx * 2);
  i32x4 xa[CPW], xb[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wave * CPW + j;
    const int kb = c * 64 + 16 * g;
    const bool live = c < nch && r < M;
    const int off = live ? (int)(r * ldx * 2) + 2 * kb : kOOB;
    xa[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
    xb[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, live ? off + 16 : kOOB, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int kb = (wave * CPW + j) * 64 + 16 * g;
    if (kb + 16 > K) mask_halves(xa[j], xb[j], kb, K);
  }

  // Multiply one block and publish the wave's partial tile (row-major,
  // m = 4*(lane/16) + i, c = lane%16), then meet at the block barrier.
  auto run_block = [&](i32x4 (&q)[CPW], int buf) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave * CPW + j;
      if (c >= nch) break;
      const int kb = c * 64 + 16 * g;
      if (kb + 16 > K) mask_codes(q[j], kb, K);
      uint32_t o[8];
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].x, ws, o[0], o[1]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].y, ws, o[2], o[3]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].z, ws, o[4], o[5]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].w, ws, o[6], o[7]);
      const i32x4 b0 = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      const i32x4 b1 = {(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
      acc = mfma16<BF16>(xa[j], b0, acc);
      acc = mfma16<BF16>(xb[j], b1, acc);
    }
    float* t = reinterpret_cast<float*>(&red[buf][wave][0]);
    t[(4 * g + 0) * 16 + r] = acc.x;
    t[(4 * g + 1) * 16 + r] = acc.y;
    t[(4 * g + 2) * 16 + r] = acc.z;
    t[(4 * g + 3) * 16 + r] = acc.w;
    stage_barrier();                 // LDS writes visible; weight prefetch stays in flight
  };
  // This thread's column parameters (bias) of a block.
  auto load_col = [&](int64_t blk) {
    typename Epi::Col c{};
    const int64_t n = blk * 16 + ecq;
    if (has_grp && em < M && n < N) c = ep.col(n, N - n < 4 ? (int)(N - n) : 4);
    return c;
  };
  // Sum the published tiles of a block in wave order and store this
  // thread's group.
  auto finish_block = [&](int64_t blk, int buf, const typename Epi::Col& col) {
    const int64_t n = blk * 16 + ecq;
    if (!has_grp || em >= M || n >= N) return;
    const int idx = em * 4 + (ecq >> 2);
    f32x4 sum = red[buf][0][idx];
#pragma unroll
    for (int wv = 1; wv < MAXW; ++wv)
      if (wv < nwaves) sum += red[buf][wv][idx];
    const float v[4] = {sum.x, sum.y, sum.z, sum.w};
    const int nv = N - n < 4 ? (int)(N - n) : 4;
    store_group(ep, em, n, nv, ep.apply(ep.rowp(em), col, v));
  };

  // Blocks blockIdx.x + i*G; the double buffers alternate by parity of i.
  // Step i: issue the weights of block i+1, finish block i-1 (its column
  // parameters were loaded in step i-1), load block i's column parameters,
  // multiply block i. Vector-memory counters complete in issue order, so the
  // epilogue then waits at most for block i's weights (which step i needs
  // anyway) and never for the prefetch just issued. The tile area of block
  // i-1 is rewritten at block i+1, after every wave passed block i's barrier
  // -- which each wave reaches only after finishing its share of block i-1.
  typename Epi::Col kc{};
  for (;;) {
    if (blk + G < nblk) load_w(blk + G, q1);
    if (blk != (int64_t)blockIdx.x) finish_block(blk - G, 1, kc);
    kc = load_col(blk);
    run_block(q0, 0);
    blk += G;
    if (blk >= nblk) {
      finish_block(blk - G, 0, kc);
      break;
    }
    if (blk + G < nblk) load_w(blk + G, q0);
    finish_block(blk - G, 0, kc);
    kc = load_col(blk);
    run_block(q1, 1);
    blk += G;
    if (blk >= nblk) {
      finish_block(blk - G, 1, kc);
      break;
    }
  }
}

}  // namespace c4q
