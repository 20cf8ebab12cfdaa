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
//   * the weights of D blocks are in flight per wave (a D-deep register
//     pipeline: block i+D-1 is issued as block i is multiplied), which is
//     what it takes to cover the HBM latency under full load (about 3 us, one
//     block's streaming time being about 2 us per CU); a block's column
//     parameters (bias) are loaded right behind its weights, so the epilogue
//     of block i-1 never waits on a newer prefetch (memory counters complete
//     in issue order);
//   * each wave publishes its partial 16 x 16 tile (row-major) in LDS and
//     goes on to the next block: one workgroup barrier closes a group of up
//     to P blocks, after which every thread sums one (row, four-column)
//     piece of the group over the waves in wave order (a fixed order: the
//     result does not depend on timing) and stores it. A barrier per block
//     would make every wave wait out the slowest one each block; the group
//     areas are double-buffered.
// Weights are dequantized in registers exactly like the tiled kernel
// (dequant4: decode, optional kitchen scale, round to the activation type).
//
// MG = 2 takes M <= 32 as two 16-row activation groups (the reference runs
// a separate small-M pipeline up to M = 64,
// _patches/fp8s_ext/w8a16_gemm.mm:215-220): each wave keeps both groups'
// K-slices in registers, every dequantized weight chunk feeds the MFMAs of
// both groups, and the partial tiles and the per-group sums double (half as
// many blocks per barrier, so the partial-tile area stays the same size).
// The weight stream, which bounds the kernel, is read once.
#pragma once
#include "gemm_tile.hpp"

namespace c4q {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
}

// Steps i0 + B, B = 0 .. D-1, while i0 + B < nb, with the buffer index B a
// constant (register arrays are only indexed statically).
template <int B, int D, class F>
__device__ __forceinline__ void unroll_steps(F& f, int64_t i0, int64_t nb) {
  if constexpr (B < D) {
    if (i0 + B < nb) {
      f(std::integral_constant<int, B>{}, i0 + B);
      unroll_steps<B + 1, D>(f, i0, nb);
    }
  }
}

constexpr int kSkinnyMaxM = 32;      // 16-row activation groups: one, or two (MG = 2)
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
// waves * CPW >= cdiv(K, 64) and waves <= MAXW; D blocks of weights in
// flight; partial tiles of up to P blocks between workgroup barriers. One
// workgroup per CU: MAXW / 4 waves per SIMD, so 512 / (MAXW / 4) VGPRs per
// wave (16 waves: 128; 12 waves: 168).
// BIAS: 0 none, 16 a bf16/f16 bias, 32 an f32 bias (Epi = EpiW8A16).
template <bool BF16, bool HAS_SCALE, int CPW, int MAXW, int D, int P, int BIAS, class Epi,
          int MG = 1>
__global__ void __launch_bounds__(64 * MAXW, MAXW / 4)
w8a16_skinny_kernel(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw,
                    const float* w_scale, int64_t M, int64_t N, int64_t K, Epi epi) {
  static_assert(MAXW <= kSkinnyMaxWaves && MAXW % 4 == 0, "whole waves per SIMD");
  static_assert(D >= 1 && P >= 1, "pipeline shape");
  static_assert(MG == 1 || MG == 2, "one or two 16-row activation groups");
  __shared__ f32x4 red[2][P][MG][MAXW][64];    // partial tiles of two groups of blocks
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nch = (int)((K + 63) / 64);
  const int64_t nblk = (N + 15) / 16;
  const float ws = OpW8A16<BF16, HAS_SCALE>::prep_scale(w_scale);
  const Epi ep = epi.prepare();

  // This workgroup's blocks are blockIdx.x + i*G, i < nb (the grid never
  // exceeds the block count), taken in groups of pg blocks.
  const int64_t G = gridDim.x;
  const int64_t nb = (nblk - 1 - (int64_t)blockIdx.x) / G + 1;
  const int pg = nwaves < P ? nwaves : P;
  // The output piece this thread stores for each group: block slot
  // threadIdx.x / 64 of the group, row em and columns ecq .. ecq+3 of it.
  const int pslot = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);   // the wave: uniform
  const int pe = (int)threadIdx.x & 63;
  const int em = pe >> 2, ecq = (pe & 3) * 4;

  auto load_w = [&](int64_t blk, i32x4 (&q)[CPW]) {
    const int64_t n0 = blk * 16;
    const int64_t rows = N - n0 < 0 ? 0 : (N - n0 < 16 ? N - n0 : 16);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + n0 * ldw, rows * ldw);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave * CPW + j;
      q[j] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, c < nch ? (int)(r * ldw) + c * 64 + 16 * g : kOOB, 0, 0);
    }
  };
  i32x4 qb[D][CPW];
  // Every step issues the same CPW loads -- past the last block they read
  // zeros out of range -- so the compiler can count the loads in flight
  // exactly; with a conditional prefetch it assumes the shortest path and
  // waits for the prefetch it just issued.
  auto fetch = [&](int64_t i, i32x4 (&q)[CPW]) {
    load_w((int64_t)blockIdx.x + (i < nb ? i : nb) * G, q);
  };
  // The first block's weights go out before the activation slice, so the two
  // latencies overlap (D = 1: each step loads its own block).
  if constexpr (D >= 2) fetch(0, qb[0]);

  // this wave's K-slice of activation rows r (+ 16 per group), kept in
  // registers
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(reinterpret_cast<const uint8_t*>(x), M * ldx * 2);
  i32x4 xa[MG][CPW], xb[MG][CPW];
#pragma unroll
  for (int mg = 0; mg < MG; ++mg)
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave * CPW + j;
      const int kb = c * 64 + 16 * g;
      const int row = r + 16 * mg;
      const bool live = c < nch && row < M;
      const int off = live ? (int)(row * ldx * 2) + 2 * kb : kOOB;
      xa[mg][j] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
      xb[mg][j] = __builtin_amdgcn_raw_buffer_load_b128(xr, live ? off + 16 : kOOB, 0, 0);
    }
  // K tail: only a wave whose slice runs past K masks (a wave-uniform test --
  // a per-lane one would make every wave wait here for its activation
  // loads, and behind them for the first block's weights, before the rest
  // of the prologue prefetch goes out)
  if ((wave + 1) * CPW * 64 > K) {
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int kb = (wave * CPW + j) * 64 + 16 * g;
        if (kb + 16 > K) mask_halves(xa[mg][j], xb[mg][j], kb, K);
      }
  }
#pragma unroll
  for (int p = 1; p < D - 1; ++p) fetch(p, qb[p]);

  // Multiply one block and publish the wave's partial tile (row-major,
  // m = 4*(lane/16) + i, c = lane%16) -- no barrier per block.
  auto run_block = [&](i32x4 (&q)[CPW], int buf, int slot) {
    f32x4 acc[MG];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) acc[mg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = wave * CPW + j;
      if (c >= nch) break;
      const int kb = c * 64 + 16 * g;
      if ((c + 1) * 64 > K && kb + 16 > K) mask_codes(q[j], kb, K);
      uint32_t o[8];
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].x, ws, o[0], o[1]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].y, ws, o[2], o[3]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].z, ws, o[4], o[5]);
      dequant4<BF16, HAS_SCALE>((uint32_t)q[j].w, ws, o[6], o[7]);
      const i32x4 b0 = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      const i32x4 b1 = {(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) {
        acc[mg] = mfma16<BF16>(xa[mg][j], b0, acc[mg]);
        acc[mg] = mfma16<BF16>(xb[mg][j], b1, acc[mg]);
      }
    }
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      float* t = reinterpret_cast<float*>(&red[buf][slot][mg][wave][0]);
      t[(4 * g + 0) * 16 + r] = acc[mg].x;
      t[(4 * g + 1) * 16 + r] = acc[mg].y;
      t[(4 * g + 2) * 16 + r] = acc[mg].z;
      t[(4 * g + 3) * 16 + r] = acc[mg].w;
    }
  };
  // Bias of this thread's four columns of block blk. The block's 16
  // bias values are wave-uniform (a wave stores the pieces of one block), so
  // they come through the scalar cache: scalar loads complete on their own
  // counter, and waiting for them never waits for the weight prefetch in
  // flight (the base is 4-byte aligned -- checked on the host; values past
  // N read as zero). The wait sits inside the same statement, so no other
  // scalar-counter wait of the compiler's can see the load outstanding.
  const u32x4 bsr = dma_rsrc(static_cast<const uint8_t*>(ep.bias), BIAS ? N * (BIAS / 8) : 0);
  auto block_col = [&](int64_t blk) {
    typename Epi::Col c{};
    if constexpr (BIAS != 0) {
      const int off = __builtin_amdgcn_readfirstlane((int)(blk * 16 * (BIAS / 8)));
      uint32_t v[16];
      if constexpr (BIAS == 32) {
        u32x16 d;
        asm volatile("s_buffer_load_dwordx16 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                     : "=s"(d) : "s"(bsr), "s"(off) : "memory");
#pragma unroll
        for (int t = 0; t < 16; ++t) v[t] = d[t];
      } else {
        u32x8 d;
        asm volatile("s_buffer_load_dwordx8 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                     : "=s"(d) : "s"(bsr), "s"(off) : "memory");
#pragma unroll
        for (int t = 0; t < 16; ++t) v[t] = (d[t >> 1] >> (16 * (t & 1))) & 0xFFFFu;
      }
      const int sel = ecq >> 2;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        c.b[q] = raw_f32(sel == 0 ? v[q] : sel == 1 ? v[4 + q] : sel == 2 ? v[8 + q] : v[12 + q],
                         ep.bias_dt);
    }
    return c;
  };
  // After the group's barrier: sum this thread's piece over the waves in
  // wave order (a fixed order: the result does not depend on timing) and
  // store it.
  auto finish_group = [&](int64_t gi, int buf) {
    const int64_t i = gi * pg + pslot;
    if (pslot >= pg || i >= nb) return;                 // wave-uniform
    const typename Epi::Col col = block_col((int64_t)blockIdx.x + i * G);
    const int64_t n = ((int64_t)blockIdx.x + i * G) * 16 + ecq;
    if (n >= N) return;
    const int idx = em * 4 + (ecq >> 2);
    const int nv = N - n < 4 ? (int)(N - n) : 4;
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      const int row = em + 16 * mg;
      if (row >= M) break;
      f32x4 sum = red[buf][pslot][mg][0][idx];
#pragma unroll
      for (int wv = 1; wv < MAXW; ++wv) {
        if (wv < nwaves) sum += red[buf][pslot][mg][wv][idx];
        if ((wv & 3) == 3) __builtin_amdgcn_sched_barrier(0);   // four tiles in flight at most
      }
      const float v[4] = {sum.x, sum.y, sum.z, sum.w};
      store_group(ep, row, n, nv, ep.apply(ep.rowp(row), col, v));
    }
  };

  // Step i (weight buffer B = i % D, group gi = i / pg, slot i % pg): issue
  // block i+D-1 into the buffer block i-1 used, multiply block i; after the
  // group's last block, meet at the barrier and store the group. Group gi's tile area
  // (parity gi & 1) is rewritten by group gi+2, whose first writes follow the
  // barrier closing group gi+1 -- which each wave reaches only after storing
  // its piece of group gi.
  static_assert(BIAS == 0 || sizeof(typename Epi::Col) == 16, "bias of four columns");
  auto step = [&](auto bconst, int64_t i) {
    constexpr int B = decltype(bconst)::value;
    constexpr int PB = (B + D - 1) % D;
    fetch(i + D - 1, qb[PB]);
    const int64_t gi = i / pg;
    const int slot = (int)(i - gi * pg), buf = (int)(gi & 1);
    run_block(qb[B], buf, slot);
    if (slot == pg - 1 || i == nb - 1) {
      stage_barrier();
      finish_group(gi, buf);
    }
  };
  for (int64_t i0 = 0; i0 < nb; i0 += D) unroll_steps<0, D>(step, i0, nb);
}

}  // namespace c4q
