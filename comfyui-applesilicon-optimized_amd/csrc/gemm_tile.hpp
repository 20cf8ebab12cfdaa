// LDS-tiled MFMA GEMM core for gfx950 (CDNA4), NT layout:
//
//     D[m, n] = epilogue( sum_k A[m, k] * B[n, k] )
//
// A is the activation [M, K] and B the weight in its stored nn.Linear
// layout [N, K]; both are K-contiguous, which is the operand order every
// MFMA wants, so neither is ever transposed.
//
// Structure (one workgroup = 4 wave64s in a 2x2 arrangement):
//   * the workgroup owns a BM x BN output tile; each wave a (BM/2) x (BN/2)
//     sub-tile built from 32x32 MFMA blocks held in accumulator registers;
//   * K advances in stages of 128 bytes per tile row (128 int8/fp8 values,
//     or 64 bf16/f16 values). Each stage is staged through LDS with 16-byte
//     global loads (a wave reads whole 128-byte rows) and double buffered:
//     the loads of stage k+1 are in flight while stage k feeds the MFMAs,
//     one barrier per stage;
//   * LDS rows are 128 bytes with the 16-byte chunks XOR-swizzled by row so
//     that the MFMA fragment reads (32 rows, one chunk) hit distinct banks;
//   * workgroup ids are remapped so that each of the 8 XCDs owns a
//     contiguous run of tiles, walked in GROUP_M-row bands, keeping the A
//     and B panels a band shares inside that XCD's L2.
//
// Operand policies supply the MFMA (int8 32x32x32, fp8 32x32x64 f8f6f4,
// bf16/f16 32x32x16); stage loaders supply the global->LDS copy (including
// the fp8->bf16 dequant of W8A16 weights and the gate/up row pairing of the
// FFN-pair kernel); epilogue functors consume the accumulators.
#pragma once
#include "numerics.hpp"

namespace c4q {

typedef int      i32x4  __attribute__((ext_vector_type(4)));
typedef int      i32x8  __attribute__((ext_vector_type(8)));
typedef int      i32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x2  __attribute__((ext_vector_type(2)));
typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16   bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2  __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kRowBytes = 128;       // LDS bytes per tile row per stage
constexpr int kGroupM = 8;           // tile rows per raster band

template <class T, class F>
__device__ __forceinline__ T bitcast(const F& f) { return __builtin_bit_cast(T, f); }

// physical 16-byte chunk of logical chunk c in LDS row r
__device__ __forceinline__ int swz_chunk(int r, int c) { return c ^ (r & 7); }

// ---------------------------------------------------------------- MFMA ---
struct MmaI8 {
  using Acc = i32x16;
  using Scalar = int32_t;
  static constexpr int kChunks = 1;           // 16-byte chunks per lane fragment
  __device__ static Acc mma(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], b[0], c, 0, 0, 0);
  }
};
struct MmaF8 {                                 // OCP e4m3 x e4m3, fp32 accumulate
  using Acc = f32x16;
  using Scalar = float;
  static constexpr int kChunks = 2;
  __device__ static Acc mma(const i32x4* a, const i32x4* b, Acc c) {
    i32x8 av = {a[0].x, a[0].y, a[0].z, a[0].w, a[1].x, a[1].y, a[1].z, a[1].w};
    i32x8 bv = {b[0].x, b[0].y, b[0].z, b[0].w, b[1].x, b[1].y, b[1].z, b[1].w};
    // cbsz = blgp = 0 select e4m3 for both operands; zero scales select the
    // unscaled multiply.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 0, 0, 0);
  }
};
struct MmaBF16 {
  using Acc = f32x16;
  using Scalar = float;
  static constexpr int kChunks = 1;
  __device__ static Acc mma(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a[0]), bitcast<bf16x8>(b[0]), c, 0, 0, 0);
  }
};
struct MmaF16 {
  using Acc = f32x16;
  using Scalar = float;
  static constexpr int kChunks = 1;
  __device__ static Acc mma(const i32x4* a, const i32x4* b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a[0]), bitcast<f16x8>(b[0]), c, 0, 0, 0);
  }
};

// ------------------------------------------------------- stage loaders ---
// Row sources map a tile row to a global row pointer (already clamped into
// range: rows past the end re-read the last row; their results are never
// stored).
struct RowsPlain {
  const uint8_t* base; int64_t ld_bytes; int64_t rows;
  __device__ __forceinline__ const uint8_t* row(int64_t r) const {
    return base + (r < rows ? r : rows - 1) * ld_bytes;
  }
};
// FFN pair: in the doubled-N space every 32-row MFMA block alternates
// between gate rows (even blocks) and up rows (odd blocks) of the same 32
// output columns, so one lane ends up holding gate and up accumulators of
// the same (m, col).
struct RowsPair {
  const uint8_t* gate; const uint8_t* up; int64_t ld_bytes; int64_t rows;  // rows = N_out
  __device__ __forceinline__ const uint8_t* row(int64_t r2) const {
    int64_t blk = r2 >> 5;
    int64_t col = ((blk >> 1) << 5) + (r2 & 31);
    col = col < rows ? col : rows - 1;
    return ((blk & 1) ? up : gate) + col * ld_bytes;
  }
};

// Copies ROWS x 128 bytes per stage; every thread owns ROWS/32 chunks of
// 16 bytes (row = tid/8 + 32 i, chunk = tid % 8). K is masked at 16-byte
// granularity (chunks at or past k_bytes load zeros).
template <int ROWS, class Src>
struct Load8 {
  static constexpr int kN = ROWS * 8 / kThreads;
  i32x4 v[kN];
  __device__ __forceinline__ void load(const Src& src, int64_t r0, int64_t kb0, int64_t k_bytes) {
    const int tid = threadIdx.x;
    const int c = tid & 7;
    const int64_t kb = kb0 + c * 16;
    const bool ok = kb < k_bytes;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int r = (tid >> 3) + 32 * i;
      if (ok) v[i] = *reinterpret_cast<const i32x4*>(src.row(r0 + r) + kb);
      else v[i] = i32x4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
    const int tid = threadIdx.x;
    const int c = tid & 7;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int r = (tid >> 3) + 32 * i;
      *reinterpret_cast<i32x4*>(lds + r * kRowBytes + swz_chunk(r, c) * 16) = v[i];
    }
  }
};

// fp8 e4m3fn -> bf16/f16 dequantization of one packed word (4 codes) into
// two 32-bit words of 2 halves each:  out = T(decode(code) * scale), where
// scale is the per-tensor weight scale already rounded to T (the kitchen
// dequant formula x.to(T) * scale.to(T)); HAS_SCALE = false is the exact
// plain decode of an unscaled fp8 weight.
template <bool BF16, bool HAS_SCALE>
__device__ __forceinline__ void dequant4(uint32_t w, float s, uint32_t& lo, uint32_t& hi) {
  f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  if (HAS_SCALE) { a.x *= s; a.y *= s; b.x *= s; b.y *= s; }
  if (BF16) {
    bf16x2 ha = {(__bf16)a.x, (__bf16)a.y};
    bf16x2 hb = {(__bf16)b.x, (__bf16)b.y};
    lo = bitcast<uint32_t>(ha); hi = bitcast<uint32_t>(hb);
  } else {
    f16x2 ha = {(_Float16)a.x, (_Float16)a.y};
    f16x2 hb = {(_Float16)b.x, (_Float16)b.y};
    lo = bitcast<uint32_t>(ha); hi = bitcast<uint32_t>(hb);
  }
}

// W8A16 weight stage: 64 fp8 values (64 bytes) per row per stage expand to
// 64 halves (128 LDS bytes). Every thread owns ROWS/64 source chunks of 16
// codes (row = tid/4 + 64 i, source chunk = tid % 4 -> LDS chunks 2c, 2c+1).
template <int ROWS, bool BF16, bool HAS_SCALE>
struct LoadW8 {
  static constexpr int kN = ROWS * 4 / kThreads;
  i32x4 v[kN];
  __device__ __forceinline__ void load(const RowsPlain& src, int64_t r0, int64_t kb0, int64_t k_bytes) {
    const int tid = threadIdx.x;
    const int c = tid & 3;
    const int64_t kb = kb0 + c * 16;
    const bool ok = kb < k_bytes;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int r = (tid >> 2) + 64 * i;
      if (ok) v[i] = *reinterpret_cast<const i32x4*>(src.row(r0 + r) + kb);
      else v[i] = i32x4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds, float s) const {
    const int tid = threadIdx.x;
    const int c = tid & 3;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      const int r = (tid >> 2) + 64 * i;
      uint32_t o[8];
      dequant4<BF16, HAS_SCALE>((uint32_t)v[i].x, s, o[0], o[1]);
      dequant4<BF16, HAS_SCALE>((uint32_t)v[i].y, s, o[2], o[3]);
      dequant4<BF16, HAS_SCALE>((uint32_t)v[i].z, s, o[4], o[5]);
      dequant4<BF16, HAS_SCALE>((uint32_t)v[i].w, s, o[6], o[7]);
      uint8_t* row = lds + r * kRowBytes;
      *reinterpret_cast<i32x4*>(row + swz_chunk(r, 2 * c) * 16) =
          i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      *reinterpret_cast<i32x4*>(row + swz_chunk(r, 2 * c + 1) * 16) =
          i32x4{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
    }
  }
};

// ----------------------------------------------------- tile scheduling ---
struct TileCoord { int tm, tn; };

// Remap the dispatch order (blocks go round-robin over the 8 XCDs) so each
// XCD owns a contiguous run of tiles, then raster that run in bands of
// kGroupM tile rows.
__device__ __forceinline__ TileCoord tile_of(int bid, int nblocks, int tiles_m, int tiles_n) {
  const int full = nblocks & ~7;
  if (bid < full) bid = (bid & 7) * (full >> 3) + (bid >> 3);
  const int band = kGroupM * tiles_n;
  const int first_m = (bid / band) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_band = bid - (bid / band) * band;
  TileCoord t;
  t.tm = first_m + in_band % gm;
  t.tn = in_band / gm;
  return t;
}

// ------------------------------------------------------------ epilogue ---
// Walk the accumulators of one wave and hand every in-range element to the
// epilogue functor.  32x32 MFMA output layout: lane l, register r hold
// row 8*(r/4) + 4*(l/32) + r%4, column l%32.
template <int TM, int TN, class Acc, class Epi>
__device__ __forceinline__ void epilogue_single(const Acc (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                int64_t M, int64_t N, const Epi& epi) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + j * 32 + (lane & 31);
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m < M) epi(m, n, acc[i][j][r]);
      }
    }
  }
}

// Pair epilogue: blocks 2t (gate) and 2t+1 (up) cover the same 32 output
// columns c0 + 32 t + lane%32.
template <int TM, int TN, class Acc, class Epi>
__device__ __forceinline__ void epilogue_pair(const Acc (&acc)[TM][TN], int64_t m0, int64_t c0,
                                              int64_t M, int64_t NC, const Epi& epi) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < TN / 2; ++t) {
    const int64_t col = c0 + t * 32 + (lane & 31);
    if (col >= NC) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m < M) epi.pair(m, col, acc[i][2 * t][r], acc[i][2 * t + 1][r]);
      }
    }
  }
}

// --------------------------------------------------------- main kernel ---
struct GemmShape {
  int64_t M, N, K;          // N = output columns (pair kernels: 2 * N_out)
  int64_t a_kbytes;         // K * sizeof(A element)
  int64_t b_kbytes;         // K * sizeof(B element in global memory)
  int tiles_m, tiles_n;
};

// One K stage of MFMAs on LDS buffer `sm` for this wave's sub-tile.
template <class Mma, int BM, int TM, int TN>
__device__ __forceinline__ void mma_stage(const uint8_t* sm, typename Mma::Acc (&acc)[TM][TN],
                                          int wm, int wn) {
  constexpr int KC = Mma::kChunks;
  constexpr int KSTEPS = 8 / (2 * KC);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31;
  const int half = lane >> 5;
  const uint8_t* sa = sm;
  const uint8_t* sb = sm + BM * kRowBytes;
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    i32x4 af[TM][KC], bf[TN][KC];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * (TM * 32) + i * 32 + lr;
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        const int c = s * 2 * KC + half * KC + u;
        af[i][u] = *reinterpret_cast<const i32x4*>(sa + r * kRowBytes + swz_chunk(r, c) * 16);
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * (TN * 32) + j * 32 + lr;
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        const int c = s * 2 * KC + half * KC + u;
        bf[j][u] = *reinterpret_cast<const i32x4*>(sb + r * kRowBytes + swz_chunk(r, c) * 16);
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = Mma::mma(af[i], bf[j], acc[i][j]);
  }
}

// PAIR = false: plain GEMM, epilogue(m, n, acc).
// PAIR = true : gate/up pair, epilogue.pair(m, col, acc_gate, acc_up).
template <class Mma, int BM, int BN, class LoadA, class SrcA, class LoadB, class SrcB,
          class BStoreArg, bool PAIR, class Epi>
__global__ void __launch_bounds__(kThreads)
gemm_tile_kernel(GemmShape sh, SrcA srca, SrcB srcb, BStoreArg barg, Epi epi) {
  constexpr int TM = BM / 64, TN = BN / 64;    // 32x32 blocks per wave (2x2 waves)
  static_assert(!PAIR || (TN % 2 == 0), "pair tiles need whole gate/up block pairs");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][(BM + BN) * kRowBytes];

  const TileCoord tc = tile_of(blockIdx.x, gridDim.x, sh.tiles_m, sh.tiles_n);
  const Epi ep = epi.prepare();
  const BStoreArg bst = barg.prepare();
  const int64_t m0 = (int64_t)tc.tm * BM;
  const int64_t n0 = (int64_t)tc.tn * BN;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  typename Mma::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // stage geometry: 128 bytes of A per row per stage; B advances by the same
  // number of K elements (its global bytes per stage may differ: fp8 weights
  // under bf16 activations advance 64 bytes).
  constexpr int64_t kAStage = kRowBytes;
  const int64_t b_stage = sh.b_kbytes == sh.a_kbytes ? kRowBytes : kRowBytes / 2;
  const int nst = (int)((sh.a_kbytes + kAStage - 1) / kAStage);

  LoadA la;
  LoadB lb;
  const int64_t bn0 = n0;   // B row origin (pair sources interpret it in doubled-N space)
  la.load(srca, m0, 0, sh.a_kbytes);
  lb.load(srcb, bn0, 0, sh.b_kbytes);
  la.store(smem[0]);
  bst.store(lb, smem[0] + BM * kRowBytes);
  __syncthreads();

  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < nst;
    if (more) {
      la.load(srca, m0, (int64_t)(st + 1) * kAStage, sh.a_kbytes);
      lb.load(srcb, bn0, (int64_t)(st + 1) * b_stage, sh.b_kbytes);
    }
    mma_stage<Mma, BM, TM, TN>(smem[cur], acc, wm, wn);
    if (more) {
      la.store(smem[cur ^ 1]);
      bst.store(lb, smem[cur ^ 1] + BM * kRowBytes);
    }
    __syncthreads();
  }

  const int64_t wm0 = m0 + wm * (TM * 32);
  if constexpr (PAIR) {
    const int64_t c0 = (n0 >> 1) + wn * (TN * 16);
    epilogue_pair<TM, TN>(acc, wm0, c0, sh.M, sh.N >> 1, ep);
  } else {
    epilogue_single<TM, TN>(acc, wm0, n0 + wn * (TN * 32), sh.M, sh.N, ep);
  }
}

// B-stage store adaptors: plain copy, or dequantizing fp8 -> half types.
struct BStorePlain {
  __device__ __forceinline__ BStorePlain prepare() const { return *this; }
  template <class L>
  __device__ __forceinline__ void store(const L& l, uint8_t* lds) const { l.store(lds); }
};
// The per-tensor weight scale lives in device memory (a [1] fp32 tensor);
// it is read once per workgroup and rounded to the activation type, as
// scale.to(T) does in the kitchen dequant formula.
template <bool BF16>
struct BStoreDequant {
  const float* sp; float s;
  __device__ __forceinline__ BStoreDequant prepare() const {
    BStoreDequant r = *this;
    if (sp) r.s = BF16 ? bf16_f32(bf16_rte(sp[0])) : f16_f32(f16_rte(sp[0]));
    else r.s = 1.0f;
    return r;
  }
  template <class L>
  __device__ __forceinline__ void store(const L& l, uint8_t* lds) const { l.store(lds, s); }
};

}  // namespace c4q
