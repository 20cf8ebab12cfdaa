// LDS-tiled MFMA GEMM core for gfx950 (CDNA4), NT layout:
//
//     D[m, n] = epilogue( sum_k A[m, k] * B[n, k] )
//
// A is the activation [M, K] and B the weight in its stored nn.Linear
// layout [N, K]; both are K-contiguous, which is the operand order every
// MFMA wants, so neither is ever transposed.
//
// Structure:
//   * a workgroup of WM x WN wave64s owns a BM x BN output tile; each wave a
//     (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks held in registers;
//   * K advances in stages of 64 elements. Operands are copied global ->
//     LDS by buffer_load_dwordx4 ... lds (no register round trip) into a
//     ring of NBUF stage buffers, issued up to NBUF-1 stages ahead of the
//     MFMAs that consume them, so the copy latency (~1.3 us from L2/MALL)
//     hides behind several stages of MFMA work; one barrier per stage;
//   * inside a stage the LDS fragments of the next K step are read while the
//     current step multiplies, across stage boundaries too;
//   * the epilogue stages each wave's accumulators through LDS, then applies
//     the output arithmetic in a compact loop over 4-column groups and
//     stores whole 8/16-byte chunks of output rows;
//   * the copy reads through buffer resources based at the tile origin whose
//     range ends at the matrix end: tail rows and the K tail read as zero in
//     hardware (stages past K are issued with out-of-range offsets, so every
//     stage issues the same number of copies);
//   * LDS rows are 64 or 128 bytes per stage with the 16-byte chunks
//     XOR-swizzled by row, so that fragment reads (32 lanes on 32 rows, one
//     chunk) are bank-conflict free;
//   * W8A16: the fp8 weight is staged as fp8 and dequantized to bf16/f16 in
//     registers right after each fragment read (one ds_read_b128 of 16 codes
//     feeds two K steps);
//   * workgroup ids are remapped so that each of the 8 XCDs owns a
//     contiguous run of tiles, walked in kGroupM-row bands, keeping the A and
//     B panels a band shares inside that XCD's L2.
#pragma once
#include <type_traits>

#include "epilogues.hpp"
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

constexpr int kStageK = 64;          // K elements per pipeline stage
constexpr int kGroupM = 8;           // tile rows per raster band

template <class T, class F>
__device__ __forceinline__ T bitcast(const F& f) { return __builtin_bit_cast(T, f); }

// ------------------------------------------------------------ swizzles ---
// Physical 16-byte chunk of logical chunk c in LDS row r. A fragment read
// has 32 consecutive lanes on 32 consecutive rows at one logical chunk; the
// row permutations below send any 8 consecutive rows to 8 distinct 16-byte
// bank groups of a 128-byte window and any 16 consecutive rows to 16
// distinct groups of a 256-byte window, so ds_read_b128 is conflict-free
// whether the LDS serves 8 or 16 lanes per cycle.
template <int ROWB> struct Swz;
template <> struct Swz<128> {   // 8 chunks per row
  __device__ __forceinline__ static int f(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }
};
template <> struct Swz<64> {    // 4 chunks per row
  __device__ __forceinline__ static int f(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }
};
template <int ROWB>
__device__ __forceinline__ int phys_chunk(int r, int c) { return c ^ Swz<ROWB>::f(r); }

// ------------------------------------------------------------- buffers ---
// Buffer resource (V#) over [base, base + bytes); offsets at or past the
// range read zeros. Ranges are clamped below 2^31 (a tile spans <= 256 rows,
// so its offsets stay far below that).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint8_t* base, int64_t bytes) {
  const int32_t n = bytes > 0x7FFFFFF0ll ? 0x7FFFFFF0 : (int32_t)(bytes < 0 ? 0 : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, n, 0x00020000);
}
constexpr int kOOB = 0x7FFFFFF0;   // an offset past any range

// Direct global->LDS copy of one stage of a ROWS x ROWB-byte operand slab.
// One buffer_load_dwordx4 ... lds moves 1 KB: lane L fills LDS row
// RPI*q + L/CPR at physical chunk L%CPR, so it fetches the logical chunk
// that the swizzle stores there -- the layout comes from choosing sources.
// PAIR (FFN gate/up): in the doubled-N tile space every 32-row MFMA block
// alternates between the gate matrix (even blocks) and the up matrix (odd
// blocks) for the same 32 output columns, so one lane ends up holding gate
// and up accumulators of the same (m, col).
template <int ROWS, int ROWB, int NT, bool PAIR>
struct DirectLoad {
  static constexpr int CPR = ROWB / 16;             // chunks per row
  static constexpr int RPI = 64 / CPR;              // rows per instruction
  static constexpr int kWaves = NT / 64;
  static constexpr int kInstr = ROWS / RPI / kWaves;
  static_assert(kInstr >= 1 && kInstr * RPI * kWaves == ROWS, "tile rows must split over the waves");
  int voff[kInstr];
  int kofs[kInstr];           // byte offset of this lane's chunk within the stage row
  __device__ __forceinline__ void init(int64_t ld_bytes) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
      const int q = wave + kWaves * j;
      const int r = RPI * q + lane / CPR;                      // LDS row
      const int blk = (RPI * q) >> 5;
      const int src = PAIR ? ((blk >> 1) * 32 + ((RPI * q) & 31) + lane / CPR) : r;
      kofs[j] = ((lane % CPR) ^ Swz<ROWB>::f(r)) * 16;
      voff[j] = (int)(src * ld_bytes) + kofs[j];
    }
  }
  // Copy K bytes [kb, kb + ROWB) of every row into `lds`; bytes at or past
  // k_bytes read zeros.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1,
                                        uint8_t* lds, int kb, int k_bytes) const {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
      const int q = wave + kWaves * j;
      const __amdgpu_buffer_rsrc_t rs = (PAIR && (((RPI * q) >> 5) & 1)) ? r1 : r0;
      const int vo = kb + kofs[j] < k_bytes ? voff[j] : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(lds + (RPI * q) * ROWB), 16, vo, kb, 0, 0);
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

// ------------------------------------------------------ operand policies ---
// Each policy fixes the MFMA, the stage row sizes of A and B in LDS (SA, SB
// bytes per row per stage) and how one stage's fragments are read and
// multiplied.
template <int ROWB>
__device__ __forceinline__ i32x4 lds_chunk(const uint8_t* sm, int r, int c) {
  return *reinterpret_cast<const i32x4*>(sm + r * ROWB + phys_chunk<ROWB>(r, c) * 16);
}

// Policies expose one stage as S "K steps": frags(s) reads the LDS
// fragments of step s into registers, mma(frags) multiplies them. The
// kernel reads step s+1 while step s multiplies.

// int8 x int8 -> int32, v_mfma_i32_32x32x32_i8: a lane holds 16 K values
// (one chunk); a 64-byte stage row is 2 K steps.
struct OpI8 {
  using Acc = i32x16;
  static constexpr int SA = 64, SB = 64, S = 2;
  template <int TM, int TN> struct Frag { i32x4 a[TM], b[TN]; };
  __device__ __forceinline__ static float prep_scale(const float*) { return 1.0f; }
  template <int TM, int TN>
  __device__ __forceinline__ static void frags(Frag<TM, TN>& f, const uint8_t* sa, const uint8_t* sb,
                                               int ra0, int rb0, int s) {
    const int lane = threadIdx.x & 63, lr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < TM; ++i) f.a[i] = lds_chunk<SA>(sa, ra0 + i * 32 + lr, 2 * s + h);
#pragma unroll
    for (int j = 0; j < TN; ++j) f.b[j] = lds_chunk<SB>(sb, rb0 + j * 32 + lr, 2 * s + h);
  }
  template <int TM, int TN>
  __device__ __forceinline__ static void mma(const Frag<TM, TN>& f, Acc (&acc)[TM][TN], float) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
  }
};

// OCP e4m3 x e4m3 -> fp32, v_mfma_f32_32x32x64_f8f6f4 (cbsz = blgp = 0:
// e4m3 operands; zero scales: unscaled): a lane holds 32 K values (two
// chunks); a 64-byte stage row is one K step.
struct OpF8 {
  using Acc = f32x16;
  static constexpr int SA = 64, SB = 64, S = 1;
  template <int TM, int TN> struct Frag { i32x8 a[TM], b[TN]; };
  __device__ __forceinline__ static float prep_scale(const float*) { return 1.0f; }
  template <int TM, int TN>
  __device__ __forceinline__ static void frags(Frag<TM, TN>& f, const uint8_t* sa, const uint8_t* sb,
                                               int ra0, int rb0, int) {
    const int lane = threadIdx.x & 63, lr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const i32x4 x = lds_chunk<SA>(sa, ra0 + i * 32 + lr, 2 * h);
      const i32x4 y = lds_chunk<SA>(sa, ra0 + i * 32 + lr, 2 * h + 1);
      f.a[i] = i32x8{x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const i32x4 x = lds_chunk<SB>(sb, rb0 + j * 32 + lr, 2 * h);
      const i32x4 y = lds_chunk<SB>(sb, rb0 + j * 32 + lr, 2 * h + 1);
      f.b[j] = i32x8{x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ static void mma(const Frag<TM, TN>& f, Acc (&acc)[TM][TN], float) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[i][j], 0, 0,
                                                                    0, 0, 0, 0);
  }
};

// W8A16: bf16 (or f16) activations x fp8 weights dequantized in registers,
// v_mfma_f32_32x32x16_{bf16,f16}: a lane holds 8 K values. A stage row is
// 128 bytes of activations and 64 bytes of fp8 weights (64 K values = 4
// MFMA steps, taken here as 2 K steps of 2 MFMAs). The K order inside a
// stage is permuted identically for both operands: K step t, lane half h,
// takes the 16 consecutive K values [32t + 16h, 32t + 16h + 16) -- the first
// 8 in its first MFMA, the last 8 in its second -- so one 16-byte fp8 chunk
// (chunk 2t+h) feeds both, while the activation fragments are bf16 chunks
// 4t + 2h and 4t + 2h + 1.
template <bool BF16, bool HAS_SCALE>
struct OpW8A16 {
  using Acc = f32x16;
  static constexpr int SA = 128, SB = 64, S = 2;
  template <int TM, int TN> struct Frag { i32x4 a[2][TM], q[TN]; };
  // per-tensor weight scale rounded to the activation type (scale.to(T))
  __device__ __forceinline__ static float prep_scale(const float* sp) {
    if (!HAS_SCALE || !sp) return 1.0f;
    return BF16 ? bf16_f32(bf16_rte(sp[0])) : f16_f32(f16_rte(sp[0]));
  }
  __device__ __forceinline__ static f32x16 mfma(i32x4 a, i32x4 b, f32x16 c) {
    if constexpr (BF16)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
  template <int TM, int TN>
  __device__ __forceinline__ static void frags(Frag<TM, TN>& f, const uint8_t* sa, const uint8_t* sb,
                                               int ra0, int rb0, int t) {
    const int lane = threadIdx.x & 63, lr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < TN; ++j) f.q[j] = lds_chunk<SB>(sb, rb0 + j * 32 + lr, 2 * t + h);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < TM; ++i) f.a[u][i] = lds_chunk<SA>(sa, ra0 + i * 32 + lr, 4 * t + 2 * h + u);
  }
  template <int TM, int TN>
  __device__ __forceinline__ static void mma(const Frag<TM, TN>& f, Acc (&acc)[TM][TN], float ws) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      uint32_t o[8];
      dequant4<BF16, HAS_SCALE>((uint32_t)f.q[j].x, ws, o[0], o[1]);
      dequant4<BF16, HAS_SCALE>((uint32_t)f.q[j].y, ws, o[2], o[3]);
      dequant4<BF16, HAS_SCALE>((uint32_t)f.q[j].z, ws, o[4], o[5]);
      dequant4<BF16, HAS_SCALE>((uint32_t)f.q[j].w, ws, o[6], o[7]);
      const i32x4 b0 = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      const i32x4 b1 = {(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        acc[i][j] = mfma(f.a[0][i], b0, acc[i][j]);
        acc[i][j] = mfma(f.a[1][i], b1, acc[i][j]);
      }
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
// Two phases per 32-row strip of a wave's sub-tile, through a private LDS
// area (the idle operand ring):
//   1. raw 32-bit accumulators go in at their (row, column) from the MFMA
//      layout (lane l, register r hold row 8*(r/4) + 4*(l/32) + r%4, column
//      l%32 of a 32x32 block) -- straight-line register moves only;
//   2. a compact loop: each lane takes 4 consecutive columns of one row,
//      applies the epilogue arithmetic once per element and stores the 4
//      outputs as one 8- or 16-byte chunk (16 lanes cover 64 columns).
// Pair strips hold gate and up accumulators side by side (2 words per
// output). Strip rows are padded by 16 bytes so the two half-waves of a
// phase-1 write land on different banks.
template <int WORDS>          // 32-bit words per strip row
struct Strip {
  static constexpr int kStride = WORDS * 4 + 16;
  static constexpr int kBytes = 32 * kStride;
};

__device__ __forceinline__ void lds_fence_wave() {
  __builtin_amdgcn_s_waitcnt(0xc07f);                     // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
}

template <int TM, int TN, class Acc, class Epi>
__device__ __forceinline__ void epilogue_single(const Acc (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                int64_t M, int64_t N, const Epi& epi, uint8_t* lds) {
  using Scalar = std::remove_cv_t<std::remove_reference_t<decltype(acc[0][0][0])>>;
  constexpr int COLS = TN * 32;
  using St = Strip<COLS>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        *reinterpret_cast<Scalar*>(lds + row * St::kStride + col * 4) = acc[i][j][r];
      }
    }
    lds_fence_wave();
    const int64_t mb = m0 + i * 32;
    constexpr int G = COLS / 4;                           // 4-column groups per row
#pragma unroll 2
    for (int g = lane; g < 32 * G; g += 64) {
      const int row = g / G, c4 = (g % G) * 4;
      const int64_t m = mb + row, n = n0 + c4;
      if (m >= M || n >= N) continue;
      const Scalar* raw = reinterpret_cast<const Scalar*>(lds + row * St::kStride + c4 * 4);
      const Scalar v[4] = {raw[0], raw[1], raw[2], raw[3]};
      const int nv = N - n < 4 ? (int)(N - n) : 4;
      store_group(epi, m, n, nv, epi.value4(m, n, v, nv));
    }
    lds_fence_wave();
  }
}

// Pair epilogue: blocks 2t (gate) and 2t+1 (up) give the same 32 output
// columns c0 + 32 t + lane%32; the strip interleaves them per column.
template <int TM, int TN, class Acc, class Epi>
__device__ __forceinline__ void epilogue_pair(const Acc (&acc)[TM][TN], int64_t m0, int64_t c0,
                                              int64_t M, int64_t NC, const Epi& epi, uint8_t* lds) {
  constexpr int COLS = TN / 2 * 32;
  using St = Strip<2 * COLS>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int t = 0; t < TN / 2; ++t) {
      const int colw = t * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        int32_t* p = reinterpret_cast<int32_t*>(lds + row * St::kStride + colw * 8);
        p[0] = acc[i][2 * t][r];
        p[1] = acc[i][2 * t + 1][r];
      }
    }
    lds_fence_wave();
    const int64_t mb = m0 + i * 32;
    constexpr int G = COLS / 4;
#pragma unroll 2
    for (int g = lane; g < 32 * G; g += 64) {
      const int row = g / G, c4 = (g % G) * 4;
      const int64_t m = mb + row, n = c0 + c4;
      if (m >= M || n >= NC) continue;
      const int32_t* raw = reinterpret_cast<const int32_t*>(lds + row * St::kStride + c4 * 8);
      const int32_t gv[4] = {raw[0], raw[2], raw[4], raw[6]};
      const int32_t uv[4] = {raw[1], raw[3], raw[5], raw[7]};
      const int nv = NC - n < 4 ? (int)(NC - n) : 4;
      store_group(epi, m, n, nv, epi.pair4(m, n, gv, uv, nv));
    }
    lds_fence_wave();
  }
}

// --------------------------------------------------------- main kernel ---
struct GemmShape {
  int64_t M, N, K;          // N = output columns (pair kernels: 2 * N_out)
  int tiles_m, tiles_n;
};

// Operand sources: base pointers and strides; each workgroup derives its
// tile's buffer resources from them.
struct Src2 {
  const uint8_t* p0; const uint8_t* p1;   // p1: second matrix of a pair (up rows), else = p0
  int64_t ld_bytes; int64_t rows;          // rows of each matrix
};

// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Stage barrier without a memory fence. __syncthreads() is a workgroup
// release/acquire fence, which makes the compiler wait for every
// outstanding vector-memory operation (vmcnt(0)) -- that would drain the
// whole copy ring at every stage. Here each wave has already waited for the
// copies of the stage it needs (wait_vm); it waits for its own LDS reads,
// then meets the others at the hardware barrier. The asm statement is also a
// compiler barrier for memory operations.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// PAIR = false: plain GEMM, epilogue(m, n, acc).
// PAIR = true : gate/up pair, epilogue.pair(m, col, acc_gate, acc_up).
// b_scale: W8A16 per-tensor weight scale (device pointer) or null.
template <class Op, int BM, int BN, int WM, int WN, int NBUF, bool PAIR, class Epi>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_tile_kernel(GemmShape sh, Src2 sa, Src2 sb, const float* b_scale, Epi epi) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;   // 32x32 MFMA blocks per wave
  static_assert(TM >= 1 && TN >= 1 && TM * WM * 32 == BM && TN * WN * 32 == BN, "bad wave tiling");
  static_assert(!PAIR || (TN % 2 == 0), "pair tiles need whole gate/up block pairs");
  constexpr int SA = Op::SA, SB = Op::SB;
  constexpr int STAGE = BM * SA + BN * SB;
  static_assert(NBUF >= 2 && NBUF * STAGE <= 160 * 1024, "LDS ring exceeds 160 KB");
  using LA = DirectLoad<BM, SA, NT, false>;
  using LB = DirectLoad<BN, SB, NT, PAIR>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NBUF * STAGE];

  const TileCoord tc = tile_of(blockIdx.x, gridDim.x, sh.tiles_m, sh.tiles_n);
  const Epi ep = epi.prepare();
  const int64_t m0 = (int64_t)tc.tm * BM;
  const int64_t n0 = (int64_t)tc.tn * BN;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;

  LA la;
  LB lb;
  la.init(sa.ld_bytes);
  lb.init(sb.ld_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
  const int64_t brow0 = PAIR ? (n0 >> 1) : n0;     // pair: both matrices start at column n0/2
  const int64_t bleft = (sb.rows - brow0) * sb.ld_bytes;
  const __amdgpu_buffer_rsrc_t rb0 = make_rsrc(sb.p0 + brow0 * sb.ld_bytes, bleft);
  const __amdgpu_buffer_rsrc_t rb1 = PAIR ? make_rsrc(sb.p1 + brow0 * sb.ld_bytes, bleft) : rb0;
  const float ws = Op::prep_scale(b_scale);

  typename Op::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int a_kb = (int)(sh.K * (SA / kStageK)), b_kb = (int)(sh.K * (SB / kStageK));
  const int nst = (int)((sh.K + kStageK - 1) / kStageK);

  // prologue: stages 0 .. NBUF-1 in flight, stage 0 complete and visible
#pragma unroll
  for (int p = 0; p < NBUF; ++p) {
    uint8_t* buf = smem + p * STAGE;
    la.issue(ra, ra, buf, p * SA, a_kb);
    lb.issue(rb0, rb1, buf + BM * SA, p * SB, b_kb);
  }
  wait_vm<(NBUF - 1) * kPerStage>();
  stage_barrier();

  // K-step pipeline: the fragments of the next step are read while the
  // current step multiplies. The stage barrier sits before the last step of
  // each stage, whose fragments are already in registers: after it the
  // next stage is visible (its first fragments load under the last step's
  // MFMAs) and the stage just read is free to refill.
  const int ra0 = wm * (TM * 32), rb0i = wn * (TN * 32);
  using Frag = typename Op::template Frag<TM, TN>;
  Frag fr[2];
  Op::template frags<TM, TN>(fr[0], smem, smem + BM * SA, ra0, rb0i, 0);
  constexpr int S = Op::S;
  // One stage; P = parity of the stage's first K step in the global step
  // sequence (so the fragment double buffer is indexed statically).
  auto run_stage = [&](int st, auto Pc) {
    constexpr int P = decltype(Pc)::value;
    const uint8_t* cur = smem + (st % NBUF) * STAGE;
    const uint8_t* nxt = smem + ((st + 1) % NBUF) * STAGE;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (s == S - 1) {
        wait_vm<(NBUF - 2) * kPerStage>();     // this wave's copies of stage st+1 landed
        stage_barrier();                       // ... and every wave's; stage st fully read
        const int ps = st + NBUF;              // refill stage st's buffer (past K: zeros)
        uint8_t* buf = smem + (st % NBUF) * STAGE;
        la.issue(ra, ra, buf, ps * SA, a_kb);
        lb.issue(rb0, rb1, buf + BM * SA, ps * SB, b_kb);
        Op::template frags<TM, TN>(fr[(P + s + 1) & 1], nxt, nxt + BM * SA, ra0, rb0i, 0);
      } else {
        Op::template frags<TM, TN>(fr[(P + s + 1) & 1], cur, cur + BM * SA, ra0, rb0i, s + 1);
      }
      Op::template mma<TM, TN>(fr[(P + s) & 1], acc, ws);
    }
  };
  if constexpr (S % 2 == 0) {
    for (int st = 0; st < nst; ++st) run_stage(st, std::integral_constant<int, 0>{});
  } else {
    int st = 0;
    for (; st + 1 < nst; st += 2) {
      run_stage(st, std::integral_constant<int, 0>{});
      run_stage(st + 1, std::integral_constant<int, 1>{});
    }
    if (st < nst) run_stage(st, std::integral_constant<int, 0>{});
  }
  wait_vm<0>();    // past-K copies still land in the ring; drain before reusing LDS
  __syncthreads();

  // per-wave output strips in the (now idle) ring
  constexpr int kStripBytes = Strip<(PAIR ? TN / 2 * 2 : TN) * 32>::kBytes;
  static_assert(kStripBytes * WM * WN <= NBUF * STAGE, "output strips exceed the LDS ring");
  uint8_t* strip = smem + wave * kStripBytes;
  const int64_t wm0 = m0 + wm * (TM * 32);
  if constexpr (PAIR) {
    const int64_t c0 = (n0 >> 1) + wn * (TN * 16);
    epilogue_pair<TM, TN>(acc, wm0, c0, sh.M, sh.N >> 1, ep, strip);
  } else {
    epilogue_single<TM, TN>(acc, wm0, n0 + wn * (TN * 32), sh.M, sh.N, ep, strip);
  }
}

}  // namespace c4q
