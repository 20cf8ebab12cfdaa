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
//   * K advances in stages of 64 or 128 elements (a policy constant). Operands are copied global ->
//     LDS by buffer_load_dwordx4 ... lds (no register round trip) into a
//     ring of NBUF stage buffers, issued up to NBUF-1 stages ahead of the
//     MFMAs that consume them, so the copy latency (~1.3 us from L2/MALL)
//     hides behind several stages of MFMA work; one barrier per stage;
//   * inside a stage the LDS fragments of the next K step are read while the
//     current step multiplies, across stage boundaries too;
//   * the kernel is persistent: each workgroup walks a sequence of tiles
//     with one copy ring, so the next tile's first stages are copied while
//     the current tile's epilogue runs;
//   * the epilogue stages each wave's accumulators through a small private
//     LDS strip, applies the output arithmetic with column / row parameters
//     loaded once per tile and stores whole 8/16-byte chunks of output rows;
//   * the copy reads through buffer resources based at the tile origin whose
//     range ends at the matrix end: tail rows and the K tail read as zero in
//     hardware (stages past K are issued with out-of-range offsets, so every
//     stage issues the same number of copies);
//   * LDS rows are 64 or 128 bytes per stage (8-bit operands at 128 K per
//     stage move whole 128-byte cache lines) with the 16-byte chunks
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
#include <utility>

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

// Tile rows per raster band. Measured on MI355X over band heights 1, 2, 3,
// 4, 6 and 8 (fp8 16384x5120->13824 / 16384x13824->5120, int8 9216x5120 with
// N 5120 / 13824 and 9216x13824->5120, the INT8 pair, W8A16 QKV / block):
// 3 gains 5-6 % on the K = 5120 shapes over 8 and is within 1 % of the best
// everywhere else (2 and 6 also win on the K = 5120 shapes but lose 1-4 %
// on the K = 13824 down-projection and the INT8 pair).
constexpr int kGroupM = 3;

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

// One buffer_load_dwordx4 ... lds: each lane's 16 bytes at voff + soff of
// the resource land at lds_addr + 16 * lane. Issued as inline assembly so
// that the compiler does not track it as an LDS store: tracked, it would
// wait for every copy in flight (vmcnt(0)) before any later LDS access it
// cannot prove disjoint -- the fragment reads of other stages and the
// epilogue strips. The kernels order copies and reads themselves: a stage
// is read only after each copying wave's vmcnt wait and a barrier, and a
// buffer is refilled only after a barrier that follows its last reads.
// m0 (the LDS base of the copy) is set inside the statement; nothing else
// in these kernels reads m0.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The words of a raw buffer resource over [base, base + bytes) (as
// make_rsrc), kept in scalar registers for lds_dma16.
__device__ __forceinline__ u32x4 dma_rsrc(const uint8_t* base, int64_t bytes) {
  const uint32_t n = bytes > 0x7FFFFFF0ll ? 0x7FFFFFF0u : (uint32_t)(bytes < 0 ? 0 : bytes);
  const uint64_t a = (uint64_t)(uintptr_t)base;
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xFFFFu);   // stride 0
  r.z = __builtin_amdgcn_readfirstlane(n);
  r.w = 0x00020000u;
  return r;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(u32x4 rsrc, const uint8_t* lds, int voff, int soff) {
  const uint32_t addr = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(addr), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

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
  // The swizzles repeat every 16 rows and one copy round of all waves spans
  // a multiple of 16 rows, so a lane's chunk within the stage row is the
  // same for every copy it issues.
  static_assert((RPI * kWaves) % 16 == 0, "swizzle period must divide the copy round");
  // Source offsets: plain operands step by a fixed number of rows per copy
  // (one base register and a uniform stride); pair operands interleave the
  // gate and up matrices by 32-row block and keep one offset per copy.
  static constexpr int kOff = PAIR ? kInstr : 1;
  int voff[kOff];
  int kofs;                   // byte offset of this lane's chunk within the stage row
  int step;                   // plain operands: bytes between the rows of consecutive copies
  int wv;                     // this wave's index among the NT / 64 copying waves
  int row0;                   // first stage row the copying waves fill (a multiple of 64)
  __device__ __forceinline__ void init(int64_t ld_bytes, int wave, int first_row) {
    const int lane = threadIdx.x & 63;
    wv = __builtin_amdgcn_readfirstlane(wave);          // wave-uniform: keeps copy
    row0 = __builtin_amdgcn_readfirstlane(first_row);   // addresses in scalar registers
    kofs = ((lane % CPR) ^ Swz<ROWB>::f(row0 + RPI * wave + lane / CPR)) * 16;
    step = (int)(RPI * kWaves * ld_bytes);
#pragma unroll
    for (int j = 0; j < kOff; ++j) {
      const int rq = row0 + RPI * (wave + kWaves * j);          // first LDS row of copy j
      const int r = rq + lane / CPR;
      const int src = PAIR ? ((rq >> 6) * 32 + (rq & 31) + lane / CPR) : r;
      voff[j] = (int)(src * ld_bytes) + kofs;
    }
  }
  // Copy J of issue() alone, for schedules that spread a stage's copies.
  template <int J>
  __device__ __forceinline__ void issue_one(u32x4 r0, u32x4 r1, uint8_t* lds, int kb,
                                            int k_bytes) const {
    static_assert(J >= 0 && J < kInstr, "copy index");
    const bool in_k = kb + kofs < k_bytes;
    const int rq = row0 + RPI * (wv + kWaves * J);
    const u32x4 rs = (PAIR && ((rq >> 5) & 1)) ? r1 : r0;
    const int vo = PAIR ? voff[PAIR ? J : 0] : voff[0] + J * step;
    lds_dma16(rs, lds + rq * ROWB, in_k ? vo : kOOB, kb);
  }
  // Copy K bytes [kb, kb + ROWB) of every row into `lds`; bytes at or past
  // k_bytes read zeros.
  __device__ __forceinline__ void issue(u32x4 r0, u32x4 r1,
                                        uint8_t* lds, int kb, int k_bytes) const {
    const bool in_k = kb + kofs < k_bytes;
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
      const int rq = row0 + RPI * (wv + kWaves * j);
      const u32x4 rs = (PAIR && ((rq >> 5) & 1)) ? r1 : r0;
      const int vo = PAIR ? voff[PAIR ? j : 0] : voff[0] + j * step;
      lds_dma16(rs, lds + rq * ROWB, in_k ? vo : kOOB, kb);
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
  if constexpr (!HAS_SCALE) {
    // e4m3fn -> bf16/f16 is exact; the scaled conversion with scale 1.0 (a
    // power of two, the only scales it applies exactly) does two codes per
    // instruction
    if constexpr (BF16) {
      lo = bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
      hi = bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
    } else {
      lo = bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
      hi = bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
    }
    return;
  }
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

// Calls f(std::integral_constant<int, Q>{}) for Q = Q0 .. Q1-1.
template <int Q0, int Q1, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (Q0 < Q1) {
    f(std::integral_constant<int, Q0>{});
    static_for<Q0 + 1, Q1>(f);
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
// (one chunk); a stage of KS K values (KS-byte rows) is KS/32 K steps.
template <int KS>
struct OpI8T {
  using Acc = i32x16;
  static constexpr int kStageK = KS, SA = KS, SB = KS, S = KS / 32;
  static constexpr bool kPingPong = false;   // see gemm_pingpong_kernel
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
// chunks); a stage of KS K values is KS/64 K steps.
template <int KS>
struct OpF8T {
  using Acc = f32x16;
  static constexpr int kStageK = KS, SA = KS, SB = KS, S = KS / 64;
  static constexpr bool kPingPong = false;
  template <int TM, int TN> struct Frag { i32x8 a[TM], b[TN]; };
  __device__ __forceinline__ static float prep_scale(const float*) { return 1.0f; }
  template <int ROWB>
  __device__ __forceinline__ static i32x8 pair_chunks(const uint8_t* sm, int r, int c) {
    const i32x4 x = lds_chunk<ROWB>(sm, r, c);
    const i32x4 y = lds_chunk<ROWB>(sm, r, c + 1);
    return i32x8{x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
  }
  template <int TM, int TN>
  __device__ __forceinline__ static void frags(Frag<TM, TN>& f, const uint8_t* sa, const uint8_t* sb,
                                               int ra0, int rb0, int s) {
    const int lane = threadIdx.x & 63, lr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < TM; ++i) f.a[i] = pair_chunks<SA>(sa, ra0 + i * 32 + lr, 4 * s + 2 * h);
#pragma unroll
    for (int j = 0; j < TN; ++j) f.b[j] = pair_chunks<SB>(sb, rb0 + j * 32 + lr, 4 * s + 2 * h);
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
  // One fragment block (Q < TM: A block Q, else B block Q - TM) and one
  // MFMA, for schedules that interleave them with other work.
  template <int TM, int TN, int Q>
  __device__ __forceinline__ static void frag_one(Frag<TM, TN>& f, const uint8_t* sa,
                                                  const uint8_t* sb, int ra0, int rb0, int s) {
    const int lane = threadIdx.x & 63, lr = lane & 31, h = lane >> 5;
    if constexpr (Q < TM) f.a[Q] = pair_chunks<SA>(sa, ra0 + Q * 32 + lr, 4 * s + 2 * h);
    else f.b[Q - TM] = pair_chunks<SB>(sb, rb0 + (Q - TM) * 32 + lr, 4 * s + 2 * h);
  }
  template <int TM, int TN, int I, int J>
  __device__ __forceinline__ static void mma_one(const Frag<TM, TN>& f, Acc (&acc)[TM][TN]) {
    acc[I][J] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[I], f.b[J], acc[I][J], 0, 0,
                                                                0, 0, 0, 0);
  }
};
// The fp8 policy always stages 128 K (two K steps; the pipeline needs an
// even step count), whatever stage depth a tile asks of 8-bit policies.
template <int KS>
using OpF8Any = OpF8T<128>;

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
  static constexpr int kStageK = 64, SA = 128, SB = 64, S = 2;
  static constexpr bool kPingPong = true;
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
      // both K halves of a block go into the same accumulator, first half
      // first; the other blocks' MFMAs sit between the two, so an MFMA never
      // waits on the one issued right before it
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][j] = mfma(f.a[0][i], b0, acc[i][j]);
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][j] = mfma(f.a[1][i], b1, acc[i][j]);
    }
  }
  // Word W (0..3) of a raw 16-code chunk dequantized into its two MFMA
  // operands (word W feeds K half W / 2), for schedules that interleave the
  // dequant with MFMAs one word at a time (gemm_w4a16_kernel).
  template <int W>
  __device__ __forceinline__ static void dequant_word(const i32x4& q, float ws, i32x4 (&b)[2]) {
    uint32_t lo, hi;
    dequant4<BF16, HAS_SCALE>((uint32_t)q[W], ws, lo, hi);
    b[W / 2][2 * (W % 2)] = (int)lo;
    b[W / 2][2 * (W % 2) + 1] = (int)hi;
  }
};

// bf16 x bf16 -> fp32, v_mfma_f32_32x32x16_bf16 (the MOSS bf16 FFN pair):
// both operands staged as 128-byte rows (64 K values); a lane holds 8 K
// values (one chunk), so a stage is 4 K steps of one MFMA each, in natural K
// order on both operands (step s, lane half h: chunk 2s + h).
struct OpBF16T {
  using Acc = f32x16;
  static constexpr int kStageK = 64, SA = 128, SB = 128, S = 4;
  static constexpr bool kPingPong = false;
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
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(f.a[i]),
                                                            bitcast<bf16x8>(f.b[j]), acc[i][j], 0, 0, 0);
  }
};

// ----------------------------------------------------- tile scheduling ---
struct TileCoord { int tm, tn; };

// Remap the dispatch order (blocks go round-robin over the 8 XCDs) so each
// XCD owns a contiguous run of tiles, then raster that run in bands of
// kGroupM tile rows.
__host__ __device__ inline TileCoord tile_of(int bid, int nblocks, int tiles_m, int tiles_n,
                                             int group_m = kGroupM) {
  const int full = nblocks & ~7;
  if (bid < full) bid = (bid & 7) * (full >> 3) + (bid >> 3);
  const int band = group_m * tiles_n;
  const int first_m = (bid / band) * group_m;
  const int gm = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_band = bid - (bid / band) * band;
  TileCoord t;
  t.tm = first_m + in_band % gm;
  t.tn = in_band / gm;
  return t;
}

// A launch covers `count` kernel tiles: mapped tiles first, first+1, ... of
// the tiles_m x tiles_n grid (in tile_of order), each split into sub_m x
// sub_n kernel tiles (1 x 1: the kernel tile is the mapped tile). A large
// GEMM runs its whole rounds of big tiles in one launch and the leftover
// mapped tiles, split, in a second launch of a smaller tile, so that the
// leftover work spreads over every CU.
struct GemmShape {
  int64_t M, N, K;          // N = output columns (pair kernels: 2 * N_out)
  int tiles_m, tiles_n;     // grid of mapped tiles
  int first, count;
  int sub_m, sub_n;
  int group_m = kGroupM;    // tile rows per raster band
};

// Kernel tile i of a launch, in kernel-tile units. Split tiles: the
// dispatch-order remap of tile_of first gives each XCD a contiguous run of
// kernel tiles, so the pieces of one mapped tile share an L2.
__host__ __device__ inline TileCoord tile_at(const GemmShape& sh, int i) {
  const int nmapped = sh.tiles_m * sh.tiles_n;
  if (sh.sub_m == 1 && sh.sub_n == 1)
    return tile_of(sh.first + i, nmapped, sh.tiles_m, sh.tiles_n, sh.group_m);
  const int full = sh.count & ~7;
  if (i < full) i = (i & 7) * (full >> 3) + (i >> 3);
  const int per = sh.sub_m * sh.sub_n;
  const int t = i / per, s = i - t * per;
  const TileCoord b = tile_of(sh.first + t, nmapped, sh.tiles_m, sh.tiles_n, sh.group_m);
  TileCoord r;
  r.tm = b.tm * sh.sub_m + s / sh.sub_n;
  r.tn = b.tn * sh.sub_n + s % sh.sub_n;
  return r;
}

// ------------------------------------------------------------ epilogue ---
// Per 8-row group of each 32-row MFMA block of a wave's sub-tile, through a
// private 8-row LDS strip that lies outside the operand ring (the ring holds
// the next tile's first stages by then):
//   1. raw 32-bit accumulators go in at their (row, column) from the MFMA
//      layout (lane l, register r hold row 8*(r/4) + 4*(l/32) + r%4, column
//      l%32 of a 32x32 block; group q is registers 4q .. 4q+3) -- register
//      moves only;
//   2. each lane takes one row (lane/8) and applies the epilogue to store
//      units of UNIT consecutive columns (16 bytes of output, at most the
//      lane's share): unit h of lane l starts at column UNIT*(8h + l%8), so
//      one store instruction writes 8 whole 16-byte chunks per row, one
//      128-byte line.
// A lane's columns are the same for the whole tile, so their parameters
// (scales, bias) are loaded once per tile; its row parameters are loaded once
// per tile as well (TM*4 rows). Pair strips hold gate and up accumulators
// side by side (2 words per output column).
template <int WORDS>          // 32-bit words per strip row
struct Strip {
  static_assert(WORDS >= 64, "strip rows must span both bank halves");
  static constexpr int kBytes = 8 * WORDS * 4;
  // Rows 4..7 (written by the upper half-wave) keep their words XOR-ed by
  // 32, so the two halves of a phase-1 write land on different banks; runs
  // of 4 aligned words stay contiguous.
  __device__ __forceinline__ static int word(int r, int w) { return r * WORDS + (w ^ ((r & 4) << 3)); }
};

__device__ __forceinline__ void lds_fence_wave() {
  __builtin_amdgcn_s_waitcnt(0xc07f);                     // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
}

// Lane layout of the store phase for COLS output columns of OutT.
template <int COLS, class OutT>
struct StoreMap {
  static constexpr int CPL = COLS / 8;                                  // columns per lane
  static constexpr int UNIT = (16 / (int)sizeof(OutT)) < CPL ? 16 / (int)sizeof(OutT) : CPL;
  static constexpr int UPL = CPL / UNIT;                                // units per lane
  static constexpr int GPU = UNIT / 4;                                  // 4-column groups per unit
  static constexpr int NG = CPL / 4;                                    // groups per lane
  static_assert(UNIT % 4 == 0 && UPL * UNIT == CPL, "bad store map");
  // first column (relative to the sub-tile) of group g = h * GPU + gg
  __device__ __forceinline__ static int col(int lane, int g) {
    return UNIT * ((g / GPU) * 8 + (lane & 7)) + 4 * (g % GPU);
  }
};

// Store one unit (GPU packed 4-column groups) at (m, n .. n+nv-1): one 8- or
// 16-byte store where the row allows, else per group. The 16-byte stores are
// non-temporal: the output is written once and not read back by the kernel,
// and streaming it keeps the A/B panels in cache (MI355X, interleaved A/B:
// fp8 16384x5120->13824 and 16384x13824->5120 +5 %, INT8 pair, W8A16 QKV and
// the int8 WAN shapes within noise).
template <int GPU, class Epi, class Packed>
__device__ __forceinline__ void store_unit(const Epi& epi, int64_t m, int64_t n, int nv,
                                           const Packed* p) {
  if (epi.vec && nv >= 4 * GPU) {
    uint8_t* dst = epi.addr(m, n);
    if constexpr (sizeof(Packed) == 8 && GPU == 2)
      __builtin_nontemporal_store(u32x4{p[0].x, p[0].y, p[1].x, p[1].y}, reinterpret_cast<u32x4*>(dst));
    else if constexpr (sizeof(Packed) == 16)
      __builtin_nontemporal_store(bitcast<u32x4>(p[0]), reinterpret_cast<u32x4*>(dst));
    else
      *reinterpret_cast<Packed*>(dst) = p[0];
    return;
  }
#pragma unroll
  for (int gg = 0; gg < GPU; ++gg) {
    const int k = nv - 4 * gg;
    if (k > 0) store_group(epi, m, n + 4 * gg, k < 4 ? k : 4, p[gg]);
  }
}

// Column parameters of a lane's groups; groups at or past N load nothing
// (nothing is stored for them).
template <class Map, class Epi>
__device__ __forceinline__ void load_cols(const Epi& epi, int64_t n0, int64_t N, int lane,
                                          typename Epi::Col (&col)[Map::NG]) {
#pragma unroll
  for (int g = 0; g < Map::NG; ++g) {
    const int64_t c = n0 + Map::col(lane, g);
    const int64_t k = N - c;
    col[g] = typename Epi::Col{};
    if (k > 0) col[g] = epi.col(c, k < 4 ? (int)k : 4);
  }
}

template <int TM, class Epi>
__device__ __forceinline__ void load_rows(const Epi& epi, int64_t m0, int64_t M, int prow,
                                          float (&rp)[TM][4]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = m0 + i * 32 + q * 8 + prow;
      rp[i][q] = 0.0f;                       // rows past M load nothing
      if (m < M) rp[i][q] = epi.rowp(m);
    }
}

// The epilogue parameters of one wave's sub-tile: its lanes' column groups
// and rows (loaded by load(), or ahead of the epilogue by the kernel).
template <int TM, int TN, bool PAIR, class Epi>
struct EpiParams {
  static constexpr int COLS = PAIR ? TN / 2 * 32 : TN * 32;
  using Map = StoreMap<COLS, typename Epi::OutT>;
  typename Epi::Col col[Map::NG];
  float rp[TM][4];
  // n0: first output column of the sub-tile (pair: first output column)
  __device__ __forceinline__ void load(const Epi& epi, int64_t m0, int64_t n0, int64_t M,
                                       int64_t N) {
    const int lane = threadIdx.x & 63;
    load_cols<Map>(epi, n0, N, lane, col);
    load_rows<TM>(epi, m0, M, lane >> 3, rp);
  }
};

// The same parameters in compact raw form, for loading early: lane l holds
// the raw words of column n0 + l and of rows m0 + l + 64 r. Loading issues
// buffer loads only; nothing reads the words until settle(), so the loads
// are waited for where settle() stands. expand() then spreads them to the
// lanes that use them with cross-lane reads (ds_bpermute: LDS hardware, no
// memory wait) and converts them.
template <int TM, int TN, bool PAIR, class Epi>
struct EpiParamsEarly {
  using Full = EpiParams<TM, TN, PAIR, Epi>;
  static constexpr int F = Epi::kColFields;
  static constexpr int CW = (Full::COLS + 63) / 64;
  static constexpr int RR = (TM * 32 + 63) / 64;
  static_assert(F == 0 || (int)sizeof(typename Epi::Col) == F * 16, "Col is float[F][4]");
  uint32_t cw[F > 0 ? F : 1][CW];
  uint32_t rw[RR];
  __device__ __forceinline__ void load(const Epi& epi, int64_t m0, int64_t n0, int64_t M,
                                       int64_t N) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
      for (int w = 0; w < CW; ++w) cw[f][w] = epi.col_raw(f, n0 + lane + 64 * w, N);
#pragma unroll
    for (int r = 0; r < RR; ++r) rw[r] = epi.row_raw(m0 + lane + 64 * r, M);
  }
  __device__ __forceinline__ void settle() {
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
      for (int w = 0; w < CW; ++w) asm volatile("" : "+v"(cw[f][w]));
#pragma unroll
    for (int r = 0; r < RR; ++r) asm volatile("" : "+v"(rw[r]));
  }
  // The column words converted to f32 bits (col_val applied once per word,
  // before the cross-lane reads that spread them).
  __device__ __forceinline__ EpiParamsEarly converted(const Epi& epi) const {
    EpiParamsEarly c = *this;
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
      for (int w = 0; w < CW; ++w) c.cw[f][w] = f32_bits(epi.col_val(f, cw[f][w]));
    return c;
  }
  __device__ __forceinline__ void expand(const Epi& epi, Full& out) const {
    using Map = typename Full::Map;
    const int lane = threadIdx.x & 63, prow = lane >> 3;
    const EpiParamsEarly cv = converted(epi);
    if constexpr (F > 0) {
#pragma unroll
      for (int g = 0; g < Map::NG; ++g) {
        // a group's columns lie in one 64-column word: w is the same for
        // every lane (unit starts are UNIT * 8 apart, UNIT * 8 <= 64)
        const int w = (Map::UNIT * 8 * (g / Map::GPU)) >> 6;
        struct { float v[F][4]; } c;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int src = Map::col(lane, g) + q - 64 * w;
#pragma unroll
          for (int f = 0; f < F; ++f) c.v[f][q] = bits_f32((uint32_t)__shfl((int)cv.cw[f][w], src));
        }
        out.col[g] = __builtin_bit_cast(typename Epi::Col, c);
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r0 = i * 32 + q * 8;              // + prow < 8: stays in one 64-row word
        out.rp[i][q] = bits_f32((uint32_t)__shfl((int)rw[r0 >> 6], (r0 & 63) + prow));
      }
  }
};

// Calls f(std::integral_constant<int, V>{}) with V = epi.variant() (a
// wave-uniform bit mask of the functor's optional terms), so that the store
// loop instantiated for V has no per-element test of them. Measured on
// MI355X against per-element tests and a runtime output type (same process,
// same box): C3 fp8 up +4.5 %, C2 W8A16 +2.1 %, C4 pair +1.8 %.
template <class Epi, class F>
__device__ __forceinline__ void with_variant(const Epi& epi, F&& f) {
  if constexpr (Epi::kVariants == 1) {
    f(std::integral_constant<int, 0>{});
  } else if constexpr (Epi::kVariants == 2) {
    if (epi.variant() == 1) f(std::integral_constant<int, 1>{});
    else f(std::integral_constant<int, 0>{});
  } else {
    switch (epi.variant()) {
      case 1: f(std::integral_constant<int, 1>{}); break;
      case 2: f(std::integral_constant<int, 2>{}); break;
      case 3: f(std::integral_constant<int, 3>{}); break;
      default: f(std::integral_constant<int, 0>{}); break;
    }
  }
}

// Epilogues with an element-wise term (E::kElem): elem(m, n, nv, packed)
// is applied to each 4-column group after apply().
template <class E, class = void> struct HasElem : std::false_type {};
template <class E>
struct HasElem<E, std::void_t<decltype(E::kElem)>> : std::bool_constant<E::kElem> {};

template <int V, int TM, int TN, class Acc, class Epi, class Params>
__device__ __forceinline__ void epilogue_single_v(const Acc (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                  int64_t M, int64_t N, const Epi& epi, uint8_t* lds,
                                                  const Params& pr) {
  using Scalar = std::remove_cv_t<std::remove_reference_t<decltype(acc[0][0][0])>>;
  constexpr int COLS = TN * 32;
  using Map = StoreMap<COLS, typename Epi::OutT>;
  using St = Strip<COLS>;
  using Packed = typename Epi::Packed;
  Scalar* sw = reinterpret_cast<Scalar*>(lds);
  const int lane = threadIdx.x & 63, prow = lane >> 3;
  const auto& col = pr.col;
  const auto& rp = pr.rp;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sw[St::word((lane >> 5) * 4 + r, j * 32 + (lane & 31))] = acc[i][j][4 * q + r];
      lds_fence_wave();
      const int64_t m = m0 + i * 32 + q * 8 + prow;
      if (m < M) {
#pragma unroll
        for (int h = 0; h < Map::UPL; ++h) {
          const int c = Map::col(lane, h * Map::GPU);
          const int64_t nv = N - (n0 + c);
          if (nv <= 0) continue;
          Packed out[Map::GPU];
#pragma unroll
          for (int gg = 0; gg < Map::GPU; ++gg) {
            const Scalar* w = sw + St::word(prow, c + 4 * gg);
            const Scalar v[4] = {w[0], w[1], w[2], w[3]};
            out[gg] = epi.template apply<V>(rp[i][q], col[h * Map::GPU + gg], v);
            if constexpr (HasElem<Epi>::value) {
              const int64_t kv = nv - 4 * gg;
              if (kv > 0) out[gg] = epi.elem(m, n0 + c + 4 * gg, kv < 4 ? (int)kv : 4, out[gg]);
            }
          }
          store_unit<Map::GPU>(epi, m, n0 + c, nv < Map::UNIT ? (int)nv : Map::UNIT, out);
        }
      }
      lds_fence_wave();
    }
  }
}

// Pair epilogue: blocks 2t (gate) and 2t+1 (up) give the same 32 output
// columns c0 + 32 t + lane%32; the strip interleaves them per column.
template <int TM, int TN, class Acc, class Epi, class Params>
__device__ __forceinline__ void epilogue_single(const Acc (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                int64_t M, int64_t N, const Epi& epi, uint8_t* lds,
                                                const Params& pr) {
  with_variant(epi, [&](auto vc) {
    epilogue_single_v<decltype(vc)::value, TM, TN>(acc, m0, n0, M, N, epi, lds, pr);
  });
}

template <int V, int TM, int TN, class Acc, class Epi, class Params>
__device__ __forceinline__ void epilogue_pair_v(const Acc (&acc)[TM][TN], int64_t m0, int64_t c0,
                                                int64_t M, int64_t NC, const Epi& epi, uint8_t* lds,
                                                const Params& pr) {
  using Scalar = std::remove_cv_t<std::remove_reference_t<decltype(acc[0][0][0])>>;
  constexpr int COLS = TN / 2 * 32;
  using Map = StoreMap<COLS, typename Epi::OutT>;
  using St = Strip<2 * COLS>;
  Scalar* sw = reinterpret_cast<Scalar*>(lds);
  const int lane = threadIdx.x & 63, prow = lane >> 3;
  const auto& col = pr.col;
  const auto& rp = pr.rp;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int t = 0; t < TN / 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int x = St::word((lane >> 5) * 4 + r, 2 * (t * 32 + (lane & 31)));
          sw[x] = acc[i][2 * t][4 * q + r];
          sw[x + 1] = acc[i][2 * t + 1][4 * q + r];
        }
      lds_fence_wave();
      const int64_t m = m0 + i * 32 + q * 8 + prow;
      if (m < M) {
#pragma unroll
        for (int h = 0; h < Map::UPL; ++h) {
          const int c = Map::col(lane, h * Map::GPU);
          const int64_t nv = NC - (c0 + c);
          if (nv <= 0) continue;
          uint2 out[Map::GPU];
#pragma unroll
          for (int gg = 0; gg < Map::GPU; ++gg) {
            const Scalar* w = sw + St::word(prow, 2 * (c + 4 * gg));
            const Scalar gv[4] = {w[0], w[2], w[4], w[6]};
            const Scalar uv[4] = {w[1], w[3], w[5], w[7]};
            out[gg] = epi.template apply<V>(rp[i][q], col[h * Map::GPU + gg], gv, uv);
          }
          store_unit<Map::GPU>(epi, m, c0 + c, nv < Map::UNIT ? (int)nv : Map::UNIT, out);
        }
      }
      lds_fence_wave();
    }
  }
}

template <int TM, int TN, class Acc, class Epi, class Params>
__device__ __forceinline__ void epilogue_pair(const Acc (&acc)[TM][TN], int64_t m0, int64_t c0,
                                              int64_t M, int64_t NC, const Epi& epi, uint8_t* lds,
                                              const Params& pr) {
  with_variant(epi, [&](auto vc) {
    epilogue_pair_v<decltype(vc)::value, TM, TN>(acc, m0, c0, M, NC, epi, lds, pr);
  });
}

// Epilogues that reduce over whole 128-column heads (EpiQKVNormRope).
template <class E, class = void> struct IsHeadNorm : std::false_type {};
template <class E>
struct IsHeadNorm<E, std::void_t<decltype(E::kHeadNorm)>> : std::bool_constant<E::kHeadNorm> {};

// Q/K RMSNorm + partial RoPE epilogue of a wave whose sub-tile spans one
// head: 128 columns starting at n0, a multiple of 128, so the kind (Q, K or
// V) and the head are the same for the whole sub-tile, and output row m of
// it is the 256 contiguous bytes at hb + 256 m. R (rotation pairs) is a
// multiple of 8 here, so each 8-column unit of a lane lies wholly in the
// first rotated half (d < R), the second (R <= d < 2R) or the pass-through
// part (d >= 2R): the per-element arithmetic is branch-free, with per-unit
// constants set once per tile. Per strip of 8 rows:
//   1. the accumulators pass through the strip as in epilogue_single; lane l
//      forms the bf16 projection values of row l/8, columns c0 + k for its
//      units c0 = 64 h + 8 (l%8), exactly the QKV scatter's values;
//   2. V: stored as they are;
//   3. Q, K: head_rms_norm over the 8 lanes of the row; the normalized
//      values go back to the strip, each lane reads the 8 RoPE partners of
//      each unit (columns c0 + R or c0 - R) and applies rope_split_half.
// The row scale of the next strip is loaded one strip ahead, and with
// AHEAD (a wave that has the register file of its SIMD to itself) the freqs
// words as well; otherwise they load at the strip's RoPE step.
template <int TM, int TN, bool AHEAD, class Acc, class Epi, class Params>
__device__ __forceinline__ void epilogue_head_norm(const Acc (&acc)[TM][TN], int64_t m0, int64_t n0,
                                                   int64_t M, int64_t N, const Epi& epi,
                                                   uint8_t* lds, const Params& pr) {
  static_assert(TN == 4, "head epilogue: a wave's sub-tile spans one 128-column head");
  constexpr int COLS = TN * 32;
  using Map = StoreMap<COLS, typename Epi::OutT>;
  static_assert(Map::UNIT == 8 && Map::UPL == 2 && Map::GPU == 2, "head epilogue lane map");
  using St = Strip<COLS>;
  if (n0 >= N) return;                                   // wave-uniform: past the last head
  int32_t* sw = reinterpret_cast<int32_t*>(lds);
  float* sf = reinterpret_cast<float*>(lds);
  const int lane = threadIdx.x & 63, prow = lane >> 3;
  const uint32_t kind = (uint32_t)n0 / epi.width;        // 0 Q, 1 K, 2 V
  uint8_t* const hb = epi.addr(0, n0);                   // row 0 of this head
  const int R = epi.pairs;
  // per unit h: its first column, where its partners start, the byte offset
  // of its first freqs word in a freqs row, the half-swap of those words
  // (second half: the diagonal factor is the high bf16), pass-through
  int c0[2], pc[2], fo[2];
  uint32_t swap[2];
  bool pass[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    c0[h] = Map::col(lane, 2 * h);
    const bool first = c0[h] < R, second = !first && c0[h] < 2 * R;
    pass[h] = !first && !second;
    pc[h] = first ? c0[h] + R : (second ? c0[h] - R : c0[h]);
    fo[h] = first ? 8 * c0[h] : (second ? 8 * (c0[h] - R) + 4 : 0);
    swap[h] = second ? 16u : 0u;
  }
  float w[16];
  float rsv = epi.rowp(m0 + prow < M ? m0 + prow : M - 1);   // row scale, current strip
  uint32_t fw[16];                                       // freqs words, current strip
  // word k of unit h in freqs row m (clamped into [0, M)): freqs[m, i, r]
  // for column c0 + k = i + r R
  auto load_freqs = [&](int64_t m) __attribute__((always_inline)) {
    const uint8_t* fr = reinterpret_cast<const uint8_t*>(epi.freqs) + (m < M ? m : M - 1) * R * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (!pass[h]) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(fr + fo[h]);
#pragma unroll
        for (int k = 0; k < 8; ++k) fw[8 * h + k] = p[2 * k];
      }
    }
  };
  if (kind < 2) {
    const float* wp = epi.weight(kind);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < 8; k += 4) {
        const float4 f = *reinterpret_cast<const float4*>(wp + c0[h] + k);
        w[8 * h + k] = f.x; w[8 * h + k + 1] = f.y; w[8 * h + k + 2] = f.z; w[8 * h + k + 3] = f.w;
      }
    if constexpr (AHEAD) load_freqs(m0 + prow);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sw[St::word((lane >> 5) * 4 + r, j * 32 + (lane & 31))] = acc[i][j][4 * q + r];
      lds_fence_wave();
      const int64_t m = m0 + i * 32 + q * 8 + prow;
      uint2 pv[4];                                        // group g = 2 h + gg: 4 columns
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int32_t* s = sw + St::word(prow, Map::col(lane, g));
        const int32_t v[4] = {s[0], s[1], s[2], s[3]};
        pv[g] = epi.apply(rsv, pr.col[g], v);
      }
      const bool more = i * 4 + q + 1 < TM * 4;
      if (more) rsv = epi.rowp(m + 8 < M ? m + 8 : M - 1);
      uint8_t* const dst = hb + m * 256;
      if (kind == 2) {
        if (m < M) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *reinterpret_cast<uint4*>(dst + 2 * c0[h]) =
                uint4{pv[2 * h].x, pv[2 * h].y, pv[2 * h + 1].x, pv[2 * h + 1].y};
        }
      } else {
        float x[16], y[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          x[4 * g] = bf16lo(pv[g].x); x[4 * g + 1] = bf16hi(pv[g].x);
          x[4 * g + 2] = bf16lo(pv[g].y); x[4 * g + 3] = bf16hi(pv[g].y);
        }
        head_rms_norm(x, w, epi.eps, y);
        // each lane overwrites only the strip words it read itself
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int k = 0; k < 8; k += 4)
            *reinterpret_cast<float4*>(sf + St::word(prow, c0[h] + k)) =
                float4{y[8 * h + k], y[8 * h + k + 1], y[8 * h + k + 2], y[8 * h + k + 3]};
        if constexpr (!AHEAD) load_freqs(m);
        lds_fence_wave();
        uint4 ov[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float yp[8], o[8];
#pragma unroll
          for (int k = 0; k < 8; k += 4) {
            const float4 t = *reinterpret_cast<const float4*>(sf + St::word(prow, pc[h] + k));
            yp[k] = t.x; yp[k + 1] = t.y; yp[k + 2] = t.z; yp[k + 3] = t.w;
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t f = __builtin_amdgcn_alignbit(fw[8 * h + k], fw[8 * h + k], swap[h]);
            const float r = rope_split_half(y[8 * h + k], yp[k], f, false);
            o[k] = pass[h] ? y[8 * h + k] : r;
          }
          ov[h] = uint4{bf16x2_rne(o[0], o[1]), bf16x2_rne(o[2], o[3]), bf16x2_rne(o[4], o[5]),
                        bf16x2_rne(o[6], o[7])};
        }
        // the next strip's freqs load under this strip's stores and the
        // next strip's transpose and norm
        if constexpr (AHEAD) {
          if (more) load_freqs(m + 8);
        }
        if (m < M) {
#pragma unroll
          for (int h = 0; h < 2; ++h) *reinterpret_cast<uint4*>(dst + 2 * c0[h]) = ov[h];
        }
      }
      lds_fence_wave();
    }
  }
}

// --------------------------------------------------------- main kernel ---

// Operand sources: base pointers and strides; each workgroup derives its
// tiles' buffer resources from them.
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

// stage_barrier with the LDS wait issued as a builtin, so the compiler's
// wait insertion knows every LDS read before it has completed and adds no
// waits of its own for them afterwards.
__device__ __forceinline__ void stage_barrier_tracked() {
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0); vmcnt and expcnt unconstrained
  asm volatile("s_barrier" ::: "memory");
}

// Bytes of one wave's epilogue strip.
template <int TN, bool PAIR>
constexpr int strip_bytes() { return Strip<(PAIR ? TN / 2 * 2 : TN) * 32>::kBytes; }

// Persistent kernel: workgroup b takes tiles b, b + G, b + 2G, ... (G =
// gridDim.x) in the XCD-aware order of tile_of, and runs one copy ring
// through all of them: the last stages of a tile already copy the next
// tile's first stages, which land while the epilogue stores.
//
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
  constexpr int SA = Op::SA, SB = Op::SB, S = Op::S;
  static_assert(S % 2 == 0, "the fragment double buffer assumes an even step count per stage");
  constexpr int STAGE = BM * SA + BN * SB;
  constexpr int RING = NBUF * STAGE;
  constexpr int kStrip = strip_bytes<TN, PAIR>();
  static_assert(NBUF >= 2 && RING + kStrip * WM * WN <= 160 * 1024, "LDS exceeds 160 KB");
  using LA = DirectLoad<BM, SA, NT, false>;
  using LB = DirectLoad<BN, SB, NT, PAIR>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING + kStrip * WM * WN];

  const int ntiles = sh.count;
  const int G = (int)gridDim.x;
  const int my_tiles = (ntiles - 1 - (int)blockIdx.x) / G + 1;
  const Epi ep = epi.prepare();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int wm = wave / WN, wn = wave % WN;
  const float ws = Op::prep_scale(b_scale);

  LA la;
  LB lb;
  la.init(sa.ld_bytes, wave, 0);
  lb.init(sb.ld_bytes, wave, 0);
  constexpr int KS = Op::kStageK;
  const int a_kb = (int)(sh.K * SA / KS), b_kb = (int)(sh.K * SB / KS);
  const int nst = (int)((sh.K + KS - 1) / KS);

  // Copy cursor: next stage to issue is stage ips of this workgroup's tile ij.
  int ij = 0, ips = 0;
  u32x4 ra, rb0, rb1;
  auto tile_rsrc = [&](int j) __attribute__((always_inline)) {
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t m0 = (int64_t)tc.tm * BM;
    const int64_t brow0 = PAIR ? ((int64_t)tc.tn * BN >> 1) : (int64_t)tc.tn * BN;
    const int64_t bleft = (sb.rows - brow0) * sb.ld_bytes;
    ra = dma_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
    rb0 = dma_rsrc(sb.p0 + brow0 * sb.ld_bytes, bleft);
    rb1 = PAIR ? dma_rsrc(sb.p1 + brow0 * sb.ld_bytes, bleft) : rb0;
  };
  // Issue the next stage into `buf`; past this workgroup's last tile the
  // copies read zeros (every stage issues the same number of copies, which
  // keeps the vmcnt arithmetic fixed).
  auto issue_next = [&](uint8_t* buf) __attribute__((always_inline)) {
    if (ij < my_tiles) {
      la.issue(ra, ra, buf, ips * SA, a_kb);
      lb.issue(rb0, rb1, buf + BM * SA, ips * SB, b_kb);
      if (++ips == nst) {
        ips = 0;
        if (++ij < my_tiles) tile_rsrc(ij);
      }
    } else {
      la.issue(ra, ra, buf, 0, 0);
      lb.issue(rb0, rb1, buf + BM * SA, 0, 0);
    }
  };
  tile_rsrc(0);

  // prologue: stages 0 .. NBUF-1 in flight, stage 0 complete and visible
#pragma unroll
  for (int p = 0; p < NBUF; ++p) issue_next(smem + p * STAGE);
  wait_vm<(NBUF - 1) * kPerStage>();
  stage_barrier();

  // K-step pipeline: the fragments of the next step are read while the
  // current step multiplies. The stage barrier sits before the last step of
  // each stage, whose fragments are already in registers: after it the
  // next stage is visible (its first fragments load under the last step's
  // MFMAs) and the stage just read is free to refill.
  const int ra0 = wm * (TM * 32), rb0i = wn * (TN * 32);
  // Eight waves (two per SIMD) and at least four K steps per stage: the
  // upper four waves issue their copies after the last step's MFMAs instead
  // of right after the barrier, so that on every SIMD one wave feeds the
  // matrix pipe while the other waits for the address unit to take its
  // copies (int8 128-K stages: +1-5 %). With two steps per stage (fp8,
  // W8A16) that delay is half a stage of the copies' latency budget in the
  // two-stage ring, and costs 14 % (fp8).
  const bool late = WM * WN == 8 && S >= 4 && wave >= 4;
  using Frag = typename Op::template Frag<TM, TN>;
  Frag fr[2];
  uint8_t* strip = smem + RING + wave * kStrip;
  int gs = 0;                                   // stage counter over all tiles
  for (int j = 0; j < my_tiles; ++j) {
    typename Op::Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0;
    {
      const uint8_t* cur = smem + (gs % NBUF) * STAGE;
      Op::template frags<TM, TN>(fr[0], cur, cur + BM * SA, ra0, rb0i, 0);
    }
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t wm0 = (int64_t)tc.tm * BM + wm * (TM * 32);
    const int64_t wn0 = PAIR ? ((int64_t)tc.tn * BN >> 1) + wn * (TN * 16)
                             : (int64_t)tc.tn * BN + wn * (TN * 32);
    EpiParams<TM, TN, PAIR, Epi> prm;
    EpiParamsEarly<TM, TN, PAIR, Epi> early;
    // One stage; LAST: the tile's last stage, after which the epilogue runs.
    // With a two-stage ring every stage ends by waiting for all of this
    // wave's copies (vmcnt(0)). The last stage then loads the epilogue
    // parameters (raw, compact) first and settles them right after that
    // wait, before the next tile's first copies are issued: loaded later,
    // they would be newer than those copies, and their first use would wait
    // for the copies too (memory counters complete in issue order).
    // (Only where the early parameters fit: at most 8 accumulator blocks per
    // wave; larger wave tiles keep one loop and load them at the epilogue.)
    constexpr bool kEarlyParams = NBUF == 2 && TM * TN <= 8;
    auto stage = [&](auto last, bool has_next) __attribute__((always_inline)) {
      constexpr bool kEarly = decltype(last)::value && kEarlyParams;
      if constexpr (kEarly) early.load(ep, wm0, wn0, sh.M, PAIR ? sh.N >> 1 : sh.N);
      uint8_t* cur = smem + (gs % NBUF) * STAGE;
      const uint8_t* nxt = smem + ((gs + 1) % NBUF) * STAGE;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if (s == S - 1) {
          wait_vm<(NBUF - 2) * kPerStage>();   // this wave's copies of stage gs+1 landed
          if constexpr (kEarly) early.settle();
          stage_barrier();                     // ... and every wave's; stage gs fully read
          if (!late) issue_next(cur);          // refill with stage gs+NBUF
          if (has_next) Op::template frags<TM, TN>(fr[0], nxt, nxt + BM * SA, ra0, rb0i, 0);
        } else {
          Op::template frags<TM, TN>(fr[(s + 1) & 1], cur, cur + BM * SA, ra0, rb0i, s + 1);
          // keep the next step's LDS reads ahead of this step's MFMAs: left to
          // the scheduler they sink behind most of them, and the LDS latency
          // then lands on the stage barrier (2-4% on the large shapes)
          __builtin_amdgcn_sched_barrier(0);
        }
        Op::template mma<TM, TN>(fr[s & 1], acc, ws);
        if (s == S - 1 && late) {
          __builtin_amdgcn_sched_barrier(0);
          issue_next(cur);
        }
      }
      ++gs;
    };
    if constexpr (kEarlyParams) {
      for (int st = 0; st + 1 < nst; ++st) stage(std::false_type{}, true);
      stage(std::true_type{}, false);
      early.expand(ep, prm);
    } else {
      for (int st = 0; st < nst; ++st) stage(std::false_type{}, st + 1 < nst);
      prm.load(ep, wm0, wn0, sh.M, PAIR ? sh.N >> 1 : sh.N);
    }
    if constexpr (PAIR) {
      epilogue_pair<TM, TN>(acc, wm0, wn0, sh.M, sh.N >> 1, ep, strip, prm);
    } else if constexpr (IsHeadNorm<Epi>::value) {
      epilogue_head_norm<TM, TN, (WM * WN <= 4)>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
    } else {
      epilogue_single<TM, TN>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
    }
  }
  wait_vm<0>();    // zero-fill copies past the last tile still target the ring
}

// Ping-pong schedule of the 8-wave tile (WM = 2, WN = 4). The two wave
// rows are two groups (waves 0-3 and 4-7, one of each on every SIMD) that
// own the upper and lower halves of the tile and run half a stage apart:
//
//   group 0:  | mem k   | mma k   | mem k+1 | mma k+1 | ...
//   group 1:  |         | mem k   | mma k   | mem k+1 | ...
//                       ^ one workgroup barrier between intervals
//
// In its memory interval a group reads all fragments of stage k from LDS
// and issues its half of the copies of stage k + NBUF - 1 (its A rows, half
// of the B rows) into the buffer both groups finished reading one interval
// earlier; in its MFMA interval it multiplies from registers only. Each
// SIMD's MFMA pipe is fed by one group while the other group's LDS reads,
// copies and address work proceed, instead of both waves of a SIMD wanting
// the MFMA pipe and the LDS at the same moments. A tile's epilogue runs in
// its group's next memory interval. Stage k (both halves) is complete before
// barrier 2k, where group 0 starts reading it: group 0 waits for its copies
// at the end of its MFMA interval, group 1 at the end of its memory
// interval, in both cases for the copies it issued NBUF - 2 stages earlier.
template <class Op, int BM, int BN, int NBUF, bool PAIR, class Epi>
__global__ void __launch_bounds__(512)
gemm_pingpong_kernel(GemmShape sh, Src2 sa, Src2 sb, const float* b_scale, Epi epi) {
  constexpr int WM = 2, WN = 4, NT = 512;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && TM * WM * 32 == BM && TN * WN * 32 == BN, "bad wave tiling");
  static_assert(!PAIR || (TN % 2 == 0), "pair tiles need whole gate/up block pairs");
  static_assert((BM / 2) % 64 == 0 && (BN / 2) % 64 == 0, "group halves must align to 64 rows");
  constexpr int SA = Op::SA, SB = Op::SB, S = Op::S;
  constexpr int STAGE = BM * SA + BN * SB;
  constexpr int RING = NBUF * STAGE;
  constexpr int kStrip = strip_bytes<TN, PAIR>();
  static_assert(NBUF >= 3 && RING + kStrip * WM * WN <= 160 * 1024, "LDS exceeds 160 KB");
  using LA = DirectLoad<BM / 2, SA, NT / 2, false>;
  using LB = DirectLoad<BN / 2, SB, NT / 2, PAIR>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING + kStrip * WM * WN];

  const int ntiles = sh.count;
  const int G = (int)gridDim.x;
  const int my_tiles = (ntiles - 1 - (int)blockIdx.x) / G + 1;
  const Epi ep = epi.prepare();
  const int wave = threadIdx.x >> 6;
  const int grp = __builtin_amdgcn_readfirstlane(wave >> 2), wn = wave & 3;
  const float ws = Op::prep_scale(b_scale);

  LA la;
  LB lb;
  la.init(sa.ld_bytes, wn, grp * (BM / 2));
  lb.init(sb.ld_bytes, wn, grp * (BN / 2));
  constexpr int KS = Op::kStageK;
  const int a_kb = (int)(sh.K * SA / KS), b_kb = (int)(sh.K * SB / KS);
  const int nst = (int)((sh.K + KS - 1) / KS);

  int ij = 0, ips = 0;
  u32x4 ra, rb0, rb1;
  auto tile_rsrc = [&](int j) __attribute__((always_inline)) {
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t m0 = (int64_t)tc.tm * BM;
    const int64_t brow0 = PAIR ? ((int64_t)tc.tn * BN >> 1) : (int64_t)tc.tn * BN;
    const int64_t bleft = (sb.rows - brow0) * sb.ld_bytes;
    ra = dma_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
    rb0 = dma_rsrc(sb.p0 + brow0 * sb.ld_bytes, bleft);
    rb1 = PAIR ? dma_rsrc(sb.p1 + brow0 * sb.ld_bytes, bleft) : rb0;
  };
  auto issue_next = [&](uint8_t* buf) __attribute__((always_inline)) {
    if (ij < my_tiles) {
      la.issue(ra, ra, buf, ips * SA, a_kb);
      lb.issue(rb0, rb1, buf + BM * SA, ips * SB, b_kb);
      if (++ips == nst) {
        ips = 0;
        if (++ij < my_tiles) tile_rsrc(ij);
      }
    } else {
      la.issue(ra, ra, buf, 0, 0);
      lb.issue(rb0, rb1, buf + BM * SA, 0, 0);
    }
  };
  tile_rsrc(0);

  // prologue: stages 0 .. NBUF-2 in flight; stage 0 complete and visible
#pragma unroll
  for (int p = 0; p < NBUF - 1; ++p) issue_next(smem + p * STAGE);
  wait_vm<(NBUF - 2) * kPerStage>();
  stage_barrier();
  if (grp == 1) stage_barrier();               // group 1 runs one interval behind

  const int ra0 = grp * (TM * 32), rb0i = wn * (TN * 32);
  using Frag = typename Op::template Frag<TM, TN>;
  Frag fr[S];
  uint8_t* strip = smem + RING + wave * kStrip;
  typename Op::Acc acc[TM][TN];
  int gs = 0;                                   // stage counter over all tiles
  for (int j = 0; j < my_tiles; ++j) {
    for (int st = 0; st < nst; ++st, ++gs) {
      // memory interval
      const uint8_t* cur = smem + (gs % NBUF) * STAGE;
#pragma unroll
      for (int s = 0; s < S; ++s) Op::template frags<TM, TN>(fr[s], cur, cur + BM * SA, ra0, rb0i, s);
      issue_next(smem + ((gs + NBUF - 1) % NBUF) * STAGE);
      if (grp == 1) wait_vm<(NBUF - 2) * kPerStage>();
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // MFMA interval
      if (st == 0) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < TN; ++jj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0;
      }
#pragma unroll
      for (int s = 0; s < S; ++s) Op::template mma<TM, TN>(fr[s], acc, ws);
      if (grp == 0) wait_vm<(NBUF - 2) * kPerStage>();
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t wm0 = (int64_t)tc.tm * BM + grp * (TM * 32);
    const int64_t wn0 = PAIR ? ((int64_t)tc.tn * BN >> 1) + wn * (TN * 16)
                             : (int64_t)tc.tn * BN + wn * (TN * 32);
    EpiParams<TM, TN, PAIR, Epi> prm;
    prm.load(ep, wm0, wn0, sh.M, PAIR ? sh.N >> 1 : sh.N);
    if constexpr (PAIR) {
      epilogue_pair<TM, TN>(acc, wm0, wn0, sh.M, sh.N >> 1, ep, strip, prm);
    } else {
      epilogue_single<TM, TN>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
    }
  }
  if (grp == 0) stage_barrier();               // matches group 1's extra barrier
  wait_vm<0>();    // zero-fill copies past the last tile still target the ring
}

// One wave per SIMD: a 256 x 256 tile of four waves of 128 x 128 (16
// accumulator blocks, 256 accumulation registers each), 8-bit operands
// through a ring of NBUF stages (fp8: two 128-K stages). With one wave on a
// SIMD nothing covers a stall of that wave, so each K step is issued as one
// interleaved stream: after every MFMA the wave issues the fragment reads
// that the MFMA freed (fragments are refilled in place for the next step)
// and, in the stage's last step, after the barrier that frees the stage's
// buffer, one of its copies of stage gs + NBUF. LDS reads and copy issue
// then run under the MFMAs. Each accumulator takes its K steps in the same
// order as in gemm_tile_kernel, so the results are the same bits.
// Measured on MI355X against the 8-wave kernel on the same tile (fp8, 16384
// rows): per 128-K stage the MFMAs take ~2000 cycles, the fragment reads
// add ~120 and the copy issue ~500 (the address unit is saturated while the
// copies of a stage are issued in its last step); the epilogue is ~27k
// cycles per tile and is not overlapped.
template <class Op, int NBUF, bool PAIR, class Epi>
__global__ void __launch_bounds__(256)
gemm_w4_kernel(GemmShape sh, Src2 sa, Src2 sb, const float* b_scale, Epi epi) {
  constexpr int BM = 256, BN = 256, WM = 2, WN = 2, NT = 256;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(!PAIR || (TN % 2 == 0), "pair tiles need whole gate/up block pairs");
  constexpr int SA = Op::SA, SB = Op::SB, S = Op::S;
  constexpr int STAGE = BM * SA + BN * SB;
  constexpr int RING = NBUF * STAGE;
  constexpr int kStrip = strip_bytes<TN, PAIR>();
  static_assert(NBUF >= 2 && RING + kStrip * WM * WN <= 160 * 1024, "LDS exceeds 160 KB");
  using LA = DirectLoad<BM, SA, NT, false>;
  using LB = DirectLoad<BN, SB, NT, PAIR>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  constexpr int kMfma = TM * TN;                          // MFMAs per K step
  static_assert(kMfma % kPerStage == 0, "one MFMA slot per copy");
  constexpr int kCopyEvery = kMfma / kPerStage;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING + kStrip * WM * WN];

  const int ntiles = sh.count;
  const int G = (int)gridDim.x;
  const int my_tiles = (ntiles - 1 - (int)blockIdx.x) / G + 1;
  const Epi ep = epi.prepare();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int wm = wave / WN, wn = wave % WN;

  LA la;
  LB lb;
  la.init(sa.ld_bytes, wave, 0);
  lb.init(sb.ld_bytes, wave, 0);
  constexpr int KS = Op::kStageK;
  const int a_kb = (int)(sh.K * SA / KS), b_kb = (int)(sh.K * SB / KS);
  const int nst = (int)((sh.K + KS - 1) / KS);

  // Copy cursor: next stage to issue is stage ips of this workgroup's tile ij.
  int ij = 0, ips = 0;
  u32x4 ra, rb0, rb1;
  auto tile_rsrc = [&](int j) __attribute__((always_inline)) {
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t m0 = (int64_t)tc.tm * BM;
    const int64_t brow0 = PAIR ? ((int64_t)tc.tn * BN >> 1) : (int64_t)tc.tn * BN;
    const int64_t bleft = (sb.rows - brow0) * sb.ld_bytes;
    ra = dma_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
    rb0 = dma_rsrc(sb.p0 + brow0 * sb.ld_bytes, bleft);
    rb1 = PAIR ? dma_rsrc(sb.p1 + brow0 * sb.ld_bytes, bleft) : rb0;
  };
  // Copy C of the next stage (A copies first) into `buf`. Past this
  // workgroup's last tile the copies read zeros (k limit 0), so every stage
  // issues the same number of copies and the vmcnt arithmetic stays fixed.
  auto issue_copy = [&](auto cc, uint8_t* buf, bool live) __attribute__((always_inline)) {
    constexpr int C = decltype(cc)::value;
    if constexpr (C < LA::kInstr) {
      la.template issue_one<C>(ra, ra, buf, live ? ips * SA : 0, live ? a_kb : 0);
    } else {
      lb.template issue_one<C - LA::kInstr>(rb0, rb1, buf + BM * SA, live ? ips * SB : 0,
                                            live ? b_kb : 0);
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (ij < my_tiles && ++ips == nst) {
      ips = 0;
      if (++ij < my_tiles) tile_rsrc(ij);
    }
  };
  tile_rsrc(0);

  // prologue: stages 0 .. NBUF-1 in flight, stage 0 complete and visible
#pragma unroll
  for (int p = 0; p < NBUF; ++p) {
    const bool live = ij < my_tiles;
    static_for<0, kPerStage>([&](auto cc) { issue_copy(cc, smem + p * STAGE, live); });
    advance();
  }
  wait_vm<(NBUF - 1) * kPerStage>();
  stage_barrier();

  const int ra0 = wm * (TM * 32), rb0i = wn * (TN * 32);
  using Frag = typename Op::template Frag<TM, TN>;
  Frag fr;
  Op::template frags<TM, TN>(fr, smem, smem + BM * SA, ra0, rb0i, 0);
  uint8_t* strip = smem + RING + wave * kStrip;
  int gs = 0;                                   // stage counter over all tiles
  for (int j = 0; j < my_tiles; ++j) {
    typename Op::Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0;
    // One stage. The fragments live in one set of registers, refilled in
    // place for the next K step: A block i right after its last MFMA (row
    // i, column TN-1), B block j right after its last (row TM-1, column j),
    // so the reads of the next step run under this step's remaining MFMAs.
    // The last step first waits for this wave's copies of stage gs + 1, then
    // the barrier makes every wave's copies visible and frees stage gs's
    // buffer (all its reads happened in earlier steps); that step's refills
    // read stage gs + 1, and its copies refill the freed buffer with stage
    // gs + NBUF.
    auto stage = [&]() __attribute__((always_inline)) {
      uint8_t* cur = smem + (gs % NBUF) * STAGE;
      const uint8_t* nxt = smem + ((gs + 1) % NBUF) * STAGE;
      static_for<0, S>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        constexpr bool kLast = s == S - 1;
        if constexpr (kLast) {
          wait_vm<(NBUF - 2) * kPerStage>();
          stage_barrier_tracked();
        }
        const uint8_t* src = kLast ? nxt : cur;
        constexpr int fs = kLast ? 0 : s + 1;
        const bool live = ij < my_tiles;
        static_for<0, kMfma>([&](auto qc) {
          constexpr int q = decltype(qc)::value, i = q / TN, jn = q % TN;
          Op::template mma_one<TM, TN, i, jn>(fr, acc);
          if constexpr (jn == TN - 1)
            Op::template frag_one<TM, TN, i>(fr, src, src + BM * SA, ra0, rb0i, fs);
          if constexpr (i == TM - 1)
            Op::template frag_one<TM, TN, TM + jn>(fr, src, src + BM * SA, ra0, rb0i, fs);
          if constexpr (kLast && q % kCopyEvery == kCopyEvery - 1)
            issue_copy(std::integral_constant<int, q / kCopyEvery>{}, cur, live);
          __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (kLast) advance();
      });
      ++gs;
    };
    for (int st = 0; st < nst; ++st) stage();
    // The epilogue parameters (raw, compact) are all issued first and waited
    // for together with this wave's copies in flight (one drain per tile).
    // Loaded one group at a time instead, each first use would wait for
    // every copy in flight (memory counters complete in issue order).
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t wm0 = (int64_t)tc.tm * BM + wm * (TM * 32);
    const int64_t wn0 = PAIR ? ((int64_t)tc.tn * BN >> 1) + wn * (TN * 16)
                             : (int64_t)tc.tn * BN + wn * (TN * 32);
    EpiParamsEarly<TM, TN, PAIR, Epi> early;
    early.load(ep, wm0, wn0, sh.M, PAIR ? sh.N >> 1 : sh.N);
    wait_vm<0>();
    early.settle();
    EpiParams<TM, TN, PAIR, Epi> prm;
    early.expand(ep, prm);
    if constexpr (PAIR) {
      epilogue_pair<TM, TN>(acc, wm0, wn0, sh.M, sh.N >> 1, ep, strip, prm);
    } else {
      epilogue_single<TM, TN>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
    }
  }
  wait_vm<0>();    // zero-fill copies past the last tile still target the ring
}

// W8A16 with one wave per SIMD: a 256 x 256 tile of four waves, each a
// TM x TN grid of 32x32 blocks (WM x WN = 1 x 4: 256 x 64 per wave, each
// dequantized weight block feeds 8 MFMAs; 2 x 2: 128 x 128, 4 MFMAs),
// bf16/f16 activations and fp8 weights through a three-stage ring of 64-K
// stages (48 KB each). Against the 8-wave ping-pong tile the waves meet at
// one barrier per stage instead of two, and with 1 x 4 they dequantize
// each weight element once per tile row instead of twice.
//
// A K step (32 K values) is a stream of 2 TM TN MFMA slots, blocks in
// column order: slot k = (j, h, i) multiplies A block i (K half h) with
// weight block j. The fragments and dequantized weights of the next step
// are produced under this step's MFMAs, each right after the slot that
// frees its registers:
//   * raw fp8 chunk q[j] of the next step is read at the first slot of
//     block j's column for j < TN - 1 (its previous contents were
//     dequantized in the previous step) and of block 1 for j = TN - 1;
//   * q[j] (j < TN - 1) is dequantized into the operands b[j][.] during the
//     slots of column j + 1, after the last MFMA that reads b[j][.]; q[TN-1]
//     during column 0 of the step it belongs to (its operands are first
//     read in the last column);
//   * A fragment (h, i) is read after its last reader in the last column;
//   * in a stage's last step, after the stage barrier, the wave's 12
//     copies of stage gs + NBUF go out one every other slot.
// LDS reads use per-lane offsets computed once (the swizzled chunk of a
// lane is the same for every block row), plus the stage base, plus a
// constant block offset in the instruction. Reads of the next step come
// from the current stage buffer (first step) or, after the barrier, from
// the next one (last step); across tiles the ring already holds the next
// tile's first stage. Each accumulator takes its K steps and K halves in
// the order of gemm_pingpong_kernel, so the results are the same bits.
//
// BM_ = 224 (1 x 4 waves of 224 x 64, seven block rows) evens out the rounds
// of GEMMs whose 256-row tiles leave most of a last round idle (9216 rows x
// 3072 columns: 432 tiles of 256 x 256 on 256 CUs are 1.69 rounds, 504
// tiles of 224 x 256 are 1.97); the schedule is the same with 14 slots per
// block column and the four dequant words at slots 2, 5, 8 and 11 of a
// column.
template <bool BF16, bool HAS_SCALE, int WM, int WN, int NBUF, class Epi, int BM_ = 256>
__global__ void __launch_bounds__(256)
gemm_w4a16_kernel(GemmShape sh, Src2 sa, Src2 sb, const float* b_scale, Epi epi) {
  using Op = OpW8A16<BF16, HAS_SCALE>;
  constexpr int BM = BM_, BN = 256, NT = 256;
  static_assert(WM * WN == 4, "four waves");
  static_assert(BM % (32 * WM) == 0 && (BM == 256 || WM == 1), "whole block rows per wave");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TN >= 2 && TM >= 4, "the slot schedule needs two block columns and four rows");
  constexpr int SA = Op::SA, SB = Op::SB, S = Op::S;
  static_assert(S == 2, "two K steps per stage");
  constexpr int STAGE = BM * SA + BN * SB;
  constexpr int RING = NBUF * STAGE;
  constexpr int kStrip = strip_bytes<TN, false>();
  static_assert(NBUF >= 3 && RING + kStrip * WM * WN <= 160 * 1024, "LDS exceeds 160 KB");
  using LA = DirectLoad<BM, SA, NT, false>;
  using LB = DirectLoad<BN, SB, NT, false>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  constexpr int kSlots = 2 * TM * TN, kCol = 2 * TM;      // MFMA slots per step / per column
  static_assert(2 * kPerStage <= kSlots, "one copy every other slot");
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING + kStrip * WM * WN];

  const int ntiles = sh.count;
  const int G = (int)gridDim.x;
  const int my_tiles = (ntiles - 1 - (int)blockIdx.x) / G + 1;
  const Epi ep = epi.prepare();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int wm = wave / WN, wn = wave % WN;
  const float ws = Op::prep_scale(b_scale);

  LA la;
  LB lb;
  la.init(sa.ld_bytes, wave, 0);
  lb.init(sb.ld_bytes, wave, 0);
  constexpr int KS = Op::kStageK;
  const int a_kb = (int)(sh.K * SA / KS), b_kb = (int)(sh.K * SB / KS);
  const int nst = (int)((sh.K + KS - 1) / KS);

  int ij = 0, ips = 0;
  u32x4 ra, rb0;
  auto tile_rsrc = [&](int j) __attribute__((always_inline)) {
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t m0 = (int64_t)tc.tm * BM;
    const int64_t brow0 = (int64_t)tc.tn * BN;
    ra = dma_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
    rb0 = dma_rsrc(sb.p0 + brow0 * sb.ld_bytes, (sb.rows - brow0) * sb.ld_bytes);
  };
  // Copy C of the next stage (A copies first) into `buf`; past this
  // workgroup's last tile the copies read zeros, so every stage issues the
  // same number of copies and the vmcnt arithmetic stays fixed.
  auto issue_copy = [&](auto cc, uint8_t* buf, bool live) __attribute__((always_inline)) {
    constexpr int C = decltype(cc)::value;
    if constexpr (C < LA::kInstr) {
      la.template issue_one<C>(ra, ra, buf, live ? ips * SA : 0, live ? a_kb : 0);
    } else {
      lb.template issue_one<C - LA::kInstr>(rb0, rb0, buf + BM * SA, live ? ips * SB : 0,
                                            live ? b_kb : 0);
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (ij < my_tiles && ++ips == nst) {
      ips = 0;
      if (++ij < my_tiles) tile_rsrc(ij);
    }
  };
  tile_rsrc(0);

  // prologue: stages 0 .. NBUF-1 in flight, stage 0 complete and visible
#pragma unroll
  for (int p = 0; p < NBUF; ++p) {
    const bool live = ij < my_tiles;
    static_for<0, kPerStage>([&](auto cc) { issue_copy(cc, smem + p * STAGE, live); });
    advance();
  }
  wait_vm<(NBUF - 1) * kPerStage>();
  stage_barrier();

  // Per-lane LDS byte offsets within a stage: A fragment of K step t, half
  // H, block row 0 (block row i adds 32 i rows), and the raw weight chunk of
  // K step t, block column 0 (column j adds 32 j rows). The swizzle of a row
  // depends on its low 4 bits only, so the chunk a lane reads is the same
  // for every block.
  const int lane = threadIdx.x & 63, lr = lane & 31, hl = lane >> 5;
  const int ra0 = wm * (TM * 32), rb0i = wn * (TN * 32);
  uint32_t offa[2][2], offb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      offa[t][hh] = (uint32_t)((ra0 + lr) * SA + phys_chunk<SA>(ra0 + lr, 4 * t + 2 * hl + hh) * 16);
    offb[t] = (uint32_t)(BM * SA + (rb0i + lr) * SB + phys_chunk<SB>(rb0i + lr, 2 * t + hl) * 16);
  }
  typedef __attribute__((address_space(3))) const i32x4 lds_i32x4;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)smem;
  i32x4 fa[2][TM];        // A fragments of the current step: [K half][block row]
  i32x4 fq[TN];           // raw fp8 chunks (next step's, once read)
  i32x4 bq[TN][2];        // dequantized weight operands: [block column][K half]
  // step 0 of the first tile: A and all raw chunks; columns 0 .. TN-2
  // dequantized now, the last one in the first step's column 0
  static_for<0, 2>([&](auto hc) {
    constexpr int hh = decltype(hc)::value;
    static_for<0, TM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      fa[hh][i] = reinterpret_cast<lds_i32x4*>(lds0 + offa[0][hh])[i * 32 * SA / 16];
    });
  });
  static_for<0, TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    fq[j] = reinterpret_cast<lds_i32x4*>(lds0 + offb[0])[j * 32 * SB / 16];
  });
  static_for<0, TN - 1>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    static_for<0, 4>([&](auto wc) { Op::template dequant_word<decltype(wc)::value>(fq[j], ws, bq[j]); });
  });
  uint8_t* strip = smem + RING + wave * kStrip;
  int gs = 0;                                   // stage counter over all tiles
  for (int j = 0; j < my_tiles; ++j) {
    typename Op::Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0;
    auto stage = [&]() __attribute__((always_inline)) {
      const int cb = gs % NBUF, nb = (gs + 1) % NBUF;
      uint8_t* cur = smem + cb * STAGE;
      static_for<0, S>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        constexpr bool kLast = s == S - 1;
        if constexpr (kLast) {
          wait_vm<(NBUF - 2) * kPerStage>();   // this wave's copies of stage gs + 1 landed
          stage_barrier_tracked();             // ... and every wave's; stage gs fully read
        }
        constexpr int ft = kLast ? 0 : s + 1;  // K step (within its stage) being prefetched
        const uint32_t sbase = lds0 + (uint32_t)((kLast ? nb : cb) * STAGE);
        const uint32_t pa0 = sbase + offa[ft][0], pa1 = sbase + offa[ft][1], pb = sbase + offb[ft];
        const bool live = ij < my_tiles;
        static_for<0, kSlots>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          constexpr int jb = k / kCol, hh = (k % kCol) / TM, i = k % TM;
          acc[i][jb] = Op::mfma(fa[hh][i], bq[jb][hh], acc[i][jb]);
          // raw chunks of the next step
          if constexpr (k % kCol == 0 && jb < TN - 1)
            fq[jb] = reinterpret_cast<lds_i32x4*>(pb)[jb * 32 * SB / 16];
          if constexpr (k == kCol)
            fq[TN - 1] = reinterpret_cast<lds_i32x4*>(pb)[(TN - 1) * 32 * SB / 16];
          // dequant: the last column of this step during column 0, column
          // jb - 1 of the next step during column jb; one word every kCol / 4
          // slots (rounded down: words 0..3 at slots kW - 1, 2 kW - 1, ...)
          constexpr int kW = kCol / 4;
          static_assert(kW >= 1 && 4 * kW <= kCol, "four dequant words per column");
          if constexpr ((k % kCol) % kW == kW - 1 && (k % kCol) / kW < 4) {
            constexpr int w = (k % kCol) / kW;
            if constexpr (jb == 0) Op::template dequant_word<w>(fq[TN - 1], ws, bq[TN - 1]);
            else Op::template dequant_word<w>(fq[jb - 1], ws, bq[jb - 1]);
          }
          // A fragments of the next step, after their last reader
          if constexpr (jb == TN - 1)
            fa[hh][i] = reinterpret_cast<lds_i32x4*>(hh ? pa1 : pa0)[i * 32 * SA / 16];
          if constexpr (kLast && k < 2 * kPerStage && k % 2 == 1)
            issue_copy(std::integral_constant<int, k / 2>{}, cur, live);
          __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (kLast) advance();
      });
      ++gs;
    };
    for (int st = 0; st < nst; ++st) stage();
    // epilogue parameters: issued, then waited for with this wave's copies
    // in flight (one drain per tile)
    const TileCoord tc = tile_at(sh, (int)blockIdx.x + j * G);
    const int64_t wm0 = (int64_t)tc.tm * BM + wm * (TM * 32);
    const int64_t wn0 = (int64_t)tc.tn * BN + wn * (TN * 32);
    EpiParamsEarly<TM, TN, false, Epi> early;
    early.load(ep, wm0, wn0, sh.M, sh.N);
    wait_vm<0>();
    early.settle();
    EpiParams<TM, TN, false, Epi> prm;
    early.expand(ep, prm);
    epilogue_single<TM, TN>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
  }
  wait_vm<0>();    // zero-fill copies past the last tile still target the ring
}

// Split-K tile kernel for small pieces (the leftover tiles of a large GEMM,
// split): KG groups of WM x WN waves share one BM x BN tile. Stage s holds
// KG consecutive K blocks of kStageK; group g copies and multiplies block
// s * KG + g into its own slice of the stage, so every group runs the
// pipeline of gemm_tile_kernel over a quarter (KG = 4) of K, in lockstep
// with the others at the stage barriers. A wave holds at least a 32 x 64
// sub-tile; a one-wave-per-SIMD piece of that size is bound by the latency
// of its own LDS -> dequant -> MFMA chain, and the groups give every SIMD
// KG / 4 * WM * WN independent chains instead. At the end groups 1..KG-1
// leave their accumulators in the (drained) ring and group 0 adds them in
// group order, then runs the epilogue. Pieces are few (at most a round), so
// each workgroup drains its ring after every piece instead of prefetching
// the next one.
template <class Op, int BM, int BN, int WM, int WN, int KG, int NBUF, bool PAIR, class Epi>
__global__ void __launch_bounds__(64 * WM * WN * KG)
gemm_splitk_kernel(GemmShape sh, Src2 sa, Src2 sb, const float* b_scale, Epi epi) {
  constexpr int GW = WM * WN;                            // waves per group
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && TM * WM * 32 == BM && TN * WN * 32 == BN, "bad wave tiling");
  static_assert(!PAIR || (TN % 2 == 0), "pair tiles need whole gate/up block pairs");
  constexpr int SA = Op::SA, SB = Op::SB, S = Op::S;
  static_assert(S % 2 == 0, "the fragment double buffer assumes an even step count per stage");
  constexpr int SUB = BM * SA + BN * SB;                 // one group's K block
  constexpr int STAGE = KG * SUB;
  constexpr int RING = NBUF * STAGE;
  constexpr int kStrip = strip_bytes<TN, PAIR>();
  using Scalar = std::remove_cv_t<std::remove_reference_t<decltype(typename Op::Acc{}[0])>>;
  constexpr int kPart = (KG - 1) * GW * TM * TN * 16 * 64 * (int)sizeof(Scalar);
  static_assert(KG >= 2 && kPart <= RING, "partial sums must fit the ring");
  static_assert(NBUF >= 2 && RING + kStrip * GW <= 160 * 1024, "LDS exceeds 160 KB");
  using LA = DirectLoad<BM, SA, 64 * GW, false>;
  using LB = DirectLoad<BN, SB, 64 * GW, PAIR>;
  constexpr int kPerStage = LA::kInstr + LB::kInstr;     // copies per wave per stage
  static_assert((NBUF - 1) * kPerStage < 64, "too many copies in flight for vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING + kStrip * GW];

  const Epi ep = epi.prepare();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave / GW, gw = wave % GW;
  const int wm = gw / WN, wn = gw % WN;
  const int lane = threadIdx.x & 63;
  const float ws = Op::prep_scale(b_scale);

  LA la;
  LB lb;
  la.init(sa.ld_bytes, gw, 0);
  lb.init(sb.ld_bytes, gw, 0);
  constexpr int KS = Op::kStageK;
  const int a_kb = (int)(sh.K * SA / KS), b_kb = (int)(sh.K * SB / KS);
  const int nblk = (int)((sh.K + KS - 1) / KS);
  const int nst = (nblk + KG - 1) / KG;                  // stages; blocks past K read zeros
  const int ra0 = wm * (TM * 32), rb0i = wn * (TN * 32);
  using Frag = typename Op::template Frag<TM, TN>;
  Scalar* part = reinterpret_cast<Scalar*>(smem);
  uint8_t* strip = smem + RING + gw * kStrip;

  for (int t = (int)blockIdx.x; t < sh.count; t += (int)gridDim.x) {
    const TileCoord tc = tile_at(sh, t);
    const int64_t m0 = (int64_t)tc.tm * BM;
    const int64_t brow0 = PAIR ? ((int64_t)tc.tn * BN >> 1) : (int64_t)tc.tn * BN;
    const int64_t bleft = (sb.rows - brow0) * sb.ld_bytes;
    const u32x4 ra = dma_rsrc(sa.p0 + m0 * sa.ld_bytes, (sa.rows - m0) * sa.ld_bytes);
    const u32x4 rb0 = dma_rsrc(sb.p0 + brow0 * sb.ld_bytes, bleft);
    const u32x4 rb1 = PAIR ? dma_rsrc(sb.p1 + brow0 * sb.ld_bytes, bleft) : rb0;
    // stage s of this group: K block s * KG + grp (zeros past K, so every
    // stage issues the same copies and the vmcnt arithmetic stays fixed)
    auto issue = [&](int s) __attribute__((always_inline)) {
      uint8_t* buf = smem + (s % NBUF) * STAGE + grp * SUB;
      const int blk = s * KG + grp;
      la.issue(ra, ra, buf, blk * SA, a_kb);
      lb.issue(rb0, rb1, buf + BM * SA, blk * SB, b_kb);
    };
#pragma unroll
    for (int p = 0; p < NBUF; ++p) issue(p);
    wait_vm<(NBUF - 1) * kPerStage>();
    stage_barrier();

    typename Op::Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0;
    Frag fr[2];
    {
      const uint8_t* cur = smem + grp * SUB;
      Op::template frags<TM, TN>(fr[0], cur, cur + BM * SA, ra0, rb0i, 0);
    }
    for (int st = 0; st < nst; ++st) {
      const uint8_t* cur = smem + (st % NBUF) * STAGE + grp * SUB;
      const uint8_t* nxt = smem + ((st + 1) % NBUF) * STAGE + grp * SUB;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if (s == S - 1) {
          wait_vm<(NBUF - 2) * kPerStage>();   // this wave's copies of stage st+1 landed
          stage_barrier();                     // ... and every wave's; stage st fully read
          issue(st + NBUF);                    // refill with stage st+NBUF
          if (st + 1 < nst) Op::template frags<TM, TN>(fr[0], nxt, nxt + BM * SA, ra0, rb0i, 0);
        } else {
          Op::template frags<TM, TN>(fr[(s + 1) & 1], cur, cur + BM * SA, ra0, rb0i, s + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        Op::template mma<TM, TN>(fr[s & 1], acc, ws);
      }
    }
    // every copy (the zero stages past K included) has landed and every
    // fragment read is done: the ring is free for the partial sums
    wait_vm<0>();
    stage_barrier();
    auto slot = [&](int g, int i, int jj, int r) {
      return ((((g - 1) * GW + gw) * TM + i) * TN * 16 + jj * 16 + r) * 64 + lane;
    };
    if (grp > 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[slot(grp, i, jj, r)] = acc[i][jj][r];
    }
    stage_barrier();
    if (grp == 0) {
      for (int g = 1; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < TN; ++jj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jj][r] += part[slot(g, i, jj, r)];
      const int64_t wm0 = m0 + wm * (TM * 32);
      const int64_t wn0 = brow0 + wn * (PAIR ? TN * 16 : TN * 32);
      EpiParams<TM, TN, PAIR, Epi> prm;
      prm.load(ep, wm0, wn0, sh.M, PAIR ? sh.N >> 1 : sh.N);
      if constexpr (PAIR) {
        epilogue_pair<TM, TN>(acc, wm0, wn0, sh.M, sh.N >> 1, ep, strip, prm);
      } else {
        epilogue_single<TM, TN>(acc, wm0, wn0, sh.M, sh.N, ep, strip, prm);
      }
    }
    stage_barrier();                           // partial sums read before the ring refills
  }
}

}  // namespace c4q
