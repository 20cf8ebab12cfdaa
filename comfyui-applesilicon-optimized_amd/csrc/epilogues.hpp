// Epilogue functors: turn accumulators into stored output elements.
//
// Every rounding step is explicit and the library is compiled with
// -ffp-contract=off, so each multiply and add below rounds exactly once, in
// the order written. That order is the reference's; the citation sits on
// each functor.
//
// Interface (used by the tiled kernels' staged store and by the generic
// kernels):
//   OutT                       stored element type (16- or 32-bit bits)
//   prepare()                  per-workgroup copy with scalars loaded
//   Col, col(n, nv)            the parameters of columns n .. n+3 (scales,
//                              bias); only the first nv are valid (the rest
//                              repeat column n and are never stored)
//   rowp(m)                    the parameter of row m (a scale, or 0)
//   apply(r, c, v)             packed outputs of 4 elements of one row from
//                              accumulators v[0..3] and the row / column
//                              parameters; pair epilogues: apply(r, c, g, u)
//                              from gate / up sums
//   kVariants, variant(),      the optional terms present (a bias, a result
//   apply<V>(...)              scale, activation tables) as a bit mask V
//                              fixed per call: apply<V> has no per-element
//                              test of them; apply(...) dispatches on
//                              variant() (the tiled kernels select V once
//                              per tile, see with_variant)
//   value4(m, n, v, nv)        = apply(rowp(m), col(n, nv), v)
//   row(m), vec                byte pointer to output row m; rows are
//                              16-byte aligned (chunked stores allowed)
//   addr(m, n)                 byte address of output (m, n): row(m) + n
//                              elements, or a functor's own layout (columns
//                              n .. n+7 from a multiple of 8 are contiguous)
//   kColFields, col_raw(f, n, N), col_val(f, w), row_raw(m, M)
//                              the same parameters as raw words, one column
//                              or row per call: col_raw / row_raw only load
//                              (buffer loads: reads past N or M return 0),
//                              col_val converts field f of a loaded word;
//                              col(n, nv) field f, element q equals
//                              col_val(f, col_raw(f, n + q, N)) for q < nv
// The tiled kernels load a lane's column parameters once per tile and its
// row parameters once per 32-row block, so the store loop does no loads
// besides activation-table lookups.
//
// Neutral elements keep absent terms branch-free and exact: an absent scale
// multiplies by 1.0f (x * 1 == x for every x), an absent bias adds -0.0f
// (x + -0 == x for every x, -0 included).
#pragma once
#include <type_traits>

#include "numerics.hpp"

namespace c4q {

enum : int { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };
enum : int { SC_NONE = 0, SC_TENSOR = 1, SC_VECTOR = 2 };

typedef __bf16 epi_bf16x2 __attribute__((ext_vector_type(2)));

// Two floats to packed bf16 with one v_cvt_pk_bf16_f32 (round to nearest
// even): bit-identical to bf16_rte for every non-NaN float (all 2^32 inputs
// are compared on the GPU in tests/test_gpu_numerics.py).
__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
  const epi_bf16x2 h = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, h);
}
// Two floats to packed IEEE half, round to nearest even (v_cvt_f16_f32;
// checked the same way against f16_rte). The empty asm makes the two f32
// values exist as written: otherwise the compiler fuses the f32 multiply or
// add that produced them into v_fma_mixlo_f16, which rounds the exact result
// to half once instead of to f32 first (a different half at f32 ties).
__device__ __forceinline__ uint32_t f16x2_rne(float lo, float hi) {
  asm("" : "+v"(lo), "+v"(hi));
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t p) { return bits_f32(p << 16); }
__device__ __forceinline__ float bf16hi(uint32_t p) { return bits_f32(p & 0xFFFF0000u); }

__device__ const float kOneF = 1.0f;     // target of absent-scale pointers

__device__ __forceinline__ float load_f32(const void* p, int dt, int64_t i) {
  if (dt == DT_BF16) return bf16_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == DT_F16) return f16_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}
// f32 value of raw bias bits (f32, or bf16/f16 in the low half).
__device__ __forceinline__ float raw_f32(uint32_t raw, int dt) {
  if (dt == DT_BF16) return bf16_f32((uint16_t)raw);
  if (dt == DT_F16) return f16_f32((uint16_t)raw);
  return __builtin_bit_cast(float, raw);
}

// Raw parameter words through buffer resources over [p, p + n elements):
// loads only (reads past the range return 0), so that a caller can issue
// them long before it converts them.
__device__ __forceinline__ uint32_t raw_load32(const void* p, int64_t n, int64_t i) {
  const int64_t bytes = p ? n * 4 : 0;
  const int32_t range = bytes > 0x7FFFFFF0ll ? 0x7FFFFFF0 : (int32_t)bytes;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, range, 0x00020000);
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)(i * 4), 0, 0);
}
__device__ __forceinline__ uint32_t raw_load16(const void* p, int64_t n, int64_t i) {
  const int64_t bytes = p ? n * 2 : 0;
  const int32_t range = bytes > 0x7FFFFFF0ll ? 0x7FFFFFF0 : (int32_t)bytes;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, range, 0x00020000);
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)(i * 2), 0, 0);
}
// A bias / scale element of dtype dt (DT_F32 or a 16-bit type), raw.
__device__ __forceinline__ uint32_t raw_load_dt(const void* p, int dt, int64_t n, int64_t i) {
  if (dt == DT_F32) return raw_load32(p, n, i);
  return raw_load16(p, n, i);
}

template <class T>
struct EpiOut {
  using OutT = T;
  using Packed = typename std::conditional<sizeof(T) == 2, uint2, uint4>::type;
  void* d; int64_t ldd; int vec;
  __device__ __forceinline__ uint8_t* row(int64_t m) const {
    return static_cast<uint8_t*>(d) + m * ldd * (int64_t)sizeof(T);
  }
  __device__ __forceinline__ uint8_t* addr(int64_t m, int64_t n) const {
    return row(m) + n * (int64_t)sizeof(T);
  }
};

// Column index for parameter loads of element q of a group: past-the-end
// columns read column n instead (their results are discarded).
__device__ __forceinline__ int64_t colq(int64_t n, int q, int nv) { return q < nv ? n + q : n; }

template <class Packed>
__device__ __forceinline__ Packed pack_bf16x4(float a, float b, float c, float d) {
  return Packed{bf16x2_rne(a, b), bf16x2_rne(c, d)};
}

// Raw INT32 store: torch._int_mm / i8_matmul2d_nt
// (reference _patches/int8_ext/int8_gemm.mm:81-94).
struct EpiI32 : EpiOut<uint32_t> {
  struct Col {};
  __device__ __forceinline__ EpiI32 prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t, int) const { return {}; }
  __device__ __forceinline__ float rowp(int64_t) const { return 0.0f; }
  static constexpr int kColFields = 0;
  __device__ __forceinline__ uint32_t col_raw(int, int64_t, int64_t) const { return 0; }
  __device__ __forceinline__ float col_val(int, uint32_t) const { return 0.0f; }
  __device__ __forceinline__ uint32_t row_raw(int64_t, int64_t) const { return 0; }
  static constexpr int kVariants = 1;
  __device__ __forceinline__ int variant() const { return 0; }
  template <int V = 0>
  __device__ __forceinline__ uint4 apply(float, const Col&, const int32_t (&v)[4]) const {
    return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
  }
  __device__ __forceinline__ uint4 value4(int64_t m, int64_t n, const int32_t (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

// Per-tensor fused dequant: D = bf16(f32(C) * row_scale[m]), then optional
// bias as a second bf16 rounding: bf16(f32(D) + f32(bias[n]))
// (reference _patches/int8_ext/int8_gemm.mm:97-122).
struct EpiRowScale : EpiOut<uint16_t> {
  const float* rs; const uint16_t* bias;
  struct Col { float b[4]; };
  __device__ __forceinline__ EpiRowScale prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t n, int nv) const {
    Col c;
#pragma unroll
    for (int q = 0; q < 4; ++q) c.b[q] = bias ? bf16_f32(bias[colq(n, q, nv)]) : 0.0f;
    return c;
  }
  __device__ __forceinline__ float rowp(int64_t m) const { return rs[m]; }
  static constexpr int kColFields = 1;
  __device__ __forceinline__ uint32_t col_raw(int, int64_t n, int64_t N) const { return raw_load16(bias, N, n); }
  __device__ __forceinline__ float col_val(int, uint32_t w) const { return bias ? bf16_f32((uint16_t)w) : 0.0f; }
  __device__ __forceinline__ uint32_t row_raw(int64_t m, int64_t M) const { return raw_load32(rs, M, m); }
  static constexpr int kVariants = 2;                       // bit 0: bias
  __device__ __forceinline__ int variant() const { return bias ? 1 : 0; }
  template <int V>
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const int32_t (&v)[4]) const {
    uint2 p = pack_bf16x4<uint2>((float)v[0] * r, (float)v[1] * r, (float)v[2] * r, (float)v[3] * r);
    if constexpr ((V & 1) != 0)
      p = pack_bf16x4<uint2>(bf16lo(p.x) + c.b[0], bf16hi(p.x) + c.b[1], bf16lo(p.y) + c.b[2],
                             bf16hi(p.y) + c.b[3]);
    return p;
  }
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const int32_t (&v)[4]) const {
    return bias ? apply<1>(r, c, v) : apply<0>(r, c, v);
  }
  __device__ __forceinline__ uint2 value4(int64_t m, int64_t n, const int32_t (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

// Per-channel fused dequant: s = col_scale[n] * row_scale[m] first, then
// D = T(f32(C) * s), optional bias as a second rounding T(f32(D) + f32(bias[n]))
// with T = bf16 (reference _patches/int8_ext/int8_gemm.mm:417-443) or, F16,
// IEEE half with a half bias (the fp16 epilogue nax_frag_store_dequant_cs_half,
// _patches/int8_ext/int8_gemm.mm:1161-1183).
template <bool F16>
struct EpiRowColScaleT : EpiOut<uint16_t> {
  const float* rs; const float* cs; const uint16_t* bias;
  struct Col { float s[4], b[4]; };
  __device__ __forceinline__ static float out_f32(uint16_t h) { return F16 ? f16_f32(h) : bf16_f32(h); }
  __device__ __forceinline__ EpiRowColScaleT prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t n, int nv) const {
    Col c;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c.s[q] = cs[colq(n, q, nv)];
      c.b[q] = bias ? out_f32(bias[colq(n, q, nv)]) : 0.0f;
    }
    return c;
  }
  __device__ __forceinline__ float rowp(int64_t m) const { return rs[m]; }
  static constexpr int kColFields = 2;   // s, b
  __device__ __forceinline__ uint32_t col_raw(int f, int64_t n, int64_t N) const {
    return f == 0 ? raw_load32(cs, N, n) : raw_load16(bias, N, n);
  }
  __device__ __forceinline__ float col_val(int f, uint32_t w) const {
    return f == 0 ? bits_f32(w) : (bias ? out_f32((uint16_t)w) : 0.0f);
  }
  __device__ __forceinline__ uint32_t row_raw(int64_t m, int64_t M) const { return raw_load32(rs, M, m); }
  __device__ __forceinline__ static uint2 pack(float a, float b, float c, float d) {
    if constexpr (F16) return uint2{f16x2_rne(a, b), f16x2_rne(c, d)};
    return pack_bf16x4<uint2>(a, b, c, d);
  }
  static constexpr int kVariants = 2;                       // bit 0: bias
  __device__ __forceinline__ int variant() const { return bias ? 1 : 0; }
  template <int V>
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const int32_t (&v)[4]) const {
    float x[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = (float)v[q] * (c.s[q] * r);
    uint2 p = pack(x[0], x[1], x[2], x[3]);
    if constexpr ((V & 1) != 0)
      p = pack(out_f32((uint16_t)p.x) + c.b[0], out_f32((uint16_t)(p.x >> 16)) + c.b[1],
               out_f32((uint16_t)p.y) + c.b[2], out_f32((uint16_t)(p.y >> 16)) + c.b[3]);
    return p;
  }
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const int32_t (&v)[4]) const {
    return bias ? apply<1>(r, c, v) : apply<0>(r, c, v);
  }
  __device__ __forceinline__ uint2 value4(int64_t m, int64_t n, const int32_t (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

using EpiRowColScale = EpiRowColScaleT<false>;
using EpiRowColScaleF16 = EpiRowColScaleT<true>;

// H3 QKV scatter: the per-channel bf16 epilogue above, with column n of the
// [M, 3 H D] product stored into the attention layout [1, H, M, D] of Q
// (n < H D), K or V (reference nax_frag_store_dequant_cs_qkv,
// _patches/int8_ext/int8_gemm.mm:445-474). D is a multiple of 8, so a
// 16-byte store unit or a 4-column group never crosses a head.
struct EpiRowColScaleQKV : EpiRowColScaleT<false> {
  // K and V as byte offsets from Q (the output pointer d): the destination
  // is then arithmetic in `kind`; a select among three pointers was turned
  // into an indexed table in scratch memory by the compiler
  int64_t koff, voff;
  int64_t rows;              // M
  uint32_t width, hd;        // H * D, D
  __device__ __forceinline__ EpiRowColScaleQKV prepare() const { return *this; }
  __device__ __forceinline__ uint8_t* addr(int64_t m, int64_t n) const {
    const uint32_t nn = (uint32_t)n;
    const uint32_t kind = nn / width, inner = nn - kind * width;
    const uint32_t h = inner / hd, dd = inner - h * hd;
    const int64_t off = koff * (int64_t)(kind == 1) + voff * (int64_t)(kind == 2);
    return static_cast<uint8_t*>(this->d) + off + (((int64_t)h * rows + m) * hd + dd) * 2;
  }
  __device__ __forceinline__ uint2 value4(int64_t m, int64_t n, const int32_t (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

// H3 runtime-LoRA partition (reference int8_matmul_fused_cs_qk_lora_rms_rope
// and _v_lora, _patches/int8_ext/int8_gemm.mm:915-1085, host :2211-2330):
// the QKV scatter of ONE partition (Q, K or V: its H D weight rows, so every
// column has kind 0 and goes to d), with a bf16 low-rank delta [M, H D]
// added to each projection value after the bias:
//   sd = bf16(f32(delta[m, n]) * ls),  ls = f32(bf16(delta_scale))
//   out = bf16(f32(value) + f32(sd))
// The tiled epilogue calls elem() on each 4-column group after apply().
struct EpiQKVLora : EpiRowColScaleQKV {
  static constexpr bool kElem = true;
  const uint16_t* delta;    // [M, width] bf16, rows contiguous, 8-byte aligned
  float ls;
  __device__ __forceinline__ EpiQKVLora prepare() const { return *this; }
  // the delta term of the 4-column group at (m, n), nv of its columns live
  // (width % 4 == 0 and n % 4 == 0: a whole group is one 8-byte load)
  __device__ __forceinline__ uint2 elem(int64_t m, int64_t n, int nv, uint2 p) const {
    const uint16_t* src = delta + m * (int64_t)width + n;
    uint32_t w[2];
    if (nv >= 4) {
      const uint2 u = *reinterpret_cast<const uint2*>(src);
      w[0] = u.x;
      w[1] = u.y;
    } else {
      uint16_t h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = src[q < nv ? q : 0];
      w[0] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
      w[1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
    }
    const uint32_t sd0 = bf16x2_rne(bf16lo(w[0]) * ls, bf16hi(w[0]) * ls);
    const uint32_t sd1 = bf16x2_rne(bf16lo(w[1]) * ls, bf16hi(w[1]) * ls);
    return uint2{bf16x2_rne(bf16lo(p.x) + bf16lo(sd0), bf16hi(p.x) + bf16hi(sd0)),
                 bf16x2_rne(bf16lo(p.y) + bf16lo(sd1), bf16hi(p.y) + bf16hi(sd1))};
  }
  __device__ __forceinline__ uint2 value4(int64_t m, int64_t n, const int32_t (&v)[4], int nv) const {
    return elem(m, n, nv, apply(rowp(m), col(n, nv), v));
  }
};

// bf16 rounding (nearest even) of an f32 value, as f32.
__device__ __forceinline__ float round_bf16(float v) { return bf16lo(bf16x2_rne(v, v)); }

// RMSNorm of one 128-element head row held by the 8 lanes 8p .. 8p+7 of a
// wave: lane j holds x[k] = column 64 h + 8 j + k' (k = 8 h + k'). The squares
// (exact in f32: x is a bf16 value) are summed per lane in k order, then over
// the 8 lanes by xor partners 4, 2, 1 -- ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7))
// on every lane; inv = 1 / sqrt(ss / 128 + eps) with correctly rounded sqrt
// and division; y = bf16((x * inv) * w). Reference
// _patches/int8_ext/int8_gemm.mm:806-833 (its sum order is Metal's simd_sum).
// Sum of v over the 8 lanes 8p .. 8p+7 by xor partners 4, 2, 1, read
// through DPP (row shifts by 4, quad permutes): every lane gets
// ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)). Needs all 64 lanes active.
__device__ __forceinline__ float sum8_lanes(float v) {
  const int iv = __builtin_bit_cast(int, v);
  const int from_up = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xF, 0xF, true);   // row_shl:4
  const int from_dn = __builtin_amdgcn_update_dpp(0, iv, 0x114, 0xF, 0xF, true);   // row_shr:4
  v = v + __builtin_bit_cast(float, (threadIdx.x & 4) ? from_dn : from_up);
  v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E,
                                                                0xF, 0xF, true));  // lane ^ 2
  v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1,
                                                                0xF, 0xF, true));  // lane ^ 1
  return v;
}

__device__ __forceinline__ void head_rms_norm(const float (&x)[16], const float (&w)[16], float eps,
                                              float (&y)[16]) {
  float ss = 0.0f;
  // x * x is exact in f32 (x is a bf16 value), so the fused multiply-add
  // rounds exactly like ss + x * x
#pragma unroll
  for (int k = 0; k < 16; ++k) ss = __builtin_fmaf(x[k], x[k], ss);
  ss = sum8_lanes(ss);
  const float inv = 1.0f / __builtin_sqrtf(ss * 0.0078125f + eps);
#pragma unroll
  for (int k = 0; k < 16; k += 2) {
    const uint32_t p = bf16x2_rne((x[k] * inv) * w[k], (x[k + 1] * inv) * w[k + 1]);
    y[k] = bf16lo(p);
    y[k + 1] = bf16hi(p);
  }
}

// Split-half RoPE of column d < 2R (reference int8_gemm.mm:843-854, the
// eager `out = y * diag; out.addcmul_(y_partner, off)`): fw holds the bf16
// pair freqs[m, d mod R, r, 0..1], r = (d >= R); the diagonal product is
// rounded to bf16, the off-diagonal one (exact in f32) added with one
// rounding.
__device__ __forceinline__ float rope_split_half(float yd, float yp, uint32_t fw, bool second) {
  const float f0 = bf16lo(fw), f1 = bf16hi(fw);
  const float diag = second ? f1 : f0, off = second ? f0 : f1;
  return round_bf16(round_bf16(diag * yd) + off * yp);
}

// H3 QKV projection with Q/K RMSNorm and partial split-half RoPE
// (reference int8_matmul_fused_cs_qkv_rms_rope_impl,
// _patches/int8_ext/int8_gemm.mm:683-861; host :2111-2209): the QKV
// scatter above with D = 128. The tiled kernels run it with waves whose
// sub-tile spans exactly one head (128 columns) and R a multiple of 8, see
// epilogue_head_norm.
struct EpiQKVNormRope : EpiRowColScaleQKV {
  static constexpr bool kHeadNorm = true;
  const uint32_t* freqs;    // [M, R, 2, 2] bf16, as [M, R, 2] pairs; 4-byte aligned
  const float* qw;          // [128] f32 Q norm weight
  int64_t kwoff;            // the K norm weight as a byte offset from qw
  int32_t pairs;            // R, 2R <= 128
  float eps;
  __device__ __forceinline__ EpiQKVNormRope prepare() const { return *this; }
  // norm weight of Q (kind 0) or K (kind 1): offset arithmetic, not a
  // pointer select (see koff above)
  __device__ __forceinline__ const float* weight(uint32_t kind) const {
    return reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(qw) +
                                          kwoff * (int64_t)(kind == 1));
  }
};

// torch._scaled_mm on the fp8 route: out = f32 acc, then * scale_a,
// * scale_b, * scale_result, + f32(bias), each in f32 and in this order,
// one final rounding to the output dtype
// (reference _patches/scaled_mm_fp8.py:123-146). OUT is the output type
// (DT_BF16, DT_F16 or DT_F32), fixed at compile time so that the store loop
// converts one way. Scale pointers are read with a stride (0: per tensor, 1:
// per row / column); an absent scale reads 1.0f, an absent scale_result is
// skipped (x * 1.0f == x).
template <int OUT>
struct EpiScaled : EpiOut<typename std::conditional<OUT == DT_F32, uint32_t, uint16_t>::type> {
  using Base = EpiOut<typename std::conditional<OUT == DT_F32, uint32_t, uint16_t>::type>;
  using Packed = typename Base::Packed;
  const float* sa; int sa_mode; const float* sb; int sb_mode; const float* sr;
  const void* bias; int bias_dt;
  int sa_step, sb_step;
  float sr0;
  __device__ __forceinline__ EpiScaled prepare() const {
    EpiScaled e = *this;
    if (sa_mode == SC_NONE) e.sa = &kOneF;
    if (sb_mode == SC_NONE) e.sb = &kOneF;
    e.sa_step = sa_mode == SC_VECTOR ? 1 : 0;
    e.sb_step = sb_mode == SC_VECTOR ? 1 : 0;
    e.sr0 = sr ? sr[0] : 1.0f;
    return e;
  }
  struct Col { float s[4], b[4]; };
  __device__ __forceinline__ Col col(int64_t n, int nv) const {
    Col c;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c.s[q] = sb[colq(n, q, nv) * sb_step];
      c.b[q] = bias ? load_f32(bias, bias_dt, colq(n, q, nv)) : 0.0f;
    }
    return c;
  }
  __device__ __forceinline__ float rowp(int64_t m) const { return sa[m * sa_step]; }
  static constexpr int kColFields = 2;   // s, b
  __device__ __forceinline__ uint32_t col_raw(int f, int64_t n, int64_t N) const {
    if (f == 0) return raw_load32(sb, sb_step ? N : 1, n * sb_step);
    return raw_load_dt(bias, bias_dt, N, n);
  }
  __device__ __forceinline__ float col_val(int f, uint32_t w) const {
    if (f == 0) return bits_f32(w);
    return bias ? raw_f32(w, bias_dt) : 0.0f;
  }
  __device__ __forceinline__ uint32_t row_raw(int64_t m, int64_t M) const {
    return raw_load32(sa, sa_step ? M : 1, m * sa_step);
  }
  static constexpr int kVariants = 4;                       // bit 0: bias, bit 1: scale_result
  __device__ __forceinline__ int variant() const { return (bias ? 1 : 0) | (sr ? 2 : 0); }
  template <int V>
  __device__ __forceinline__ Packed apply(float a, const Col& c, const float (&v)[4]) const {
    float o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = (v[q] * a) * c.s[q];
    if constexpr ((V & 2) != 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = o[q] * sr0;
    }
    if constexpr ((V & 1) != 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = o[q] + c.b[q];
    }
    if constexpr (OUT == DT_F32) {
      return Packed{f32_bits(o[0]), f32_bits(o[1]), f32_bits(o[2]), f32_bits(o[3])};
    } else if constexpr (OUT == DT_F16) {
      return Packed{f16x2_rne(o[0], o[1]), f16x2_rne(o[2], o[3])};
    } else {
      return pack_bf16x4<Packed>(o[0], o[1], o[2], o[3]);
    }
  }
  __device__ __forceinline__ Packed apply(float a, const Col& c, const float (&v)[4]) const {
    switch (variant()) {
      case 1: return apply<1>(a, c, v);
      case 2: return apply<2>(a, c, v);
      case 3: return apply<3>(a, c, v);
      default: return apply<0>(a, c, v);
    }
  }
  __device__ __forceinline__ Packed value4(int64_t m, int64_t n, const float (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

// W8A16: D = T(acc + f32(bias[n])) with one rounding (reference
// _patches/fp8s_ext/w8a16_gemm.mm:101-119 and the f32-out + bias route of
// _patches/linear_fp8_w8a16.py:190-196). `act` (bf16 output only) is a
// 65,536-entry table applied to the rounded bf16 value: the unfused
// "bf16 linear, then bf16 activation" order of the FLUX MLP. OUT is the
// output type (DT_BF16, DT_F16 or DT_F32), fixed at compile time.
template <int OUT>
struct EpiW8A16 : EpiOut<typename std::conditional<OUT == DT_F32, uint32_t, uint16_t>::type> {
  using Base = EpiOut<typename std::conditional<OUT == DT_F32, uint32_t, uint16_t>::type>;
  using Packed = typename Base::Packed;
  const void* bias; int bias_dt; const uint16_t* act;
  struct Col { float b[4]; };
  __device__ __forceinline__ EpiW8A16 prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t n, int nv) const {
    Col c;
#pragma unroll
    for (int q = 0; q < 4; ++q) c.b[q] = bias ? load_f32(bias, bias_dt, colq(n, q, nv)) : 0.0f;
    return c;
  }
  __device__ __forceinline__ float rowp(int64_t) const { return 0.0f; }
  static constexpr int kColFields = 1;
  __device__ __forceinline__ uint32_t col_raw(int, int64_t n, int64_t N) const {
    return raw_load_dt(bias, bias_dt, N, n);
  }
  __device__ __forceinline__ float col_val(int, uint32_t w) const { return bias ? raw_f32(w, bias_dt) : 0.0f; }
  __device__ __forceinline__ uint32_t row_raw(int64_t, int64_t) const { return 0; }
  static constexpr int kVariants = OUT == DT_BF16 ? 4 : 2;   // bit 0: bias, bit 1: act
  __device__ __forceinline__ int variant() const {
    return (bias ? 1 : 0) | (OUT == DT_BF16 && act ? 2 : 0);
  }
  template <int V>
  __device__ __forceinline__ Packed apply(float, const Col& c, const float (&v)[4]) const {
    float o[4] = {v[0], v[1], v[2], v[3]};
    if constexpr ((V & 1) != 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = o[q] + c.b[q];
    }
    if constexpr (OUT == DT_F32) {
      return Packed{f32_bits(o[0]), f32_bits(o[1]), f32_bits(o[2]), f32_bits(o[3])};
    } else if constexpr (OUT == DT_F16) {
      return Packed{f16x2_rne(o[0], o[1]), f16x2_rne(o[2], o[3])};
    } else {
      Packed p = pack_bf16x4<Packed>(o[0], o[1], o[2], o[3]);
      if constexpr ((V & 2) != 0) {
        p.x = (uint32_t)act[p.x & 0xFFFFu] | ((uint32_t)act[p.x >> 16] << 16);
        p.y = (uint32_t)act[p.y & 0xFFFFu] | ((uint32_t)act[p.y >> 16] << 16);
      }
      return p;
    }
  }
  __device__ __forceinline__ Packed apply(float r, const Col& c, const float (&v)[4]) const {
    switch (variant()) {
      case 1: return apply<1>(r, c, v);
      case 2: return apply<2 % kVariants>(r, c, v);
      case 3: return apply<3 % kVariants>(r, c, v);
      default: return apply<0>(r, c, v);
    }
  }
  __device__ __forceinline__ Packed value4(int64_t m, int64_t n, const float (&v)[4], int nv) const {
    return apply(rowp(m), col(n, nv), v);
  }
};

// Fused gate/up FFN pair. Both projections use the per-channel epilogue
// (bf16 stores), then optional 65,536-entry bf16 tables, then a bf16
// product:
//   x1 = bf16(f32(C1) * (s1[col] * rs[m]));  x2 = bf16(f32(C2) * (s2[col] * rs[m]))
//   out = bf16(f32(T1[x1]) * f32(T2[x2]))     (missing table = identity)
// Krea2: T1 = SiLU, T2 = none (reference _patches/krea2_ffn_pair.metal:281-304);
// MOSS:  T1 = T_h, T2 = T_g     (reference _patches/moss_ffn_mps.metal:278-301).
struct EpiPair : EpiOut<uint16_t> {
  const float* rs; const float* s1; const float* s2;
  const uint16_t* t1; const uint16_t* t2;
  struct Col { float s1[4], s2[4]; };
  __device__ __forceinline__ EpiPair prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t n, int nv) const {
    Col c;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c.s1[q] = s1[colq(n, q, nv)];
      c.s2[q] = s2[colq(n, q, nv)];
    }
    return c;
  }
  __device__ __forceinline__ float rowp(int64_t m) const { return rs[m]; }
  static constexpr int kColFields = 2;   // s1, s2
  __device__ __forceinline__ uint32_t col_raw(int f, int64_t n, int64_t N) const {
    return raw_load32(f == 0 ? s1 : s2, N, n);
  }
  __device__ __forceinline__ float col_val(int, uint32_t w) const { return bits_f32(w); }
  __device__ __forceinline__ uint32_t row_raw(int64_t m, int64_t M) const { return raw_load32(rs, M, m); }
  static constexpr int kVariants = 4;                       // bit 0: t1, bit 1: t2
  __device__ __forceinline__ int variant() const { return (t1 ? 1 : 0) | (t2 ? 2 : 0); }
  template <int V>
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const int32_t (&g)[4],
                                         const int32_t (&u)[4]) const {
    float a[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = (float)g[q] * (c.s1[q] * r);
      b[q] = (float)u[q] * (c.s2[q] * r);
    }
    uint2 x1 = pack_bf16x4<uint2>(a[0], a[1], a[2], a[3]);
    uint2 x2 = pack_bf16x4<uint2>(b[0], b[1], b[2], b[3]);
    if constexpr ((V & 1) != 0) {
      x1.x = (uint32_t)t1[x1.x & 0xFFFFu] | ((uint32_t)t1[x1.x >> 16] << 16);
      x1.y = (uint32_t)t1[x1.y & 0xFFFFu] | ((uint32_t)t1[x1.y >> 16] << 16);
    }
    if constexpr ((V & 2) != 0) {
      x2.x = (uint32_t)t2[x2.x & 0xFFFFu] | ((uint32_t)t2[x2.x >> 16] << 16);
      x2.y = (uint32_t)t2[x2.y & 0xFFFFu] | ((uint32_t)t2[x2.y >> 16] << 16);
    }
    return pack_bf16x4<uint2>(bf16lo(x1.x) * bf16lo(x2.x), bf16hi(x1.x) * bf16hi(x2.x),
                              bf16lo(x1.y) * bf16lo(x2.y), bf16hi(x1.y) * bf16hi(x2.y));
  }
  template <class T>
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const T (&g)[4], const T (&u)[4]) const {
    switch (variant()) {
      case 1: return apply<1>(r, c, g, u);
      case 2: return apply<2>(r, c, g, u);
      case 3: return apply<3>(r, c, g, u);
      default: return apply<0>(r, c, g, u);
    }
  }
  __device__ __forceinline__ uint2 pair4(int64_t m, int64_t n, const int32_t (&g)[4],
                                         const int32_t (&u)[4], int nv) const {
    return apply(rowp(m), col(n, nv), g, u);
  }
};

// MOSS bf16 FC1/SiTU pair on fp32 accumulators of a bf16 x bf16 GEMM, no
// scales: x1 = bf16(acc_h), x2 = bf16(acc_g), out = bf16(f32(T1[x1]) *
// f32(T2[x2])) (missing table = identity)
// (reference _patches/moss_bf16_ffn_pair.metal:282-304).
struct EpiPairF : EpiOut<uint16_t> {
  const uint16_t* t1; const uint16_t* t2;
  struct Col {};
  __device__ __forceinline__ EpiPairF prepare() const { return *this; }
  __device__ __forceinline__ Col col(int64_t, int) const { return {}; }
  __device__ __forceinline__ float rowp(int64_t) const { return 0.0f; }
  static constexpr int kColFields = 0;
  __device__ __forceinline__ uint32_t col_raw(int, int64_t, int64_t) const { return 0; }
  __device__ __forceinline__ float col_val(int, uint32_t) const { return 0.0f; }
  __device__ __forceinline__ uint32_t row_raw(int64_t, int64_t) const { return 0; }
  static constexpr int kVariants = 4;                       // bit 0: t1, bit 1: t2
  __device__ __forceinline__ int variant() const { return (t1 ? 1 : 0) | (t2 ? 2 : 0); }
  template <int V>
  __device__ __forceinline__ uint2 apply(float, const Col&, const float (&g)[4],
                                         const float (&u)[4]) const {
    uint2 x1 = pack_bf16x4<uint2>(g[0], g[1], g[2], g[3]);
    uint2 x2 = pack_bf16x4<uint2>(u[0], u[1], u[2], u[3]);
    if constexpr ((V & 1) != 0) {
      x1.x = (uint32_t)t1[x1.x & 0xFFFFu] | ((uint32_t)t1[x1.x >> 16] << 16);
      x1.y = (uint32_t)t1[x1.y & 0xFFFFu] | ((uint32_t)t1[x1.y >> 16] << 16);
    }
    if constexpr ((V & 2) != 0) {
      x2.x = (uint32_t)t2[x2.x & 0xFFFFu] | ((uint32_t)t2[x2.x >> 16] << 16);
      x2.y = (uint32_t)t2[x2.y & 0xFFFFu] | ((uint32_t)t2[x2.y >> 16] << 16);
    }
    return pack_bf16x4<uint2>(bf16lo(x1.x) * bf16lo(x2.x), bf16hi(x1.x) * bf16hi(x2.x),
                              bf16lo(x1.y) * bf16lo(x2.y), bf16hi(x1.y) * bf16hi(x2.y));
  }
  template <class T>
  __device__ __forceinline__ uint2 apply(float r, const Col& c, const T (&g)[4], const T (&u)[4]) const {
    switch (variant()) {
      case 1: return apply<1>(r, c, g, u);
      case 2: return apply<2>(r, c, g, u);
      case 3: return apply<3>(r, c, g, u);
      default: return apply<0>(r, c, g, u);
    }
  }
  __device__ __forceinline__ uint2 pair4(int64_t m, int64_t n, const float (&g)[4],
                                         const float (&u)[4], int nv) const {
    return apply(rowp(m), col(n, nv), g, u);
  }
};

// Store a packed group of 4 outputs at (m, n .. n+nv-1).
template <class Epi, class Packed>
__device__ __forceinline__ void store_group(const Epi& epi, int64_t m, int64_t n, int nv, Packed p) {
  using OutT = typename Epi::OutT;
  uint8_t* dst = epi.addr(m, n);
  if (epi.vec && nv == 4) {
    *reinterpret_cast<Packed*>(dst) = p;
    return;
  }
  OutT e[4];
  __builtin_memcpy(e, &p, sizeof(e));
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (q < nv) reinterpret_cast<OutT*>(dst)[q] = e[q];
}

}  // namespace c4q
