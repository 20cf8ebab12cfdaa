// Epilogue functors: turn one accumulator into one output element.
//
// Every rounding step is explicit (bf16_rte / f16_rte from numerics.hpp) and
// the library is compiled with -ffp-contract=off, so each multiply and add
// below rounds exactly once, in the order written. That order is the
// reference's; the citation sits on each functor.
//
// Interface (used by the tiled kernels' staged store and by the generic
// kernels):
//   OutT                      stored element type (16- or 32-bit bits)
//   prepare()                 per-workgroup copy with scalars loaded
//   value(m, n, acc)          the output bits of element (m, n)
//   pair(m, col, a1, a2)      (pair epilogues) the output of column col
//   row(m)                    byte pointer to output row m
//   vec                       rows are 16-byte aligned: chunked stores allowed
#pragma once
#include <type_traits>

#include "numerics.hpp"

namespace c4q {

enum : int { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };
enum : int { SC_NONE = 0, SC_TENSOR = 1, SC_VECTOR = 2 };

__device__ __forceinline__ float load_f32(const void* p, int dt, int64_t i) {
  if (dt == DT_BF16) return bf16_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == DT_F16) return f16_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

template <class T>
struct EpiOut {
  using OutT = T;
  void* d; int64_t ldd; int vec;
  __device__ __forceinline__ uint8_t* row(int64_t m) const {
    return static_cast<uint8_t*>(d) + m * ldd * (int64_t)sizeof(T);
  }
  __device__ __forceinline__ void put(int64_t m, int64_t n, T v) const {
    reinterpret_cast<T*>(row(m))[n] = v;
  }
};

// Raw INT32 store: torch._int_mm / i8_matmul2d_nt
// (reference _patches/int8_ext/int8_gemm.mm:81-94).
struct EpiI32 : EpiOut<uint32_t> {
  __device__ __forceinline__ EpiI32 prepare() const { return *this; }
  __device__ __forceinline__ uint32_t value(int64_t, int64_t, int32_t v) const { return (uint32_t)v; }
};

// Per-tensor fused dequant: D = bf16(f32(C) * row_scale[m]), then optional
// bias as a second bf16 rounding: bf16(f32(D) + f32(bias[n]))
// (reference _patches/int8_ext/int8_gemm.mm:97-122).
struct EpiRowScale : EpiOut<uint16_t> {
  const float* rs; const uint16_t* bias;
  __device__ __forceinline__ EpiRowScale prepare() const { return *this; }
  __device__ __forceinline__ uint16_t value(int64_t m, int64_t n, int32_t v) const {
    uint16_t h = bf16_rte((float)v * rs[m]);
    if (bias) h = bf16_rte(bf16_f32(h) + bf16_f32(bias[n]));
    return h;
  }
};

// Per-channel fused dequant: s = col_scale[n] * row_scale[m] first, then
// D = bf16(f32(C) * s), optional bias as above
// (reference _patches/int8_ext/int8_gemm.mm:417-443).
struct EpiRowColScale : EpiOut<uint16_t> {
  const float* rs; const float* cs; const uint16_t* bias;
  __device__ __forceinline__ EpiRowColScale prepare() const { return *this; }
  __device__ __forceinline__ uint16_t value(int64_t m, int64_t n, int32_t v) const {
    const float s = cs[n] * rs[m];
    uint16_t h = bf16_rte((float)v * s);
    if (bias) h = bf16_rte(bf16_f32(h) + bf16_f32(bias[n]));
    return h;
  }
};

// torch._scaled_mm on the fp8 route: out = f32 acc, then * scale_a,
// * scale_b, * scale_result, + f32(bias), each in f32 and in this order,
// one final rounding to the output dtype
// (reference _patches/scaled_mm_fp8.py:123-146). F32OUT selects a 32-bit
// output; otherwise out_dt picks bf16 or f16.
template <bool F32OUT>
struct EpiScaled : EpiOut<typename std::conditional<F32OUT, uint32_t, uint16_t>::type> {
  using Base = EpiOut<typename std::conditional<F32OUT, uint32_t, uint16_t>::type>;
  using OutT = typename Base::OutT;
  int out_dt;
  const float* sa; int sa_mode; const float* sb; int sb_mode; const float* sr;
  const void* bias; int bias_dt;
  float sa0, sb0, sr0;
  __device__ __forceinline__ EpiScaled prepare() const {
    EpiScaled e = *this;
    e.sa0 = sa_mode == SC_TENSOR ? sa[0] : 1.0f;
    e.sb0 = sb_mode == SC_TENSOR ? sb[0] : 1.0f;
    e.sr0 = sr ? sr[0] : 1.0f;
    return e;
  }
  __device__ __forceinline__ OutT value(int64_t m, int64_t n, float v) const {
    float o = v;
    if (sa_mode == SC_TENSOR) o = o * sa0; else if (sa_mode == SC_VECTOR) o = o * sa[m];
    if (sb_mode == SC_TENSOR) o = o * sb0; else if (sb_mode == SC_VECTOR) o = o * sb[n];
    if (sr) o = o * sr0;
    if (bias) o = o + load_f32(bias, bias_dt, n);
    if constexpr (F32OUT) return f32_bits(o);
    else return out_dt == DT_F16 ? f16_rte(o) : bf16_rte(o);
  }
};

// W8A16: D = T(acc + f32(bias[n])) with one rounding (reference
// _patches/fp8s_ext/w8a16_gemm.mm:101-119 and the f32-out + bias route of
// _patches/linear_fp8_w8a16.py:190-196). `act` (bf16 output only) is a
// 65,536-entry table applied to the rounded bf16 value: the unfused
// "bf16 linear, then bf16 activation" order of the FLUX MLP.
template <bool F32OUT>
struct EpiW8A16 : EpiOut<typename std::conditional<F32OUT, uint32_t, uint16_t>::type> {
  using Base = EpiOut<typename std::conditional<F32OUT, uint32_t, uint16_t>::type>;
  using OutT = typename Base::OutT;
  int out_dt; const void* bias; int bias_dt; const uint16_t* act;
  __device__ __forceinline__ EpiW8A16 prepare() const { return *this; }
  __device__ __forceinline__ OutT value(int64_t, int64_t n, float v) const {
    float o = v;
    if (bias) o = o + load_f32(bias, bias_dt, n);
    if constexpr (F32OUT) {
      return f32_bits(o);
    } else {
      if (out_dt == DT_F16) return f16_rte(o);
      uint16_t h = bf16_rte(o);
      if (act) h = act[h];
      return h;
    }
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
  __device__ __forceinline__ EpiPair prepare() const { return *this; }
  __device__ __forceinline__ uint16_t pair(int64_t m, int64_t col, int32_t c1, int32_t c2) const {
    const float r = rs[m];
    uint16_t x1 = bf16_rte((float)c1 * (s1[col] * r));
    uint16_t x2 = bf16_rte((float)c2 * (s2[col] * r));
    if (t1) x1 = t1[x1];
    if (t2) x2 = t2[x2];
    return bf16_rte(bf16_f32(x1) * bf16_f32(x2));
  }
};

}  // namespace c4q
