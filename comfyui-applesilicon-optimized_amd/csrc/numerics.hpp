// Bit-exact scalar conversions shared by every kernel of the library.
//
// All rounding is spelled out with integer operations so that the result
// does not depend on compiler flags or on the hardware conversion modes:
//   * float -> bf16 / f16 : round to nearest, ties to even (torch's casts);
//   * fp8 e4m3fn -> float : exact decode;
//   * float -> fp8 e4m3fn : round to nearest even, |x| >= 480 and NaN -> NaN
//                           (torch's cast; callers clamp to +-448 first).
// The one hardware conversion here, e4m3_pair, is checked against f32_e4m3
// for every float bit pattern.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace c4q {

#define C4Q_HD __host__ __device__ __forceinline__

C4Q_HD uint32_t f32_bits(float f) {
  union { float f; uint32_t u; } v; v.f = f; return v.u;
}
C4Q_HD float bits_f32(uint32_t u) {
  union { float f; uint32_t u; } v; v.u = u; return v.f;
}

// float -> bf16 bits, RNE. NaN -> 0x7FC0 (quiet, sign dropped).
C4Q_HD uint16_t bf16_rte(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
C4Q_HD float bf16_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// float -> IEEE binary16 bits, RNE, overflow -> inf, NaN -> 0x7E00.
C4Q_HD uint16_t f16_rte(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   // >= 65520 rounds to inf
  if (a < 0x38800000u) {                                      // below 2^-14: subnormal grid 2^-24
    // value * 2^24 rounded to an integer, ties to even; exact in float
    // arithmetic because a * 2^24 < 2^10 carries <= 24 significant bits.
    float v = bits_f32(a) * 16777216.0f;
    uint32_t q = (uint32_t)v;
    float frac = v - (float)q;
    if (frac > 0.5f || (frac == 0.5f && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
  }
  // normal: rebias exponent 127 -> 15 and round 23 -> 10 mantissa bits
  uint32_t r = a - 0x38000000u;                  // (127-15) << 23
  r += 0xFFFu + ((r >> 13) & 1u);
  return (uint16_t)(sign | (r >> 13));
}
C4Q_HD float f16_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f;   // m * 2^-24, exact
    return bits_f32(f32_bits(v) | sign);
  }
  if (e == 31) return bits_f32(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// bf16(RN(x / s)) without a division per element, for bf16 values x and a
// positive normal bf16 s, given r = RN(1 / s). Both significands have 8
// bits, so x/s either lies exactly on a bf16 rounding midpoint or at least
// 2^-9 / 255 (relative) away from every midpoint; q0 = RN(x r) is within
// about 2^-23 of x/s, and the residual step q1 = RN(q0 - RN(q0 s - x) r)
// (both fused, the residual exact) lands exactly on such a midpoint. So
// bf16 rounding of q1 equals bf16 rounding of the correctly rounded
// quotient; checked for every pair of bf16 x and s with |x/s| < 2^64 on the
// GPU (tests/test_gpu_numerics.py). The residual is formed as q0 s - x and
// subtracted so that x = -0 gives -0 (x - q0 s would give +0).
C4Q_HD float div_bf16_operands(float x, float s, float r) {
  const float q0 = x * r;
  const float e = __builtin_fmaf(q0, s, -x);
  return __builtin_fmaf(-e, r, q0);
}

// fp8 e4m3fn code -> float (exact). 0x7F / 0xFF are NaN; no infinities.
C4Q_HD float e4m3_f32(uint32_t c) {
  uint32_t sign = (c & 0x80u) << 24;
  uint32_t em = c & 0x7Fu;
  if (em == 0x7Fu) return bits_f32(0x7FC00000u | sign);
  if (em < 8u) {                       // subnormal: m * 2^-9
    float v = (float)em * 0.001953125f;
    return bits_f32(f32_bits(v) | sign);
  }
  return bits_f32(sign | ((em + (120u << 3)) << 20));
}

// float -> fp8 e4m3fn code, RNE on the e4m3 grid, no saturation.
C4Q_HD uint8_t f32_e4m3(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x43F00000u) return (uint8_t)(sign | 0x7Fu);        // >= 480 or NaN
  if (a < 0x3C800000u) {                                        // < 2^-6: grid 2^-9
    float v = bits_f32(a) * 512.0f;                             // exact (power-of-two scale)
    uint32_t q = (uint32_t)v;
    float frac = v - (float)q;
    if (frac > 0.5f || (frac == 0.5f && (q & 1u))) q += 1u;     // q <= 8; 8 == code of 2^-6
    return (uint8_t)(sign | q);
  }
  // normal: rebias 127 -> 7, keep 3 mantissa bits with RNE (may carry into the exponent)
  uint32_t r = a - (120u << 23);
  r += 0x7FFFFu + ((r >> 20) & 1u);
  return (uint8_t)(sign | (r >> 20));
}

// Clamp to [-448, 448] the way torch's clamp does (NaN passes through).
C4Q_HD float clamp448(float v) { return v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v); }

// e4m3fn codes of clamp448(a) (bits 0-7) and clamp448(b) (bits 8-15):
// f32_e4m3(clamp448(.)) of each, by the gfx950 conversion v_cvt_pk_fp8_f32
// (OCP e4m3, round to nearest even; its inputs are within +-448 here). A NaN
// takes the integer path (sign | 0x7F). Equal to f32_e4m3(clamp448(.)) for
// every float bit pattern in either slot, checked on the GPU
// (tests/test_gpu_numerics.py).
__device__ __forceinline__ uint32_t e4m3_pair(float a, float b) {
  if (__builtin_expect(a != a || b != b, 0))
    return (uint32_t)f32_e4m3(clamp448(a)) | ((uint32_t)f32_e4m3(clamp448(b)) << 8);
  const float ca = fminf(fmaxf(a, -448.0f), 448.0f), cb = fminf(fmaxf(b, -448.0f), 448.0f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xFFFFu;
}

// The per-tensor fp8 activation quantizer divides by s = RN(amax / 448) with
// r = RN(1 / s) and div_bf16_operands: one multiply and two fused steps per
// element instead of an IEEE division. Used for 2^-80 <= s <= 2^126 (amax
// from about 3.7e-22 up, finite): then every quotient of magnitude 2^-10 or
// more (the smallest that does not encode as zero) has |x| >= 2^-90, so the
// residual is a normal float and exact, as the residual step needs; smaller
// quotients encode as a signed zero either way. With smaller s a subnormal x
// can leave an inexact residual (206 of the bf16 pairs below 2^-80 differ).
// The e4m3 code of the result equals the code of the correctly rounded
// quotient for every bf16 (f16) x and every s this quantizer forms from a
// bf16 (f16) amax >= |x| in that range, checked on the GPU.
C4Q_HD bool rcp_quot_ok(float s) { return s >= 8.27180613e-25f && s <= 8.50705917e37f; }

}  // namespace c4q
