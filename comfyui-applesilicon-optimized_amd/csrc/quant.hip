// Activation quantizers (rowwise int8, per-tensor fp8) and the fp8 weight
// dequantizer. Bandwidth-bound elementwise/reduction kernels.
#include "api_common.hpp"
#include "epilogues.hpp"
#include "gemm_tile.hpp"

using namespace c4q;

namespace {

__device__ __forceinline__ float half_f32(uint16_t h, bool bf16) {
  return bf16 ? bf16_f32(h) : f16_f32(h);
}
// T rounding (RNE) of v as a float; bf16 through v_cvt_pk_bf16_f32, which
// equals bf16_rte for every non-NaN float (checked on all 2^32 inputs).
__device__ __forceinline__ float round_half(float v, bool bf16) {
  return bf16 ? bf16lo(bf16x2_rne(v, 0.0f)) : f16_f32(f16_rte(v));
}

// Max over the 256 threads of a workgroup (values are >= 0).
__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

// One workgroup per row; bit-exact restatement of comfy_kitchen
// quantize_int8_rowwise (reference _patches/int8_ext/int8_gemm.mm:1337-1381):
//   scale = max(amax / 127, 1e-30)  (fp32, correctly rounded divide; stored)
//   s     = T(scale), 0 -> finfo(T).tiny
//   q     = int8(clamp(rint(T(x / s)), -128, 127))
// T(x / s) with the row's divisor s (a T value) and its reciprocal r: bf16
// rows use the reciprocal quotient (div_bf16_operands, equal after bf16
// rounding to the correctly rounded quotient); f16 rows divide.
template <bool BF16>
__device__ __forceinline__ uint32_t quant_i8(uint16_t h, float s, float r) {
  const float x = half_f32(h, BF16);
  float v = round_half(BF16 ? div_bf16_operands(x, s, r) : x / s, BF16);
  v = rintf(v);
  v = fminf(fmaxf(v, -128.0f), 127.0f);
  return (uint32_t)(uint8_t)(int8_t)(int)v;
}

// VEC: rows read 8 elements (16 bytes) and written 8 bytes at a time (the
// entry point checks alignment, strides and K % 8).
// CACHE (with VEC, K <= 8192): each thread keeps its at most four 8-element
// chunks of the row in registers, so the row is read once.
template <bool BF16, bool VEC, bool CACHE>
__global__ void __launch_bounds__(256)
quant_rowwise_kernel(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                     int64_t K) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  float mx = 0.0f;
  if constexpr (CACHE) {
    uint4 u[4];
    const int k0 = (int)threadIdx.x * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (k0 + 2048 * c < K) u[c] = *reinterpret_cast<const uint4*>(xr + k0 + 2048 * c);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (k0 + 2048 * c >= K) continue;
      const uint32_t w[4] = {u[c].x, u[c].y, u[c].z, u[c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        mx = fmaxf(mx, fmaxf(fabsf(half_f32((uint16_t)w[e], BF16)),
                             fabsf(half_f32((uint16_t)(w[e] >> 16), BF16))));
    }
    const float amax = block_max256(mx, red);
    const float scale = fmaxf(amax / 127.0f, 1e-30f);
    if (threadIdx.x == 0) scales[row] = scale;
    float s = round_half(scale, BF16);
    if (s == 0.0f) s = BF16 ? 1.1754943508222875e-38f : 6.103515625e-05f;
    const float rs = 1.0f / s;
    int8_t* qr = q + row * ldq;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (k0 + 2048 * c >= K) continue;
      const uint32_t w[4] = {u[c].x, u[c].y, u[c].z, u[c].w};
      uint32_t o[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        o[h] = quant_i8<BF16>((uint16_t)w[2 * h], s, rs) |
               (quant_i8<BF16>((uint16_t)(w[2 * h] >> 16), s, rs) << 8) |
               (quant_i8<BF16>((uint16_t)w[2 * h + 1], s, rs) << 16) |
               (quant_i8<BF16>((uint16_t)(w[2 * h + 1] >> 16), s, rs) << 24);
      *reinterpret_cast<uint2*>(qr + k0 + 2048 * c) = uint2{o[0], o[1]};
    }
    return;
  }
  if constexpr (VEC) {
    for (int64_t i = threadIdx.x * 8; i < K; i += 2048) {
      const uint4 u = *reinterpret_cast<const uint4*>(xr + i);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        mx = fmaxf(mx, fmaxf(fabsf(half_f32((uint16_t)w[c], BF16)),
                             fabsf(half_f32((uint16_t)(w[c] >> 16), BF16))));
    }
  } else {
    for (int64_t i = threadIdx.x; i < K; i += 256) mx = fmaxf(mx, fabsf(half_f32(xr[i], BF16)));
  }
  const float amax = block_max256(mx, red);
  const float scale = fmaxf(amax / 127.0f, 1e-30f);
  if (threadIdx.x == 0) scales[row] = scale;
  float s = round_half(scale, BF16);
  if (s == 0.0f) s = BF16 ? 1.1754943508222875e-38f : 6.103515625e-05f;
  const float rs = 1.0f / s;
  int8_t* qr = q + row * ldq;
  if constexpr (VEC) {
    for (int64_t i = threadIdx.x * 8; i < K; i += 2048) {
      const uint4 u = *reinterpret_cast<const uint4*>(xr + i);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
      uint32_t o[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
        o[c] = quant_i8<BF16>((uint16_t)w[2 * c], s, rs) |
               (quant_i8<BF16>((uint16_t)(w[2 * c] >> 16), s, rs) << 8) |
               (quant_i8<BF16>((uint16_t)w[2 * c + 1], s, rs) << 16) |
               (quant_i8<BF16>((uint16_t)(w[2 * c + 1] >> 16), s, rs) << 24);
      *reinterpret_cast<uint2*>(qr + i) = uint2{o[0], o[1]};
    }
  } else {
    for (int64_t i = threadIdx.x; i < K; i += 256) qr[i] = (int8_t)quant_i8<BF16>(xr[i], s, rs);
  }
}

// Fused head merge + ConvRot + rowwise quant (reference
// i8_merge_rot_quant_bf16, _patches/int8_ext/int8_gemm.mm:1429-1507): x
// [B, H, S, D] bf16 contiguous; output row (b, s) of the merged [B*S, H*D]
// matrix, element i = h*D + d. One workgroup per output row, in three
// passes over the row held in LDS:
//   1. gather: the H head runs of D elements, 16 bytes per load (all loads
//      of the row in flight at once) where D and x allow, else 2 bytes;
//   2. with ROTATE, every 256-element group is transformed in place by the
//      radix-4 Walsh-Hadamard butterflies at strides 1, 4, 16, 64 (row
//      `digit` of H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] applied
//      to the values at base + k*stride, each sum in fp32 in the written
//      order), scaled by 2^-4 and rounded to bf16. Wave w takes groups w,
//      w + 4, ...: lane l holds group elements l + 64 j (j = 0..3), so the
//      stride-64 stage is lane-local and the other three go through a
//      wave-private LDS row (no workgroup barrier);
//   3. the rowwise quant arithmetic above, 16 outputs per thread stored as
//      one 16-byte write where q allows.
// Row `digit` of H4 negates operand 3 - digit. Each row is the reference's
// expression (a0 + a1 + a2 - a3, a0 + a1 - a2 + a3, a0 - a1 + a2 + a3,
// -a0 + a1 + a2 + a3, summed left to right): x - y is x + (-y) exactly, so
// flipping one sign bit and adding in the same order gives the same bits,
// without a branch on the lane's digit.
__device__ __forceinline__ float h4_row(int digit, float a0, float a1, float a2, float a3) {
  const uint32_t sgn = 0x80000000u;
  a0 = bits_f32(f32_bits(a0) ^ (digit == 3 ? sgn : 0u));
  a1 = bits_f32(f32_bits(a1) ^ (digit == 2 ? sgn : 0u));
  a2 = bits_f32(f32_bits(a2) ^ (digit == 1 ? sgn : 0u));
  a3 = bits_f32(f32_bits(a3) ^ (digit == 0 ? sgn : 0u));
  return ((a0 + a1) + a2) + a3;
}


// Two radix-4 stages of the Walsh-Hadamard transform on 16 values held by
// one lane: v[4 hi + lo] with `lo` the digit of the first stage and `hi` the
// digit of the second (each output the reference's row expression).
__device__ __forceinline__ void h4_two_stages(float (&v)[16]) {
  float t[16];
#pragma unroll
  for (int hi = 0; hi < 4; ++hi)
#pragma unroll
    for (int lo = 0; lo < 4; ++lo)
      t[4 * hi + lo] = h4_row(lo, v[4 * hi], v[4 * hi + 1], v[4 * hi + 2], v[4 * hi + 3]);
#pragma unroll
  for (int lo = 0; lo < 4; ++lo)
#pragma unroll
    for (int hi = 0; hi < 4; ++hi)
      v[4 * hi + lo] = h4_row(hi, t[lo], t[4 + lo], t[8 + lo], t[12 + lo]);
}

constexpr int kRotSlot = 256 + 16;   // floats per group slot of a wave (padding spreads banks)

// The rotation of one 256-element group by a team of 16 lanes (c = lane &
// 15): on entry lane c holds elements 16 c + m in v[m] (the stride-1 and
// stride-4 digits are the two digits of m); on return it holds the
// transformed elements c + 16 m (times 2^-4, rounded to bf16), having passed
// through `slot` (the team's 256 + 16 floats of LDS) once. Every lane of the
// wave calls it (`live` false: the lane only keeps the wave in step).
__device__ __forceinline__ void rot_group16(float (&v)[16], float* slot, int c, bool live) {
  if (live) {
    h4_two_stages(v);                                       // strides 1 and 4
#pragma unroll
    for (int k = 0; k < 4; ++k)
      *reinterpret_cast<float4*>(slot + 16 * c + 4 * k) =
          make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  }
  lds_fence_wave();
  if (live) {
#pragma unroll
    for (int m = 0; m < 16; ++m) v[m] = slot[c + 16 * m];
    h4_two_stages(v);                                       // strides 16 and 64
#pragma unroll
    for (int m = 0; m < 16; m += 2) {
      const uint32_t p = bf16x2_rne(v[m] * 0.0625f, v[m + 1] * 0.0625f);
      v[m] = bf16lo(p);
      v[m + 1] = bf16hi(p);
    }
  }
  lds_fence_wave();                                         // slot free again
}

// Rowwise quant of a bf16 row held in LDS (256 threads, after the barrier
// that produced amax): the i8_quant_rowwise arithmetic, 16-byte stores of
// 16 codes per thread where q is aligned (K is a multiple of 256).
__device__ __forceinline__ void quant_row_from_lds(const uint16_t* rot, int K, float amax, int8_t* qr,
                                                   float* scale_out, int vec_q) {
  const int tid = threadIdx.x;
  const float scale = fmaxf(amax / 127.0f, 1e-30f);
  if (tid == 0) *scale_out = scale;
  float sc = round_half(scale, true);
  if (sc == 0.0f) sc = 1.1754943508222875e-38f;
  const float rc = 1.0f / sc;
  if (vec_q) {
    for (int i = tid * 16; i < K; i += 4096) {
      const uint4 lo = *reinterpret_cast<const uint4*>(rot + i);
      const uint4 hi = *reinterpret_cast<const uint4*>(rot + i + 8);
      const uint32_t h16[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      uint32_t out[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        out[c] = quant_i8<true>((uint16_t)h16[2 * c], sc, rc) |
                 (quant_i8<true>((uint16_t)(h16[2 * c] >> 16), sc, rc) << 8) |
                 (quant_i8<true>((uint16_t)h16[2 * c + 1], sc, rc) << 16) |
                 (quant_i8<true>((uint16_t)(h16[2 * c + 1] >> 16), sc, rc) << 24);
      *reinterpret_cast<uint4*>(qr + i) = uint4{out[0], out[1], out[2], out[3]};
    }
  } else {
    for (int i = tid; i < K; i += 256) qr[i] = (int8_t)quant_i8<true>(rot[i], sc, rc);
  }
}

template <bool ROTATE>
__global__ void __launch_bounds__(256)
merge_rot_quant_kernel(const uint16_t* x, int64_t H, int64_t S, int64_t D, int8_t* q,
                       float* scales, int vec_x, int vec_q) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rot[];   // the row, H*D bf16
  __shared__ __attribute__((aligned(16))) float work[4][4 * kRotSlot];
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t b = row / S, s = row - b * S;
  const int K = (int)(H * D);
  const int groups = K >> 8;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint16_t* xr = x + (b * H * S + s) * D;        // head h at xr + h * S * D
  const int64_t hstride = S * D;
  const int d_ = (int)D;
  if (vec_x) {
    for (int i = tid * 8; i < K; i += 2048) {
      const int h = i / d_, d = i - h * d_;
      *reinterpret_cast<uint4*>(rot + i) = *reinterpret_cast<const uint4*>(xr + h * hstride + d);
    }
  } else {
    for (int i = tid; i < K; i += 256) {
      const int h = i / d_, d = i - h * d_;
      rot[i] = xr[h * hstride + d];
    }
  }
  __syncthreads();
  // A wave takes 4 groups at a time, 16 lanes each: lane c = lane & 15 of
  // slot gq = lane >> 4 first holds elements 16 c + m (m = 0..15; the
  // stride-1 and stride-4 digits are the two digits of m), then, after a
  // transpose through the wave's LDS slots, elements c + 16 m (the stride-16
  // and stride-64 digits).
  float mx = 0.0f;
  const int gq = lane >> 4, c = lane & 15;
  float* slot = work[wave] + gq * kRotSlot;
  for (int g0 = wave * 4; g0 < groups; g0 += 16) {
    const int g = g0 + gq;
    const bool live = g < groups;
    uint16_t* grp = rot + g * 256;
    float v[16];
    if (live) {
      const uint4 lo = *reinterpret_cast<const uint4*>(grp + 16 * c);
      const uint4 hi = *reinterpret_cast<const uint4*>(grp + 16 * c + 8);
      const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[2 * k] = bf16_f32((uint16_t)w[k]);
        v[2 * k + 1] = bf16_f32((uint16_t)(w[k] >> 16));
      }
    }
    if constexpr (ROTATE) {
      rot_group16(v, slot, c, live);
      if (live) {
#pragma unroll
        for (int m = 0; m < 16; ++m) grp[c + 16 * m] = (uint16_t)(f32_bits(v[m]) >> 16);
      }
    }
    if (live) {
#pragma unroll
      for (int m = 0; m < 16; ++m) mx = fmaxf(mx, fabsf(v[m]));
    }
  }
  const float amax = block_max256(mx, red);    // its barrier also publishes the rotated row
  quant_row_from_lds(rot, K, amax, q + row * (int64_t)K, scales + row, vec_q);
}

// SwiGLU + ConvRot pre-pass of an H3 INT8 fc2 (reference i8_swiglu_rot_bf16,
// _patches/int8_ext/int8_gemm.mm:1521-1554): x [M, 2F] bf16 rows (gate
// columns [0, F), up columns [F, 2F)) -> rot [M, F] bf16 with
//   act = bf16(f32(SiLU[a]) * f32(b))   (SiLU: the 65,536-entry bf16 table)
// rotated per 256-element group as in merge_rot_quant_kernel. One workgroup
// per row; a wave takes 4 groups at a time, 16 lanes each; the rotated group
// goes back through the team's LDS slot so that each lane stores 16
// consecutive outputs (two 16-byte writes).
__global__ void __launch_bounds__(256)
swiglu_rot_kernel(const uint16_t* x, int64_t F, const uint16_t* silu, uint16_t* rot) {
  __shared__ __attribute__((aligned(16))) float work[4][4 * kRotSlot];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * 2 * F;
  uint16_t* rr = rot + row * F;
  const int groups = (int)(F >> 8);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gq = lane >> 4, c = lane & 15;
  float* slot = work[wave] + gq * kRotSlot;
  for (int g0 = wave * 4; g0 < groups; g0 += 16) {
    const int g = g0 + gq;
    const bool live = g < groups;
    float v[16];
    if (live) {
      const uint16_t* ga = xr + g * 256 + 16 * c;
      const uint4 a0 = *reinterpret_cast<const uint4*>(ga);
      const uint4 a1 = *reinterpret_cast<const uint4*>(ga + 8);
      const uint4 b0 = *reinterpret_cast<const uint4*>(ga + F);
      const uint4 b1 = *reinterpret_cast<const uint4*>(ga + F + 8);
      const uint32_t wa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t wb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float s0 = bf16_f32(silu[wa[k] & 0xFFFFu]), s1 = bf16_f32(silu[wa[k] >> 16]);
        const uint32_t p = bf16x2_rne(s0 * bf16lo(wb[k]), s1 * bf16hi(wb[k]));
        v[2 * k] = bf16lo(p);
        v[2 * k + 1] = bf16hi(p);
      }
    }
    rot_group16(v, slot, c, live);
    // back through the slot (bf16 bits) to 16 consecutive outputs per lane
    uint16_t* bslot = reinterpret_cast<uint16_t*>(slot);
    if (live) {
#pragma unroll
      for (int m = 0; m < 16; ++m) bslot[c + 16 * m] = (uint16_t)(f32_bits(v[m]) >> 16);
    }
    lds_fence_wave();
    if (live) {
      const uint4 o0 = *reinterpret_cast<const uint4*>(bslot + 16 * c);
      const uint4 o1 = *reinterpret_cast<const uint4*>(bslot + 16 * c + 8);
      *reinterpret_cast<uint4*>(rr + g * 256 + 16 * c) = o0;
      *reinterpret_cast<uint4*>(rr + g * 256 + 16 * c + 8) = o1;
    }
    lds_fence_wave();
  }
}

// The SwiGLU + ConvRot pass and the rowwise quant of its rows in one pass
// (the MLP bridge's second and third steps without the bf16 row in HBM):
// x [M, 2F] bf16 -> q [M, F] int8 and scales [M], the bytes of
// i8_quant_rowwise(swiglu_rot(x)). One workgroup per row; the rotated row
// (F bf16, F <= 15360) is kept in LDS for the quant, as in
// merge_rot_quant_kernel.
__global__ void __launch_bounds__(256)
swiglu_rot_quant_kernel(const uint16_t* x, int64_t F, const uint16_t* silu, int8_t* q,
                        float* scales, int vec_q) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rot[];   // the rotated row, F bf16
  __shared__ __attribute__((aligned(16))) float work[4][4 * kRotSlot];
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * 2 * F;
  const int groups = (int)(F >> 8);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gq = lane >> 4, c = lane & 15;
  float* slot = work[wave] + gq * kRotSlot;
  float mx = 0.0f;
  for (int g0 = wave * 4; g0 < groups; g0 += 16) {
    const int g = g0 + gq;
    const bool live = g < groups;
    float v[16];
    if (live) {
      const uint16_t* ga = xr + g * 256 + 16 * c;
      const uint4 a0 = *reinterpret_cast<const uint4*>(ga);
      const uint4 a1 = *reinterpret_cast<const uint4*>(ga + 8);
      const uint4 b0 = *reinterpret_cast<const uint4*>(ga + F);
      const uint4 b1 = *reinterpret_cast<const uint4*>(ga + F + 8);
      const uint32_t wa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t wb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float s0 = bf16_f32(silu[wa[k] & 0xFFFFu]), s1 = bf16_f32(silu[wa[k] >> 16]);
        const uint32_t p = bf16x2_rne(s0 * bf16lo(wb[k]), s1 * bf16hi(wb[k]));
        v[2 * k] = bf16lo(p);
        v[2 * k + 1] = bf16hi(p);
      }
    }
    rot_group16(v, slot, c, live);
    if (live) {
      uint16_t* grp = rot + g * 256;
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        grp[c + 16 * m] = (uint16_t)(f32_bits(v[m]) >> 16);
        mx = fmaxf(mx, fabsf(v[m]));
      }
    }
  }
  const float amax = block_max256(mx, red);    // its barrier also publishes the rotated row
  quant_row_from_lds(rot, (int)F, amax, q + row * F, scales + row, vec_q);
}

__global__ void fill_zero_kernel(float* p) { p[0] = 0.0f; }

// amax of |x| over n elements into *amax (bits of a non-negative float
// compare like unsigned integers, so atomicMax on the bits is a float max).
// VEC: x 16-byte aligned; the first n & ~7 elements are read 8 at a time.
template <bool BF16, bool VEC>
__global__ void __launch_bounds__(256)
absmax_kernel(const uint16_t* x, int64_t n, float* amax) {
  __shared__ float red[4];
  float mx = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t done = 0;
  if constexpr (VEC) {
    const int64_t n8 = n >> 3;
    for (int64_t i = t; i < n8; i += stride) {
      const uint4 u = *reinterpret_cast<const uint4*>(x + i * 8);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        mx = fmaxf(mx, fmaxf(fabsf(half_f32((uint16_t)w[c], BF16)),
                             fabsf(half_f32((uint16_t)(w[c] >> 16), BF16))));
    }
    done = n8 * 8;
  }
  for (int64_t i = done + t; i < n; i += stride) mx = fmaxf(mx, fabsf(half_f32(x[i], BF16)));
  mx = block_max256(mx, red);
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<unsigned int*>(amax), __float_as_uint(mx));
}

// q = e4m3fn(clamp(x / scale, -448, 448)); scale = amax / 448, or 1 for an
// all-zero tensor. NaN passes the clamp and encodes as NaN, as torch's
// clamp-then-cast does. VEC: x 16-byte and q 8-byte aligned. The quotient
// comes from one reciprocal per thread and a fused residual step per element
// where rcp_quot_ok(scale) (its e4m3 code equals that of the IEEE quotient,
// see numerics.hpp), else from the IEEE division; the codes from e4m3_pair
// (the hardware conversion, equal to f32_e4m3 of the clamped value).
template <bool BF16, bool FAST>
__device__ __forceinline__ float quot_scale(uint16_t h, float s, float r) {
  const float x = half_f32(h, BF16);
  return FAST ? div_bf16_operands(x, s, r) : x / s;
}

template <bool BF16, bool VEC, bool FAST>
__device__ __forceinline__ void quant_pertensor_body(const uint16_t* x, int64_t n, uint8_t* q,
                                                     float s, float r) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t done = 0;
  if constexpr (VEC) {
    const int64_t n8 = n >> 3;
    for (int64_t i = t; i < n8; i += stride) {
      const uint4 u = *reinterpret_cast<const uint4*>(x + i * 8);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
      uint32_t o[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint32_t lo = e4m3_pair(quot_scale<BF16, FAST>((uint16_t)w[2 * c], s, r),
                                      quot_scale<BF16, FAST>((uint16_t)(w[2 * c] >> 16), s, r));
        const uint32_t hi = e4m3_pair(quot_scale<BF16, FAST>((uint16_t)w[2 * c + 1], s, r),
                                      quot_scale<BF16, FAST>((uint16_t)(w[2 * c + 1] >> 16), s, r));
        o[c] = lo | (hi << 16);
      }
      *reinterpret_cast<uint2*>(q + i * 8) = uint2{o[0], o[1]};
    }
    done = n8 * 8;
  }
  for (int64_t i = done + t; i < n; i += stride)
    q[i] = (uint8_t)(e4m3_pair(quot_scale<BF16, FAST>(x[i], s, r), 0.0f) & 0xFFu);
}

template <bool BF16, bool VEC>
__global__ void __launch_bounds__(256)
quant_pertensor_kernel(const uint16_t* x, int64_t n, uint8_t* q, float* scale,
                       const float* amax) {
  float s = amax[0] / 448.0f;
  if (s == 0.0f) s = 1.0f;
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
  if (rcp_quot_ok(s)) quant_pertensor_body<BF16, VEC, true>(x, n, q, s, 1.0f / s);
  else quant_pertensor_body<BF16, VEC, false>(x, n, q, s, 0.0f);
}

// fp8 -> T dequant with the same conversion routine the W8A16 GEMM uses
// while staging weights (dequant4), plus a scalar path for the tail.
template <bool BF16, bool HAS_SCALE>
__global__ void __launch_bounds__(256)
dequant_kernel(const uint8_t* w, int64_t n, const float* sp, uint16_t* out, bool vec) {
  const float s = HAS_SCALE ? round_half(sp[0], BF16) : 1.0f;
  const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i4 >= n) return;
  if (vec && i4 + 4 <= n) {
    uint32_t word = *reinterpret_cast<const uint32_t*>(w + i4);
    uint32_t lo, hi;
    dequant4<BF16, HAS_SCALE>(word, s, lo, hi);
    out[i4 + 0] = (uint16_t)(lo & 0xFFFFu);
    out[i4 + 1] = (uint16_t)(lo >> 16);
    out[i4 + 2] = (uint16_t)(hi & 0xFFFFu);
    out[i4 + 3] = (uint16_t)(hi >> 16);
    return;
  }
  for (int64_t i = i4; i < n && i < i4 + 4; ++i) {
    float v = e4m3_f32(w[i]);
    if (HAS_SCALE) v = v * s;
    out[i] = BF16 ? bf16_rte(v) : f16_rte(v);
  }
}

__global__ void __launch_bounds__(256)
dequant_f32_kernel(const uint8_t* w, int64_t n, const float* sp, float* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v = e4m3_f32(w[i]);
  if (sp) v = v * sp[0];
  out[i] = v;
}

int grid_for(int64_t n) {
  int64_t b = cdiv(n, 256);
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

extern "C" int c4q_i8_quant_rowwise(const void* x, int x_dtype, int64_t ldx, int8_t* q,
                                    int64_t ldq, float* scales, int64_t M, int64_t K,
                                    void* stream) {
  const char* what = "c4q_i8_quant_rowwise";
  C4Q_REQUIRE(x_dtype == C4Q_BF16 || x_dtype == C4Q_F16, C4Q_ERR_ARG,
              "%s: x must be bf16 or f16", what);
  C4Q_REQUIRE(M >= 0 && K >= 0 && ldx >= K && ldq >= K, C4Q_ERR_SHAPE, "%s: bad shape", what);
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(scales && (K == 0 || (x && q)), C4Q_ERR_ARG, "%s: null pointer", what);
  C4Q_REQUIRE(M < (1ll << 31), C4Q_ERR_SHAPE, "%s: too many rows", what);
  hipStream_t s = as_stream(stream);
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  const bool vec = aligned16(xs) && ldx % 8 == 0 && K % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(q) & 7u) == 0 && ldq % 8 == 0;
  const bool cache = vec && K <= 8192;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)M), dim3(256), 0, s, xs, ldx, q, ldq, scales, K);
  };
  if (x_dtype == C4Q_BF16) {
    if (cache) launch(quant_rowwise_kernel<true, true, true>);
    else if (vec) launch(quant_rowwise_kernel<true, true, false>);
    else launch(quant_rowwise_kernel<true, false, false>);
  } else {
    if (cache) launch(quant_rowwise_kernel<false, true, true>);
    else if (vec) launch(quant_rowwise_kernel<false, true, false>);
    else launch(quant_rowwise_kernel<false, false, false>);
  }
  return check_launch(what);
}

extern "C" int c4q_i8_merge_rot_quant(const uint16_t* x, int64_t B, int64_t H, int64_t S,
                                      int64_t D, int rotate, int8_t* q, float* scales,
                                      void* stream) {
  const char* what = "c4q_i8_merge_rot_quant";
  C4Q_REQUIRE(B >= 0 && H >= 1 && S >= 0 && D > 0 && D <= 256, C4Q_ERR_SHAPE,
              "%s: need B, S >= 0, H >= 1, 0 < D <= 256 (B=%lld H=%lld S=%lld D=%lld)", what,
              (long long)B, (long long)H, (long long)S, (long long)D);
  const int64_t K = H * D;
  C4Q_REQUIRE(K % 256 == 0, C4Q_ERR_SHAPE, "%s: merged width H*D=%lld must tile 256-element groups",
              what, (long long)K);
  C4Q_REQUIRE(K * 2 <= 30 * 1024, C4Q_ERR_SHAPE, "%s: H*D=%lld too large (at most 15360)", what,
              (long long)K);
  const int64_t M = B * S;
  if (M == 0) return C4Q_OK;
  C4Q_REQUIRE(M < (1ll << 31), C4Q_ERR_SHAPE, "%s: too many rows", what);
  C4Q_REQUIRE(x && q && scales, C4Q_ERR_ARG, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const size_t lds = (size_t)K * 2;
  const int vec_x = aligned16(x) && D % 8 == 0;      // every head run: whole 16-byte chunks
  const int vec_q = aligned16(q);                     // rows of K bytes, K a multiple of 256
  if (rotate)
    hipLaunchKernelGGL(merge_rot_quant_kernel<true>, dim3((unsigned)M), dim3(256), lds, s, x, H, S,
                       D, q, scales, vec_x, vec_q);
  else
    hipLaunchKernelGGL(merge_rot_quant_kernel<false>, dim3((unsigned)M), dim3(256), lds, s, x, H, S,
                       D, q, scales, vec_x, vec_q);
  return check_launch(what);
}

extern "C" int c4q_i8_swiglu_rot(const uint16_t* x, int64_t M, int64_t F,
                                 const uint16_t* silu_table, uint16_t* rot, void* stream) {
  const char* what = "c4q_i8_swiglu_rot";
  C4Q_REQUIRE(M >= 0 && F >= 0 && F % 256 == 0, C4Q_ERR_SHAPE,
              "%s: need M >= 0 and F a multiple of 256 (M=%lld F=%lld)", what, (long long)M,
              (long long)F);
  if (M == 0 || F == 0) return C4Q_OK;
  C4Q_REQUIRE(M < (1ll << 31), C4Q_ERR_SHAPE, "%s: too many rows", what);
  C4Q_REQUIRE(x && rot && silu_table, C4Q_ERR_ARG, "%s: null pointer", what);
  C4Q_REQUIRE(aligned16(x) && aligned16(rot), C4Q_ERR_ARG, "%s: x and rot must be 16-byte aligned",
              what);
  hipLaunchKernelGGL(swiglu_rot_kernel, dim3((unsigned)M), dim3(256), 0, as_stream(stream), x, F,
                     silu_table, rot);
  return check_launch(what);
}

extern "C" int c4q_i8_swiglu_rot_quant(const uint16_t* x, int64_t M, int64_t F,
                                       const uint16_t* silu_table, int8_t* q, float* scales,
                                       void* stream) {
  const char* what = "c4q_i8_swiglu_rot_quant";
  C4Q_REQUIRE(M >= 0 && F >= 0 && F % 256 == 0 && F * 2 <= 30 * 1024, C4Q_ERR_SHAPE,
              "%s: need F a multiple of 256, at most 15360 (M=%lld F=%lld)", what, (long long)M,
              (long long)F);
  if (M == 0 || F == 0) return C4Q_OK;
  C4Q_REQUIRE(M < (1ll << 31), C4Q_ERR_SHAPE, "%s: too many rows", what);
  C4Q_REQUIRE(x && q && scales && silu_table, C4Q_ERR_ARG, "%s: null pointer", what);
  C4Q_REQUIRE(aligned16(x), C4Q_ERR_ARG, "%s: x must be 16-byte aligned", what);
  hipLaunchKernelGGL(swiglu_rot_quant_kernel, dim3((unsigned)M), dim3(256), (size_t)F * 2,
                     as_stream(stream), x, F, silu_table, q, scales, (int)aligned16(q));
  return check_launch(what);
}

extern "C" int c4q_f8_quant_pertensor(const void* x, int x_dtype, int64_t n, uint8_t* q,
                                      float* scale, float* amax_ws, void* stream) {
  const char* what = "c4q_f8_quant_pertensor";
  C4Q_REQUIRE(x_dtype == C4Q_BF16 || x_dtype == C4Q_F16, C4Q_ERR_ARG,
              "%s: x must be bf16 or f16", what);
  C4Q_REQUIRE(n >= 0, C4Q_ERR_SHAPE, "%s: negative size", what);
  C4Q_REQUIRE(scale && amax_ws && (n == 0 || (x && q)), C4Q_ERR_ARG, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  const bool vec = aligned16(xs) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0;
  const int g = grid_for(vec ? cdiv(n, 8) : n);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(1), 0, s, amax_ws);
  auto run = [&](auto amax_k, auto quant_k) {
    hipLaunchKernelGGL(amax_k, dim3(g), dim3(256), 0, s, xs, n, amax_ws);
    hipLaunchKernelGGL(quant_k, dim3(g), dim3(256), 0, s, xs, n, q, scale, amax_ws);
  };
  if (x_dtype == C4Q_BF16) {
    if (vec) run(absmax_kernel<true, true>, quant_pertensor_kernel<true, true>);
    else run(absmax_kernel<true, false>, quant_pertensor_kernel<true, false>);
  } else {
    if (vec) run(absmax_kernel<false, true>, quant_pertensor_kernel<false, true>);
    else run(absmax_kernel<false, false>, quant_pertensor_kernel<false, false>);
  }
  return check_launch(what);
}

extern "C" int c4q_fp8_dequant(const uint8_t* w, int64_t n, const float* scale, void* out,
                               int out_dtype, void* stream) {
  const char* what = "c4q_fp8_dequant";
  C4Q_REQUIRE(out_dtype == C4Q_BF16 || out_dtype == C4Q_F16 || out_dtype == C4Q_F32, C4Q_ERR_ARG,
              "%s: bad output dtype", what);
  C4Q_REQUIRE(n >= 0, C4Q_ERR_SHAPE, "%s: negative size", what);
  if (n == 0) return C4Q_OK;
  C4Q_REQUIRE(w && out, C4Q_ERR_ARG, "%s: null pointer", what);
  hipStream_t s = as_stream(stream);
  if (out_dtype == C4Q_F32) {
    const int64_t blocks = cdiv(n, 256);
    C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: too large", what);
    hipLaunchKernelGGL(dequant_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w, n, scale,
                       static_cast<float*>(out));
    return check_launch(what);
  }
  const int64_t blocks = cdiv(cdiv(n, 4), 256);
  C4Q_REQUIRE(blocks < (1ll << 31), C4Q_ERR_SHAPE, "%s: too large", what);
  const bool vec = (reinterpret_cast<uintptr_t>(w) & 3u) == 0;
  uint16_t* o = static_cast<uint16_t*>(out);
  dim3 grid((unsigned)blocks), blk(256);
  if (out_dtype == C4Q_BF16) {
    if (scale) hipLaunchKernelGGL((dequant_kernel<true, true>), grid, blk, 0, s, w, n, scale, o, vec);
    else hipLaunchKernelGGL((dequant_kernel<true, false>), grid, blk, 0, s, w, n, scale, o, vec);
  } else {
    if (scale) hipLaunchKernelGGL((dequant_kernel<false, true>), grid, blk, 0, s, w, n, scale, o, vec);
    else hipLaunchKernelGGL((dequant_kernel<false, false>), grid, blk, 0, s, w, n, scale, o, vec);
  }
  return check_launch(what);
}
