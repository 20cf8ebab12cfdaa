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
__device__ __forceinline__ float round_half(float v, bool bf16) {
  return bf16 ? bf16_f32(bf16_rte(v)) : f16_f32(f16_rte(v));
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
template <bool BF16>
__global__ void __launch_bounds__(256)
quant_rowwise_kernel(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* scales,
                     int64_t K) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  float mx = 0.0f;
  for (int64_t i = threadIdx.x; i < K; i += 256) mx = fmaxf(mx, fabsf(half_f32(xr[i], BF16)));
  const float amax = block_max256(mx, red);
  const float scale = fmaxf(amax / 127.0f, 1e-30f);
  if (threadIdx.x == 0) scales[row] = scale;
  float s = round_half(scale, BF16);
  if (s == 0.0f) s = BF16 ? 1.1754943508222875e-38f : 6.103515625e-05f;
  int8_t* qr = q + row * ldq;
  for (int64_t i = threadIdx.x; i < K; i += 256) {
    float v = round_half(half_f32(xr[i], BF16) / s, BF16);
    v = rintf(v);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    qr[i] = (int8_t)(int)v;
  }
}

// Fused head merge + ConvRot + rowwise quant (reference
// i8_merge_rot_quant_bf16, _patches/int8_ext/int8_gemm.mm:1429-1507): x
// [B, H, S, D] bf16 contiguous; output row (b, s) of the merged [B*S, H*D]
// matrix, element i = h*D + d. One workgroup per output row. With ROTATE,
// every 256-element group is transformed by the radix-4 Walsh-Hadamard
// butterflies at strides 1, 4, 16, 64 (row `digit` of
// H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] applied to the values at
// base + k*stride, each sum in fp32 in the written order), scaled by 2^-4 and
// rounded to bf16. Wave w takes groups w, w + 4, ...: lane l holds group
// elements l + 64 j (j = 0..3), so the stride-64 stage is lane-local and the
// other three stages go through a wave-private LDS row (no workgroup
// barrier). The rotated row stays in LDS for the quant pass, which is the
// rowwise arithmetic above.
__device__ __forceinline__ float h4_row(int digit, float a0, float a1, float a2, float a3) {
  if (digit == 0) return a0 + a1 + a2 - a3;
  if (digit == 1) return a0 + a1 - a2 + a3;
  if (digit == 2) return a0 - a1 + a2 + a3;
  return -a0 + a1 + a2 + a3;
}

template <bool ROTATE>
__global__ void __launch_bounds__(256)
merge_rot_quant_kernel(const uint16_t* x, int64_t H, int64_t S, int64_t D, int8_t* q,
                       float* scales) {
  extern __shared__ uint16_t rot[];            // the row's H*D rotated bf16 values
  __shared__ float work[4][256];
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t b = row / S, s = row - b * S;
  const int64_t K = H * D;
  const int groups = (int)(K >> 8);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* w = work[wave];
  float mx = 0.0f;
  for (int g = wave; g < groups; g += 4) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = (int64_t)g * 256 + lane + 64 * j;
      const int64_t h = i / D, d = i - h * D;
      v[j] = bf16_f32(x[((b * H + h) * S + s) * D + d]);
    }
    if constexpr (ROTATE) {
#pragma unroll
      for (int stride = 1; stride <= 16; stride *= 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[lane + 64 * j] = v[j];
        lds_fence_wave();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int idx = lane + 64 * j;
          const int digit = (idx / stride) & 3;
          const int base = idx - digit * stride;
          v[j] = h4_row(digit, w[base], w[base + stride], w[base + 2 * stride], w[base + 3 * stride]);
        }
        lds_fence_wave();
      }
      // stride 64: the four values of the group are this lane's v[0..3],
      // and element l + 64 j has digit j
      const float a0 = v[0], a1 = v[1], a2 = v[2], a3 = v[3];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = bf16_f32(bf16_rte(h4_row(j, a0, a1, a2, a3) * 0.0625f));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rot[g * 256 + lane + 64 * j] = (uint16_t)(f32_bits(v[j]) >> 16);   // v[j] is a bf16 value
      mx = fmaxf(mx, fabsf(v[j]));
    }
  }
  const float amax = block_max256(mx, red);    // also orders the rot writes before the reads
  const float scale = fmaxf(amax / 127.0f, 1e-30f);
  if (threadIdx.x == 0) scales[row] = scale;
  float sc = round_half(scale, true);
  if (sc == 0.0f) sc = 1.1754943508222875e-38f;
  int8_t* qr = q + row * K;
  for (int64_t i = threadIdx.x; i < K; i += 256) {
    float r = round_half(bf16_f32(rot[i]) / sc, true);
    r = rintf(r);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    qr[i] = (int8_t)(int)r;
  }
}

__global__ void fill_zero_kernel(float* p) { p[0] = 0.0f; }

// amax of |x| over n elements into *amax (bits of a non-negative float
// compare like unsigned integers, so atomicMax on the bits is a float max).
template <bool BF16>
__global__ void __launch_bounds__(256)
absmax_kernel(const uint16_t* x, int64_t n, float* amax) {
  __shared__ float red[4];
  float mx = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    mx = fmaxf(mx, fabsf(half_f32(x[i], BF16)));
  mx = block_max256(mx, red);
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<unsigned int*>(amax), __float_as_uint(mx));
}

// q = e4m3fn(clamp(x / scale, -448, 448)); scale = amax / 448, or 1 for an
// all-zero tensor. NaN passes the clamp and encodes as NaN, as torch's
// clamp-then-cast does.
template <bool BF16>
__global__ void __launch_bounds__(256)
quant_pertensor_kernel(const uint16_t* x, int64_t n, uint8_t* q, float* scale,
                       const float* amax) {
  float s = amax[0] / 448.0f;
  if (s == 0.0f) s = 1.0f;
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    float v = half_f32(x[i], BF16) / s;
    v = v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
    q[i] = f32_e4m3(v);
  }
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
  if (x_dtype == C4Q_BF16)
    hipLaunchKernelGGL(quant_rowwise_kernel<true>, dim3((unsigned)M), dim3(256), 0, s, xs, ldx, q,
                       ldq, scales, K);
  else
    hipLaunchKernelGGL(quant_rowwise_kernel<false>, dim3((unsigned)M), dim3(256), 0, s, xs, ldx, q,
                       ldq, scales, K);
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
  if (rotate)
    hipLaunchKernelGGL(merge_rot_quant_kernel<true>, dim3((unsigned)M), dim3(256), lds, s, x, H, S,
                       D, q, scales);
  else
    hipLaunchKernelGGL(merge_rot_quant_kernel<false>, dim3((unsigned)M), dim3(256), lds, s, x, H, S,
                       D, q, scales);
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
  const int g = grid_for(n);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(1), 0, s, amax_ws);
  if (x_dtype == C4Q_BF16) {
    hipLaunchKernelGGL(absmax_kernel<true>, dim3(g), dim3(256), 0, s, xs, n, amax_ws);
    hipLaunchKernelGGL(quant_pertensor_kernel<true>, dim3(g), dim3(256), 0, s, xs, n, q, scale,
                       amax_ws);
  } else {
    hipLaunchKernelGGL(absmax_kernel<false>, dim3(g), dim3(256), 0, s, xs, n, amax_ws);
    hipLaunchKernelGGL(quant_pertensor_kernel<false>, dim3(g), dim3(256), 0, s, xs, n, q, scale,
                       amax_ws);
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
