// Test-only probes: gfx950 conversion instructions, checked exhaustively
// against the library's integer-only reference roundings (numerics.hpp), and
// the host-side tile planning of the GEMM launches (launch.hpp).
// Built into tests/native/libc4q_probe.so; used by tests/test_gpu_numerics.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.hpp"
#include "numerics.hpp"

using namespace c4q;

// Every float bit pattern u in [0, 2^32): compare the hardware conversion
// with the reference rounding; NaN inputs are skipped (both give a NaN).
__global__ void __launch_bounds__(256) cvt_bf16_all(unsigned long long* bad, uint32_t* first) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  unsigned long long n = 0;
  for (uint64_t k = 0; k < 256; ++k) {
    const uint32_t u = (uint32_t)(t * 256 + k);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) continue;
    const float f = bits_f32(u);
    const uint16_t hw = __builtin_bit_cast(uint16_t, (__bf16)f);
    if (hw != bf16_rte(f)) {
      if (n == 0) atomicMin(first, u);
      ++n;
    }
  }
  if (n) atomicAdd(bad, n);
}

__global__ void __launch_bounds__(256) cvt_f16_all(unsigned long long* bad, uint32_t* first) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  unsigned long long n = 0;
  for (uint64_t k = 0; k < 256; ++k) {
    const uint32_t u = (uint32_t)(t * 256 + k);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) continue;
    const float f = bits_f32(u);
    const uint16_t hw = __builtin_bit_cast(uint16_t, (_Float16)f);
    if (hw != f16_rte(f)) {
      if (n == 0) atomicMin(first, u);
      ++n;
    }
  }
  if (n) atomicAdd(bad, n);
}

// which: 0 = bf16, 1 = f16. out: device [2] u64 (mismatch count, first
// mismatching bit pattern). Returns a hipError_t value.
extern "C" int c4q_probe_cvt_exhaustive(int which, unsigned long long* out, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* first = reinterpret_cast<uint32_t*>(out + 1);
  const dim3 grid(65536), block(256);   // 65536 * 256 * 256 = 2^32 patterns
  if (which == 0) hipLaunchKernelGGL(cvt_bf16_all, grid, block, 0, s, out, first);
  else hipLaunchKernelGGL(cvt_f16_all, grid, block, 0, s, out, first);
  return (int)hipGetLastError();
}

// Every non-NaN bf16 x and every positive normal bf16 s with |x/s| < 2^64:
// bf16 rounding of div_bf16_operands(x, s, RN(1/s)) against bf16 rounding of
// the IEEE quotient. Thread t: x = t >> 8, s = 0x0080 + 128 (t & 255) + k.
__global__ void __launch_bounds__(256) div_bf16_all(unsigned long long* bad, uint32_t* first) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const uint32_t xb = t >> 8;
  if ((xb & 0x7FFFu) > 0x7F80u) return;                     // NaN x
  const float x = bf16_f32((uint16_t)xb);
  unsigned long long n = 0;
  for (uint32_t k = 0; k < 128; ++k) {
    const uint32_t sb = 0x0080u + 128u * (t & 255u) + k;
    if (sb > 0x7F7Fu) break;                                 // positive normal bf16 only
    const float s = bf16_f32((uint16_t)sb);
    const float exact = x / s;
    if (!(fabsf(exact) < 1.8446744073709552e19f)) continue;  // |x/s| >= 2^64
    const float r = 1.0f / s;
    if (bf16_rte(div_bf16_operands(x, s, r)) != bf16_rte(exact)) {
      if (n == 0) atomicMin(first, (xb << 16) | sb);
      ++n;
    }
  }
  if (n) atomicAdd(bad, n);
}

// out: device [2] u64 (mismatch count, first mismatching pair x << 16 | s).
extern "C" int c4q_probe_div_bf16_exhaustive(unsigned long long* out, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* first = reinterpret_cast<uint32_t*>(out + 1);
  hipLaunchKernelGGL(div_bf16_all, dim3(65536), dim3(256), 0, s, out, first);
  return (int)hipGetLastError();
}

// e4m3_pair against f32_e4m3(clamp448(.)) for every float bit pattern u in
// slot 0 and u * 0x9E3779B1 (a bijection of the 2^32 patterns) in slot 1.
__global__ void __launch_bounds__(256) e4m3_pair_all(unsigned long long* bad, uint32_t* first) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  unsigned long long n = 0;
  for (uint64_t k = 0; k < 256; ++k) {
    const uint32_t u = (uint32_t)(t * 256 + k), v = u * 0x9E3779B1u;
    const float a = bits_f32(u), b = bits_f32(v);
    const uint32_t hw = e4m3_pair(a, b);
    const uint32_t ref = (uint32_t)f32_e4m3(clamp448(a)) | ((uint32_t)f32_e4m3(clamp448(b)) << 8);
    if (hw != ref) {
      if (n == 0) atomicMin(first, u);
      ++n;
    }
  }
  if (n) atomicAdd(bad, n);
}

// The per-tensor fp8 quantizer's quotient: for every non-NaN 16-bit x and
// every positive finite 16-bit amax with s = RN(amax / 448) on the
// reciprocal path (rcp_quot_ok), the e4m3 code of div_bf16_operands(x, s,
// RN(1/s)) against the code of the IEEE quotient x / s (both clamped).
// Thread t: x = t >> 8, amax = 1 + 128 (t & 255) + k. which: 0 bf16, 1 f16.
template <bool BF16>
__global__ void __launch_bounds__(256) quot_e4m3_all(unsigned long long* bad, uint32_t* first) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const uint32_t xb = t >> 8;
  const uint32_t inf = BF16 ? 0x7F80u : 0x7C00u;
  if ((xb & 0x7FFFu) > inf) return;                          // NaN x
  const float x = BF16 ? bf16_f32((uint16_t)xb) : __builtin_bit_cast(_Float16, (uint16_t)xb);
  unsigned long long n = 0;
  for (uint32_t k = 0; k < 128; ++k) {
    const uint32_t ab = 1u + 128u * (t & 255u) + k;
    if (ab >= inf) break;                                    // positive finite amax only
    const float amax = BF16 ? bf16_f32((uint16_t)ab) : (float)__builtin_bit_cast(_Float16, (uint16_t)ab);
    if (fabsf(x) > amax) continue;                           // |x| <= amax in any real tensor
    const float s = amax / 448.0f;
    if (!rcp_quot_ok(s)) continue;
    const float fast = div_bf16_operands(x, s, 1.0f / s);
    if ((e4m3_pair(fast, 0.0f) & 0xFFu) != f32_e4m3(clamp448(x / s))) {
      if (n == 0) atomicMin(first, (xb << 16) | ab);
      ++n;
    }
  }
  if (n) atomicAdd(bad, n);
}

// which: 0 = e4m3_pair over all patterns, 1 = bf16 quotients, 2 = f16
// quotients. out: device [2] u64 (mismatch count, first mismatch).
extern "C" int c4q_probe_e4m3_exhaustive(int which, unsigned long long* out, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* first = reinterpret_cast<uint32_t*>(out + 1);
  if (which == 0) hipLaunchKernelGGL(e4m3_pair_all, dim3(65536), dim3(256), 0, s, out, first);
  else if (which == 1) hipLaunchKernelGGL(quot_e4m3_all<true>, dim3(65536), dim3(256), 0, s, out, first);
  else hipLaunchKernelGGL(quot_e4m3_all<false>, dim3(65536), dim3(256), 0, s, out, first);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------- tile plans ---
// Host-side enumeration of the launches a GEMM's tile plan issues
// (plan_launches, tile_at -- the functions the library runs). cover
// [cdiv(M, CM) * cdiv(n_rows_b, 64)] counts, per CM x 64 output cell
// inside the matrix, the kernel tiles that compute it (every tile size is a
// multiple of the cell). info[8]: launches, then (tile id, kernel tiles) of
// each launch, then the main launch's first and the tail launch's sub_m,
// sub_n. Returns 0, or -1 if cover_len is too small.
template <class Set, int CM = 64>
static int probe_plan(int64_t M, int64_t n_rows_b, int64_t K, int cus, int32_t* cover,
                      int64_t cover_len, int64_t* info) {
  const int64_t cm = cdiv(M, CM), cn = cdiv(n_rows_b, 64);
  if (cm * cn > cover_len) return -1;
  for (int64_t i = 0; i < cm * cn; ++i) cover[i] = 0;
  int ids[2];
  GemmShape shs[2];
  const int n = plan_launches<Set>(M, n_rows_b, n_rows_b, K, cus, ids, shs);
  for (int k = 0; k < 8; ++k) info[k] = 0;
  info[0] = n;
  for (int l = 0; l < n; ++l) {
    const int bm = Set::bm(ids[l]), bn = Set::bn(ids[l]);
    info[1 + 2 * l] = ids[l];
    info[2 + 2 * l] = shs[l].count;
    if (l == 1) {
      info[6] = shs[l].sub_m;
      info[7] = shs[l].sub_n;
    }
    for (int i = 0; i < shs[l].count; ++i) {
      const TileCoord t = tile_at(shs[l], i);
      for (int64_t r = (int64_t)t.tm * bm; r < (int64_t)(t.tm + 1) * bm; r += CM)
        for (int64_t c = (int64_t)t.tn * bn; c < (int64_t)(t.tn + 1) * bn; c += 64)
          if (r < M && c < n_rows_b) ++cover[(r / CM) * cn + c / 64];
    }
  }
  info[5] = n ? shs[0].first : 0;
  return 0;
}

extern "C" int c4q_probe_tile_plan(int64_t M, int64_t n_rows_b, int64_t K, int cus, int32_t* cover,
                                   int64_t cover_len, int64_t* info) {
  return probe_plan<MainTiles>(M, n_rows_b, K, cus, cover, cover_len, info);
}

// The same for the W8A16 tile set (W8A16Tiles: the general ids plus 8 =
// 224x256 on 1 x 4 waves), over cells of 32 rows x 64 columns: cover has
// cdiv(M, 32) * cdiv(n_rows_b, 64) entries.
extern "C" int c4q_probe_w8a16_tile_plan(int64_t M, int64_t n_rows_b, int64_t K, int cus,
                                         int32_t* cover, int64_t cover_len, int64_t* info) {
  return probe_plan<W8A16Tiles, 32>(M, n_rows_b, K, cus, cover, cover_len, info);
}

// The same for the head-spanning tile set (HeadTiles: ids 0 = 256x256 with
// 4 waves, 1 = 128x128 with 2 waves).
extern "C" int c4q_probe_head_tile_plan(int64_t M, int64_t n_rows_b, int64_t K, int cus,
                                        int32_t* cover, int64_t cover_len, int64_t* info) {
  return probe_plan<HeadTiles>(M, n_rows_b, K, cus, cover, cover_len, info);
}
