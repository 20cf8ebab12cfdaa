// Test-only probes of gfx950 conversion instructions, checked exhaustively
// against the library's integer-only reference roundings (numerics.hpp).
// Built into tests/native/libc4q_probe.so; used by tests/test_gpu_numerics.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

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
