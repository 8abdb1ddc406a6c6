// Shared helpers of the aq HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/aq.h"

namespace aq {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// fp32 -> fp16 bits, round to nearest even (the reference's fp32->fp16 cast).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Sum_j nib_j * x[j] over the eight stored nibbles of a Q4W word XOR 0x88888888 (each nibble then holds q + 8 in
// 0..15, where q = ((nib ^ 8) - 8) is the signed value). Callers subtract 8 * sum(x) to get Sum_j q_j x_j. The
// byte-wise masks let the compiler use v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float dot8_biased(uint32_t word, const float* x) {
  const uint32_t u = word ^ 0x88888888u;
  const uint32_t lo = u & 0x0F0F0F0Fu;          // elements 0, 2, 4, 6
  const uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;   // elements 1, 3, 5, 7
  float d = (float)(lo & 0xFFu) * x[0];
  d = fmaf((float)(hi & 0xFFu), x[1], d);
  d = fmaf((float)((lo >> 8) & 0xFFu), x[2], d);
  d = fmaf((float)((hi >> 8) & 0xFFu), x[3], d);
  d = fmaf((float)((lo >> 16) & 0xFFu), x[4], d);
  d = fmaf((float)((hi >> 16) & 0xFFu), x[5], d);
  d = fmaf((float)(lo >> 24), x[6], d);
  d = fmaf((float)(hi >> 24), x[7], d);
  return d;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AQ_OK : AQ_ERR_LAUNCH;
}

}  // namespace aq
