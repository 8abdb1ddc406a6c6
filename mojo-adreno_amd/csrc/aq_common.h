// Shared helpers of the aq HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/aq.h"

namespace aq {

constexpr int kWave = 64;

// This wave's index within its workgroup as a scalar (wave-uniform) value. The compiler does not infer that
// threadIdx.x / 64 is the same across a wave: loops and branches on the vector value run under exec masks.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Cross-lane moves by DPP (a VALU operand modifier: no LDS round trip). CTRL: quad_perm 0x00-0xFF, row_mirror 0x140,
// row_half_mirror 0x141, row_ror:n 0x120 + n, row_bcast:15 0x142, row_bcast:31 0x143 (rows are 16 lanes).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF,
                                                    false));
}

// Sum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xB1>(0.f, v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp<0x4E>(0.f, v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp<0x141>(0.f, v);  // row_half_mirror: the other quad of the 8
  return v;
}

// Sum / max over the wave, in every lane: within rows by DPP, across the four rows by row_bcast into the last row,
// read back from lane 63.
__device__ __forceinline__ float wave_sum(float v) {
  v = sum8(v);
  v += dpp<0x140>(0.f, v);       // row_mirror: the other 8 of the row
  v += dpp<0x142, 0xA>(0.f, v);  // rows 1, 3 += last lane of rows 0, 2
  v += dpp<0x143, 0xC>(0.f, v);  // rows 2, 3 += lane 31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v, v));
  v = fmaxf(v, dpp<0x4E>(v, v));
  v = fmaxf(v, dpp<0x141>(v, v));
  v = fmaxf(v, dpp<0x140>(v, v));
  v = fmaxf(v, dpp<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp<0x143, 0xC>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
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

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes return zero (no branch needed).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset past any resource used here: the load returns zero

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return __builtin_bit_cast(uint4, v);
}
// The same with a cache policy (for data read once, such as the weights of a decode GEMV).
// kWPolicy: nt (streaming). The matrix-vector kernels read each weight once a launch; bench.py on MI355X, alternating
// libraries: the C4 decode step 486 -> 463 us, C0 4.83 -> 4.73 us, the int4 lm_head 38.3 -> 37.3 us, C2's ternary
// GEMV triple 21.8 -> 21.2 us, the ternary head 35.8 -> 34.1 us (sc1 | nt and sc0 | nt measured the same). Not for
// loads whose pieces share cache lines (the Q6_K head).
constexpr int kWPolicy = 2;
// Device-coherent (sc1) buffer accesses: a store written through to where every XCD reads it, a load that does not
// take a line an XCD's L2 may hold stale. For data one workgroup hands to another within a launch, with a device-scope
// atomic ordering the two (no cache writeback needed).
constexpr int kSc1 = 16;
template <int POL>
__device__ __forceinline__ uint4 buf_load16p(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
  return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ float buf_load_half(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  return half_bits_to_float(h);
}

// Argmax key: larger for a larger value and, among equal values, for a smaller index, so the maximum key names the
// first maximum (the reference's `if logits[i] > logits[best]` scan). 0 is below every key of a finite value.
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)~(uint32_t)idx;
}
// m = max(m, the 64-bit value DPP brings from another lane), both halves moved by the same DPP control
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t m) {
  const uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
  const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, CTRL, ROW_MASK, 0xF, false);
  const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, CTRL, ROW_MASK, 0xF, false);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > m ? o : m;
}
// Maximum of a 64-bit value over the wave, in every lane (the steps of wave_max, read back from lane 63).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t m) {
  m = dpp_max_u64<0xB1, 0xF>(m);
  m = dpp_max_u64<0x4E, 0xF>(m);
  m = dpp_max_u64<0x141, 0xF>(m);
  m = dpp_max_u64<0x140, 0xF>(m);
  m = dpp_max_u64<0x142, 0xA>(m);
  m = dpp_max_u64<0x143, 0xC>(m);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)m, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(m >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// The key a producer leaves when any of its values is not finite: above every key of a finite value, so the step's
// maximum is this key exactly when some logit was NaN or infinite (the token is then -1).
constexpr uint64_t kNonFiniteKey = ~0ull;

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AQ_OK : AQ_ERR_LAUNCH;
}

}  // namespace aq
