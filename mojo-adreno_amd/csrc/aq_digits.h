// Signed 4-bit digit form of fp32 activations and its int4 inner product (gfx950), shared by the matrix-vector
// kernels whose weights have one fp16 scale per 32-weight chunk (power-of-two groups >= 32).
#pragma once
#include "aq_common.h"

namespace aq {

// x staging for products with one scale per 32-weight chunk, for word j (x[32c + 8j .. + 7]) of chunk c of token t,
// a = its first four values, b = the last four. Each chunk of 32 values becomes fixed point against its own power of
// two: X = rint(x 2^sh) with the largest |X| in [2^21, 2^22], written in six signed base-16 digits, X = sum over
// d < 6 of 16^d D_d, D_d in [-8, 7] (4-bit two's complement, the Q4W code's own format). LDS layout (lane c of the
// chunk loop reads consecutive 16-byte slots of a plane: conflict-free):
//   xd[t][d][c]   uint4: digit d of the chunk's words 0..3 (nibble i of word j = digit d of x[32c + 8j + i])
//   xf[t][c]      float: 2^-sh (NaN when the chunk holds a non-finite x, so the products become NaN)
// The digits come from the float bits of fma(x, 2^sh, 1.5 * 2^23), which are 0x4B400000 + X for |X| <= 2^22: adding
// 0x888888 (8 to every digit position, keeping each in 0..15) and XORing it back leaves D_d's 4-bit pattern in nibble
// d. The 4 threads of an aligned quad hold the 4 words of one chunk (they exchange exponents by DPP), so whole quads
// must call it together.
__device__ __forceinline__ uint32_t gather_byte(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3, uint32_t b) {
  // byte b of p0, p1, p2, p3 as bytes 0, 1, 2, 3 (v_perm_b32: selector 0x0C gives a zero byte)
  const uint32_t lo = __builtin_amdgcn_perm(p1, p0, 0x0C0C0000u | ((4u + b) << 8) | b);
  const uint32_t hi = __builtin_amdgcn_perm(p3, p2, (b << 16) | ((4u + b) << 24) | 0x0C0Cu);
  return lo | hi;
}

__device__ __forceinline__ void stage_digits(int t, int c, int j, float4 a, float4 b, uint4* __restrict__ xd,
                                             float* __restrict__ xf, int nch) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t e = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) e = max(e, (__float_as_uint(v[q]) >> 23) & 0xFFu);
  e = max(e, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)e, 0xB1, 0xF, 0xF, false));
  e = max(e, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)e, 0x4E, 0xF, 0xF, false));
  // e = the biased exponent of the chunk's largest |x|, which is below 2^(e - 126): 2^(148 - e) brings it below
  // 2^22. sh stays within [-126, 126] so that 2^sh and 2^-sh are normal floats (chunks below 2^-104 keep fewer bits).
  const int sh = e ? min(max(148 - (int)e, -126), 126) : 0;
  const float p2 = __uint_as_float((uint32_t)(sh + 127) << 23);
  uint32_t z[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) z[q] = (__float_as_uint(fmaf(v[q], p2, 12582912.0f)) - 0x4AB77778u) ^ 0x00888888u;
  uint4* dst = xd + (size_t)t * 6 * nch + c;
#pragma unroll
  for (int bb = 0; bb < 3; ++bb) {
    const uint32_t ev = gather_byte(z[0], z[2], z[4], z[6], bb);  // elements 0, 2, 4, 6: digits 2bb, 2bb + 1
    const uint32_t od = gather_byte(z[1], z[3], z[5], z[7], bb);  // elements 1, 3, 5, 7
    const uint32_t d0 = (ev & 0x0F0F0F0Fu) | ((od << 4) & 0xF0F0F0F0u);
    const uint32_t d1 = ((ev >> 4) & 0x0F0F0F0Fu) | (od & 0xF0F0F0F0u);
    reinterpret_cast<uint32_t*>(dst + (2 * bb) * nch)[j] = d0;
    reinterpret_cast<uint32_t*>(dst + (2 * bb + 1) * nch)[j] = d1;
  }
  if (j == 0) xf[t * nch + c] = e == 0xFFu ? __uint_as_float(0x7FC00000u) : __uint_as_float((uint32_t)(127 - sh) << 23);
}

// One 32-weight chunk c of R rows (w: their 16 bytes, sc: their fp16 scale bits) against T tokens staged by
// stage_digits: acc[r][t] += scale_r * sum over the chunk of q * x. The Q4W words are used as they are: one
// v_dot8_i32_i4 (8 products of signed 4-bit values, exact int32 sum) per word and digit, six digits combined as
// I = sum of 16^d P_d (|I| < 2^30), then acc += I * scale * 2^-sh. About 32 VALU operations a chunk, row and token.
template <int R, int T>
__device__ __forceinline__ void chunk_dot(const uint4* __restrict__ xd, const float* __restrict__ xf, int nch, int c,
                                          const uint4 (&w)[R], const uint16_t (&sc)[R], float (&acc)[R][T]) {
  float s[R];
#pragma unroll
  for (int r = 0; r < R; ++r) s[r] = half_bits_to_float(sc[r]);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint4 d[6];
#pragma unroll
    for (int dd = 0; dd < 6; ++dd) d[dd] = xd[(t * 6 + dd) * nch + c];
    const float f = xf[t * nch + c];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int pd[6];
#pragma unroll
      for (int dd = 0; dd < 6; ++dd) {
        int q = __builtin_amdgcn_sdot8((int)w[r].x, (int)d[dd].x, 0, false);
        q = __builtin_amdgcn_sdot8((int)w[r].y, (int)d[dd].y, q, false);
        q = __builtin_amdgcn_sdot8((int)w[r].z, (int)d[dd].z, q, false);
        pd[dd] = __builtin_amdgcn_sdot8((int)w[r].w, (int)d[dd].w, q, false);
      }
      uint32_t I = (uint32_t)pd[5];
#pragma unroll
      for (int dd = 4; dd >= 0; --dd) I = (I << 4) + (uint32_t)pd[dd];
      acc[r][t] = fmaf((float)(int)I, s[r] * f, acc[r][t]);
    }
  }
}

}  // namespace aq
