// Weight-format converters (host code): the producers of the Q4W and T2W layouts the kernels consume.
//
//   aq_quantize_q4           llama/run.py:56-70 quantize4 (= llama/st2bin.c:44-66 "q4", which first rounds each bf16
//                            weight to fp16): s = fp16(max|w| / 7) per group, q = clamp(rint(w / s), -8, 7).
//   aq_quantize_q4_searched  qwen3moe/convert.c:120-159 "q4" (= gemma4/convert.c:57-81): the scale fp16(m / d) for
//                            the d in 6.5, 6.75, ..., 9 with the least squared error (first minimum), bf16 inputs.
//   aq_gguf_q4_0_to_q4w      lfm2/convert.c:59-71 q4_block: GGUF Q4_0 blocks -> Q4W words (nib ^ 8, de-interleaved)
//                            and the fp16 scales unchanged.
//   aq_gguf_q4_0_to_f16      lfm2/convert.c:73-80 + "h4": (nib - 8) * d in fp32, rounded to fp16.
//   aq_gguf_q6_k_to_q6w      lfm2/convert.c "q6" (:148-155): GGUF Q6_K super-blocks (210 bytes: ql[128], qh[64],
//                            int8 scales[16], fp16 d) -> their first 208 bytes [rows, cols/256, 208] and d apart.
//   aq_gguf_q6_k_to_f16      lfm2/convert.c:82-103 q6_dequant + "h6": (d * sc) * (q - 32) in fp32, rounded to fp16.
//   aq_t2w_scales_from_pairs bonsai/convert.cpp:44-61 emitPacked writes the codes already transposed (T2W words) and
//                            fp32 (scale, bias) pairs [K/128, N, 2]; this keeps the fp16 scales [K/128, N] of a
//                            ternary matrix (bias == -scale, the scale exact in fp16, as it came from fp16).
//   aq_t2w_from_mlx          qwen3/convert.cpp:39-74 addPacked: MLX 2-bit codes [n_i, K/16] and scales/biases
//                            [n_i, K/128] of several projections -> one transposed T2W matrix [K/16, sum n_i] and its
//                            scales [K/128, sum n_i]; every group must be ternary (bias == -scale).
//
// The arithmetic is float32 step by step in the reference's order, with no contraction (this file is compiled with
// -ffp-contract=off), and rintf rounds ties to even, so the outputs are the reference's bytes.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/aq.h"

namespace {

float bf16_to_float(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: man * 2^-24, exact in float
      float f = (float)man * 5.9604644775390625e-8f;
      std::memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (exp == 31) {
    u = sign | 0x7F800000u | (man << 13);
  } else {
    u = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// float -> fp16, round to nearest even (the C (__fp16) conversion), with overflow to infinity.
uint16_t float_to_half(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t abs = u & 0x7FFFFFFFu;
  if (abs >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));  // inf / nan
  if (abs >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520: infinity
  if (abs < 0x38800000u) {  // below 2^-14: subnormal (or zero) in fp16, spacing 2^-24
    if (abs < 0x33000000u) return sign;  // < 2^-25: rounds to zero (2^-25 itself ties to even zero)
    const uint32_t e = abs >> 23;
    const uint32_t m = (abs & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - (int)e;  // value = m * 2^(e - 150); in units of 2^-24: m >> (126 - e)
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t r = abs + 0xFFFu + ((abs >> 13) & 1u);  // round the low 13 bits to even
  r -= 0x38000000u;                                // rebias 127 -> 15
  return (uint16_t)(sign | (r >> 13));
}

int clamp_q(float v) { return v < -8.0f ? -8 : v > 7.0f ? 7 : (int)v; }

bool bad_shape(int64_t rows, int64_t cols, int64_t group) {
  return rows <= 0 || cols <= 0 || group <= 0 || group % 8 || cols % group;
}

}  // namespace

extern "C" int aq_quantize_q4(const uint16_t* w, int32_t w_is_bf16, int64_t rows, int64_t cols, int32_t group,
                              uint32_t* wq, uint16_t* ws) {
  if (!w || !wq || !ws) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 8) return AQ_ERR_SHAPE;
  if (group <= 0 || group % 8 || cols % group || group > 4096) return AQ_ERR_GROUP;
  float v[4096];
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* src = w + r * cols;
    uint32_t* dst = wq + r * (cols / 8);
    std::memset(dst, 0, (size_t)(cols / 8) * 4);
    for (int64_t g = 0; g < cols / group; ++g) {
      float maxabs = 0.0f;
      for (int j = 0; j < group; ++j) {
        const uint16_t b = src[g * group + j];
        v[j] = w_is_bf16 ? half_to_float(float_to_half(bf16_to_float(b))) : half_to_float(b);
        maxabs = std::fmax(maxabs, std::fabs(v[j]));
      }
      const uint16_t s16 = float_to_half(maxabs / 7.0f);
      const float sf = half_to_float(s16);
      ws[r * (cols / group) + g] = s16;
      for (int j = 0; j < group; ++j) {
        const float q = sf > 0 ? std::rint(v[j] / sf) : 0.0f;
        const int64_t k = g * group + j;
        dst[k / 8] |= (uint32_t)(clamp_q(q) & 15) << (4 * (k % 8));
      }
    }
  }
  return AQ_OK;
}

extern "C" int aq_quantize_q4_searched(const uint16_t* w_bf16, int64_t rows, int64_t cols, int32_t group,
                                       uint32_t* wq, uint16_t* ws) {
  if (!w_bf16 || !wq || !ws) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0) return AQ_ERR_SHAPE;
  if (bad_shape(rows, cols, group) || group > 256) return AQ_ERR_GROUP;
  const int64_t ng = rows * cols / group;
  for (int64_t g = 0; g < ng; ++g) {
    float w[256], m = 0.0f;
    for (int j = 0; j < group; ++j) {
      w[j] = bf16_to_float(w_bf16[g * group + j]);
      m = std::fmax(m, std::fabs(w[j]));
    }
    float best = INFINITY, sf = 0.0f;
    for (float d = 6.5f; d <= 9.0f; d += 0.25f) {  // the scale with the least squared error, first minimum wins
      const float t = half_to_float(float_to_half(m / d));
      if (!(t > 0)) break;
      float e = 0.0f;
      for (int j = 0; j < group; ++j) {
        const float q = std::fmin(std::fmax(std::rint(w[j] / t), -8.0f), 7.0f);
        const float r = w[j] - q * t;
        e += r * r;
      }
      if (e < best) best = e, sf = t;
    }
    ws[g] = float_to_half(sf);
    for (int k = 0; k < group / 8; ++k) {
      uint32_t word = 0;
      for (int j = 0; j < 8; ++j) {
        const float q = sf > 0 ? std::fmin(std::fmax(std::rint(w[k * 8 + j] / sf), -8.0f), 7.0f) : 0.0f;
        word |= (uint32_t)((int)q & 15) << (4 * j);
      }
      wq[g * group / 8 + k] = word;
    }
  }
  return AQ_OK;
}

extern "C" int aq_gguf_q4_0_to_q4w(const uint8_t* blocks, int64_t rows, int64_t cols, uint32_t* wq, uint16_t* ws) {
  if (!blocks || !wq || !ws) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 32) return AQ_ERR_SHAPE;
  const int64_t nb = rows * cols / 32;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = blocks + b * 18;
    std::memcpy(ws + b, blk, 2);
    const uint8_t* qs = blk + 2;
    for (int w = 0; w < 4; ++w) {
      uint32_t word = 0;
      for (int k = 0; k < 8; ++k) {
        const int e = 8 * w + k;
        const int nib = e < 16 ? (qs[e] & 15) : (qs[e - 16] >> 4);
        word |= (uint32_t)(nib ^ 8) << (4 * k);
      }
      wq[b * 4 + w] = word;
    }
  }
  return AQ_OK;
}

extern "C" int aq_gguf_q4_0_to_f16(const uint8_t* blocks, int64_t rows, int64_t cols, uint16_t* out) {
  if (!blocks || !out) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 32) return AQ_ERR_SHAPE;
  const int64_t nb = rows * cols / 32;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = blocks + b * 18;
    uint16_t dh;
    std::memcpy(&dh, blk, 2);
    const float d = half_to_float(dh);
    const uint8_t* qs = blk + 2;
    for (int j = 0; j < 16; ++j) {
      out[b * 32 + j] = float_to_half((float)((qs[j] & 15) - 8) * d);
      out[b * 32 + j + 16] = float_to_half((float)((qs[j] >> 4) - 8) * d);
    }
  }
  return AQ_OK;
}

extern "C" int aq_gguf_q6_k_to_q6w(const uint8_t* blocks, int64_t rows, int64_t cols, uint8_t* q, uint16_t* d) {
  if (!blocks || !q || !d) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 256) return AQ_ERR_SHAPE;
  const int64_t nb = rows * cols / 256;
  for (int64_t b = 0; b < nb; ++b) {
    std::memcpy(q + b * 208, blocks + b * 210, 208);
    std::memcpy(d + b, blocks + b * 210 + 208, 2);
  }
  return AQ_OK;
}

extern "C" int aq_gguf_q6_k_to_f16(const uint8_t* blocks, int64_t rows, int64_t cols, uint16_t* out) {
  if (!blocks || !out) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 256) return AQ_ERR_SHAPE;
  const int64_t nb = rows * cols / 256;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = blocks + b * 210;
    uint16_t dh;
    std::memcpy(&dh, blk + 208, 2);
    const float dd = half_to_float(dh);
    uint16_t* y = out + b * 256;
    // element 128 h + 32 j + l (j = 0..3, l = 0..31) of the super-block: the low (j = 0, 1) or high (j = 2, 3)
    // nibble of ql[64 h + 32 (j & 1) + l], bits 2 j, 2 j + 1 of qh[32 h + l] above it; scale sc[8 h + 2 j + l / 16]
    for (int h = 0; h < 2; ++h)
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
          const uint8_t lo = blk[64 * h + 32 * (j & 1) + l];
          const uint8_t hi = blk[128 + 32 * h + l];
          const int qv = (int)(((j < 2 ? lo : lo >> 4) & 15) | (((hi >> (2 * j)) & 3) << 4)) - 32;
          const int8_t sc = (int8_t)blk[192 + 8 * h + 2 * j + l / 16];
          y[128 * h + 32 * j + l] = float_to_half(dd * (float)sc * (float)qv);
        }
  }
  return AQ_OK;
}

extern "C" int aq_t2w_scales_from_pairs(const float* params, int64_t groups, int64_t n, uint16_t* s) {
  if (!params || !s) return AQ_ERR_NULL;
  if (groups <= 0 || n <= 0) return AQ_ERR_SHAPE;
  const int64_t count = groups * n;
  for (int64_t i = 0; i < count; ++i) {  // check everything first: nothing is written on an error
    const float sc = params[2 * i], b = params[2 * i + 1];
    if (b != -sc || half_to_float(float_to_half(sc)) != sc) return AQ_ERR_ARG;
  }
  for (int64_t i = 0; i < count; ++i) s[i] = float_to_half(params[2 * i]);
  return AQ_OK;
}

extern "C" int aq_t2w_from_mlx(const uint32_t* const* codes, const uint16_t* const* scales,
                               const uint16_t* const* biases, const int64_t* rows, int32_t parts, int64_t k,
                               uint32_t* w, uint16_t* s) {
  if (!codes || !scales || !biases || !rows || !w || !s) return AQ_ERR_NULL;
  if (parts <= 0 || k <= 0 || k % 128) return AQ_ERR_SHAPE;
  int64_t total = 0;
  for (int32_t p = 0; p < parts; ++p) {
    if (!codes[p] || !scales[p] || !biases[p]) return AQ_ERR_NULL;
    if (rows[p] <= 0) return AQ_ERR_SHAPE;
    for (int64_t i = 0; i < rows[p] * (k / 128); ++i)
      if (half_to_float(biases[p][i]) != -half_to_float(scales[p][i])) return AQ_ERR_ARG;  // not ternary
    total += rows[p];
  }
  int64_t col = 0;
  for (int32_t p = 0; p < parts; ++p) {
    for (int64_t r = 0; r < rows[p]; ++r) {
      for (int64_t c = 0; c < k / 16; ++c) w[c * total + col + r] = codes[p][r * (k / 16) + c];
      for (int64_t c = 0; c < k / 128; ++c) s[c * total + col + r] = scales[p][r * (k / 128) + c];
    }
    col += rows[p];
  }
  return AQ_OK;
}
