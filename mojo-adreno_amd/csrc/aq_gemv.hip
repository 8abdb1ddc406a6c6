// int4 (Q4W) matrix-vector products for decode and few-token batches, gfx950, including the MoE decode experts.
//
// The arithmetic is the reference's gemv_q4 family (llama/kernels/gemv_q4.mojo:13-30, gemv_add_q4.mojo:13-30,
// lfm2/kernels/lk.mojo:38-72,134-167, qwen3moe/kernels/moek.mojo:30-45,200-223,273-281,496-545): per row n,
//   y[n] = sum over groups of fp16 scale * sum_k ((nib ^ 8) - 8) * x[k], accumulated in fp32.
//
// Design (HBM-bound, ~0.5625 B per weight): a 256-thread workgroup stages x (fp32, all tokens) and per-word sums of
// x in LDS once, then each wave streams R weight rows at a time: every lane takes whole 16-byte, 32-weight chunks of
// the rows (chunk c = lane, lane + 64, ...), so a wave's loads of one row are 1 KB contiguous, and applies each
// decoded word to all T tokens. A word is decoded as q + 8 (XOR 0x88888888, byte masks -> v_cvt_f32_ubyte), and
// 8 * sum(x) is subtracted once per chunk: two VALU ops per weight. Row sums end in a wave reduction.
#include "aq_common.h"

namespace aq {

enum { kStore = 0, kAdd = 1, kGateUp = 2, kMoeGateUp = 3, kMoeDown = 4 };

// MoE decode: kMoeGateUp outputs o = e * f + j use gate|up rows ids[e] * 2f + j (+ f); kMoeDown output o sums, over
// expert slots t < tokens (in slot order), rw[t] * (row ids[t] * n_out + o) . x[t]. An id outside [0, experts) selects
// no row (its contribution is zero).
struct MoeArgs {
  const int32_t* ids;
  const float* rw;
  int experts;
  int add;
};

// G32: the group size is a multiple of 32 (one scale per 32-weight chunk). Otherwise every word looks up its own.
template <bool G32, int R, int T, int MODE>
__global__ __launch_bounds__(256) void k_gemv_q4(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                 const float* __restrict__ x, float* __restrict__ y, int n_out,
                                                 int k, int group, int f, int tokens, MoeArgs moe) {
  // LDS layout, conflict-free for the chunk loop (lane c reads consecutive 16-byte slots):
  //   xs4[t][p][c]  float4 p = 2j + h holds x[t, 32c + 8j + 4h .. + 3]  (T * 8 planes of nch float4)
  //   xsum[t][j][c] sum of x[t, 32c + 8j .. + 7]                        (T * 4 planes of nch floats)
  extern __shared__ float4 lds4[];
  const int kw = k >> 3;
  const int nch = k >> 5;
  float4* xs4 = lds4;
  float* xsum = reinterpret_cast<float*>(lds4 + T * 8 * nch);
  for (int i = threadIdx.x; i < T * kw; i += 256) {
    const int t = i / kw;
    const int wi = i - t * kw;
    const int c = wi >> 2;
    const int j = wi & 3;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (t < tokens) {
      const float4* src = reinterpret_cast<const float4*>(x + (size_t)t * k + wi * 8);
      a = src[0];
      b = src[1];
    }
    xs4[(t * 8 + 2 * j) * nch + c] = a;
    xs4[(t * 8 + 2 * j + 1) * nch + c] = b;
    xsum[(t * 4 + j) * nch + c] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int gpr = k / group;
  constexpr int RO = (MODE == kGateUp || MODE == kMoeGateUp) ? R / 2 : R;
  constexpr int SL = MODE == kMoeDown ? T : 1;  // weight rows per output (kMoeDown: one per expert slot)

  for (int base = (blockIdx.x * 4 + wave) * RO; base < n_out; base += gridDim.x * 4 * RO) {
    int rows[R][SL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int o = base + (r % RO);
      o = o < n_out ? o : n_out - 1;  // rows past the end repeat the last one; their sums are not written
#pragma unroll
      for (int sl = 0; sl < SL; ++sl) {
        if constexpr (MODE == kMoeGateUp) {
          const int e = o / f, j = o - e * f;
          const int ex = moe.ids[e];
          rows[r][sl] = (ex >= 0 && ex < moe.experts) ? ex * 2 * f + j + (r >= RO ? f : 0) : -1;
        } else if constexpr (MODE == kMoeDown) {
          const int ex = sl < tokens ? moe.ids[sl] : -1;
          rows[r][sl] = (ex >= 0 && ex < moe.experts) ? ex * n_out + o : -1;
        } else {
          rows[r][sl] = (MODE == kGateUp && r >= RO) ? f + o : o;
        }
      }
    }
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = 0.f;

    for (int c = lane; c < nch; c += kWave) {
      if constexpr (MODE == kMoeDown) {
        // one row per expert slot t, applied to that slot's activations only
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const int row = rows[0][t];
          if (row < 0) continue;  // wave-uniform
          const uint4 w4 = *reinterpret_cast<const uint4*>(wq + (size_t)row * kw + c * 4);
          const uint32_t wv4[4] = {w4.x, w4.y, w4.z, w4.w};
          float part = 0.f;
          if constexpr (G32) {
            const float* s4 = xsum + t * 4 * nch + c;
            part = -8.0f * ((s4[0] + s4[nch]) + (s4[2 * nch] + s4[3 * nch]));
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float xv[8];
            *reinterpret_cast<float4*>(xv) = xs4[(t * 8 + 2 * j) * nch + c];
            *reinterpret_cast<float4*>(xv + 4) = xs4[(t * 8 + 2 * j + 1) * nch + c];
            if constexpr (G32) {
              part += dot8_biased(wv4[j], xv);
            } else {
              const float sj = half_bits_to_float(ws[(size_t)row * gpr + (c * 32 + 8 * j) / group]);
              part = fmaf(dot8_biased(wv4[j], xv) - 8.0f * xsum[(t * 4 + j) * nch + c], sj, part);
            }
          }
          if constexpr (G32) part *= half_bits_to_float(ws[(size_t)row * gpr + (c * 32) / group]);
          acc[0][t] += part;
        }
        continue;
      }
      // only kMoeGateUp can name no row (an invalid expert id): its weights read as zero codes with scale 0
      uint4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (MODE != kMoeGateUp || rows[r][0] >= 0)
          wv[r] = *reinterpret_cast<const uint4*>(wq + (size_t)rows[r][0] * kw + c * 4);
        else
          wv[r] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
      }
      if constexpr (G32) {
        const int gi = (c * 32) / group;
        float sc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
          sc[r] = (MODE != kMoeGateUp || rows[r][0] >= 0) ? half_bits_to_float(ws[(size_t)rows[r][0] * gpr + gi])
                                                           : 0.f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float* sc4 = xsum + t * 4 * nch + c;
          const float xs32 = (sc4[0] + sc4[nch]) + (sc4[2 * nch] + sc4[3 * nch]);
          float part[R];
#pragma unroll
          for (int r = 0; r < R; ++r) part[r] = -8.0f * xs32;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float xv[8];
            *reinterpret_cast<float4*>(xv) = xs4[(t * 8 + 2 * j) * nch + c];
            *reinterpret_cast<float4*>(xv + 4) = xs4[(t * 8 + 2 * j + 1) * nch + c];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const uint32_t w = j == 0 ? wv[r].x : j == 1 ? wv[r].y : j == 2 ? wv[r].z : wv[r].w;
              part[r] += dot8_biased(w, xv);
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][t] = fmaf(part[r], sc[r], acc[r][t]);
        }
      } else {
        float sc[R][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int gi = (c * 32 + 8 * j) / group;
#pragma unroll
          for (int r = 0; r < R; ++r)
            sc[r][j] = (MODE != kMoeGateUp || rows[r][0] >= 0)
                           ? half_bits_to_float(ws[(size_t)rows[r][0] * gpr + gi]) : 0.f;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float xv[8];
            *reinterpret_cast<float4*>(xv) = xs4[(t * 8 + 2 * j) * nch + c];
            *reinterpret_cast<float4*>(xv + 4) = xs4[(t * 8 + 2 * j + 1) * nch + c];
            const float xs8 = xsum[(t * 4 + j) * nch + c];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const uint32_t w = j == 0 ? wv[r].x : j == 1 ? wv[r].y : j == 2 ? wv[r].z : wv[r].w;
              acc[r][t] = fmaf(dot8_biased(w, xv) - 8.0f * xs8, sc[r][j], acc[r][t]);
            }
          }
        }
      }
    }

    if constexpr (MODE == kMoeDown) {
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (t < tokens) sum = fmaf(moe.rw[t], wave_sum(acc[0][t]), sum);
      if (lane == 0) y[base] = moe.add ? y[base] + sum : sum;
      continue;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = wave_sum(acc[r][t]);

    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < RO; ++r) {
        const int o = base + r;
        if (o >= n_out) break;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (t >= tokens) break;
          float* dst = y + (size_t)t * n_out + o;
          if constexpr (MODE == kStore) *dst = acc[r][t];
          else if constexpr (MODE == kAdd) *dst += acc[r][t];
          else *dst = silu(acc[r][t]) * acc[RO + r][t];
        }
      }
    }
  }
}

template <bool G32, int R, int T, int MODE>
static int launch_t(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, hipStream_t s) {
  constexpr int RO = (MODE == kGateUp || MODE == kMoeGateUp) ? R / 2 : R;
  const size_t lds = (size_t)T * k * sizeof(float) + (size_t)T * (k / 8) * sizeof(float);
  auto kern = k_gemv_q4<G32, R, T, MODE>;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return AQ_ERR_CAPACITY;
  }
  int blocks = (n_out + 4 * RO - 1) / (4 * RO);
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, wq, ws, x, y, n_out, k, group, f, tokens, moe);
  return launch_status();
}

// Weight rows per wave iteration. Measured on MI355X (G = 32, K = 2048): R = 2 is fastest while the matrix has fewer
// than 16K rows (N = 5120: 4.5 us vs 5.3 us at R = 4; N = 8192: 5.0 vs 5.5 us; N = 2048, K = 8192: 7.6 vs 9.9 us),
// R = 4 from 16K rows on (N = 16384: 7.3 vs 7.4 us; N = 128256: 35.3 vs 38.1 us). kMoeDown reads one row per expert
// slot for each output instead.
template <bool G32, int T, int MODE>
static int launch_r(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, hipStream_t s) {
  if constexpr (MODE == kMoeDown) {
    return launch_t<G32, 1, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
  } else {
    const int64_t rows = (MODE == kGateUp || MODE == kMoeGateUp) ? 2 * (int64_t)n_out : n_out;
    if (rows < 16384) return launch_t<G32, 2, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
    return launch_t<G32, 4, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
  }
}

template <bool G32, int MODE>
static int launch_g(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, hipStream_t s) {
  if (tokens <= 1) return launch_r<G32, 1, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
  if (tokens <= 2) return launch_r<G32, 2, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
  if (tokens <= 4) return launch_r<G32, 4, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
  return launch_r<G32, 8, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, s);
}

template <int MODE>
static int gemv_entry(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n_out, int64_t k,
                      int32_t group, int64_t f, int32_t tokens, const MoeArgs& moe, void* stream) {
  if (!wq || !ws || !x || !y) return AQ_ERR_NULL;
  if (n_out <= 0 || k <= 0 || tokens < 1 || tokens > 8) return AQ_ERR_SHAPE;
  if (k % 32) return AQ_ERR_SHAPE;
  if (group <= 0 || group % 8 || k % group) return AQ_ERR_GROUP;
  const int tp = tokens <= 1 ? 1 : tokens <= 2 ? 2 : tokens <= 4 ? 4 : 8;
  if ((int64_t)tp * k > 32768) return AQ_ERR_CAPACITY;
  if (n_out > (int64_t)1 << 30) return AQ_ERR_SHAPE;
  if (!aligned(wq, 16) || !aligned(x, 16)) return AQ_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (group % 32 == 0)
    return launch_g<true, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, moe, s);
  return launch_g<false, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, moe, s);
}

}  // namespace aq

extern "C" int aq_gemv_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n, int64_t k,
                          int32_t group, int32_t tokens, int32_t add, void* stream) {
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  if (add) return aq::gemv_entry<aq::kAdd>(wq, ws, x, y, n, k, group, 0, tokens, none, stream);
  return aq::gemv_entry<aq::kStore>(wq, ws, x, y, n, k, group, 0, tokens, none, stream);
}

extern "C" int aq_gate_up_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* a, int64_t f, int64_t k,
                             int32_t group, int32_t tokens, void* stream) {
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  return aq::gemv_entry<aq::kGateUp>(wq, ws, x, a, f, k, group, f, tokens, none, stream);
}

extern "C" int aq_moe_gate_up_q4(const uint32_t* wq, const uint16_t* ws, int64_t experts, const int32_t* ids,
                                 const float* x, float* a, int64_t f, int64_t k, int32_t group, int32_t topk,
                                 void* stream) {
  if (!ids) return AQ_ERR_NULL;
  if (topk <= 0 || f <= 0 || experts <= 0 || topk * f > (1 << 30) || experts * 2 * f > INT32_MAX) return AQ_ERR_SHAPE;
  const aq::MoeArgs moe{ids, nullptr, (int)experts, 0};
  return aq::gemv_entry<aq::kMoeGateUp>(wq, ws, x, a, topk * f, k, group, f, 1, moe, stream);
}

extern "C" int aq_moe_down_q4(const uint32_t* wq, const uint16_t* ws, int64_t experts, const int32_t* ids,
                              const float* weights, const float* act, float* y, int64_t d, int64_t f, int32_t group,
                              int32_t topk, int32_t add, void* stream) {
  if (!ids || !weights) return AQ_ERR_NULL;
  if (topk <= 0 || topk > 8 || d <= 0 || experts <= 0 || experts * d > INT32_MAX) return AQ_ERR_SHAPE;
  // the expert slots are the kernel's "tokens": act [topk, f] holds one activation vector per slot
  const aq::MoeArgs moe{ids, weights, (int)experts, add ? 1 : 0};
  return aq::gemv_entry<aq::kMoeDown>(wq, ws, act, y, d, f, group, 0, topk, moe, stream);
}
