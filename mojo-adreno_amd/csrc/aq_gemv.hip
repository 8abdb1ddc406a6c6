// int4 (Q4W) matrix-vector products for decode and few-token batches, gfx950.
//
// The arithmetic is the reference's gemv_q4 family (llama/kernels/gemv_q4.mojo:13-30, gemv_add_q4.mojo:13-30,
// lfm2/kernels/lk.mojo:38-72,134-167, qwen3moe/kernels/moek.mojo:30-45,273-281,496-545): per row n,
//   y[n] = sum over groups of fp16 scale * sum_k ((nib ^ 8) - 8) * x[k], accumulated in fp32.
//
// Design (HBM-bound, ~0.5625 B per weight): a 256-thread workgroup stages x (fp32, all tokens) and per-word sums of
// x in LDS once, then each wave streams R weight rows at a time: every lane takes whole 16-byte, 32-weight chunks of
// the rows (chunk c = lane, lane + 64, ...), so a wave's loads of one row are 1 KB contiguous, and applies each
// decoded word to all T tokens. A word is decoded as q + 8 (XOR 0x88888888, byte masks -> v_cvt_f32_ubyte), and
// 8 * sum(x) is subtracted once per chunk: two VALU ops per weight. Row sums end in a wave reduction.
#include "aq_common.h"

namespace aq {

enum { kStore = 0, kAdd = 1, kGateUp = 2 };

// G32: the group size is a multiple of 32 (one scale per 32-weight chunk). Otherwise every word looks up its own.
template <bool G32, int R, int T, int MODE>
__global__ __launch_bounds__(256) void k_gemv_q4(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                 const float* __restrict__ x, float* __restrict__ y, int n_out,
                                                 int k, int group, int f, int tokens) {
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
  constexpr int RO = (MODE == kGateUp) ? R / 2 : R;

  for (int base = (blockIdx.x * 4 + wave) * RO; base < n_out; base += gridDim.x * 4 * RO) {
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int o = base + (r % RO);
      o = o < n_out ? o : n_out - 1;  // rows past the end repeat the last one; their sums are not written
      rows[r] = (MODE == kGateUp && r >= RO) ? f + o : o;
    }
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = 0.f;

    for (int c = lane; c < nch; c += kWave) {
      uint4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        wv[r] = *reinterpret_cast<const uint4*>(wq + (size_t)rows[r] * kw + c * 4);
      if constexpr (G32) {
        const int gi = (c * 32) / group;
        float sc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) sc[r] = half_bits_to_float(ws[(size_t)rows[r] * gpr + gi]);
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
          for (int r = 0; r < R; ++r) sc[r][j] = half_bits_to_float(ws[(size_t)rows[r] * gpr + gi]);
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

template <bool G32, int T, int MODE>
static int launch_t(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, hipStream_t s) {
  constexpr int R = 4;
  constexpr int RO = (MODE == kGateUp) ? R / 2 : R;
  const size_t lds = (size_t)T * k * sizeof(float) + (size_t)T * (k / 8) * sizeof(float);
  auto kern = k_gemv_q4<G32, R, T, MODE>;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return AQ_ERR_CAPACITY;
  }
  int blocks = (n_out + 4 * RO - 1) / (4 * RO);
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, wq, ws, x, y, n_out, k, group, f, tokens);
  return launch_status();
}

template <bool G32, int MODE>
static int launch_g(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, hipStream_t s) {
  if (tokens <= 1) return launch_t<G32, 1, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, s);
  if (tokens <= 2) return launch_t<G32, 2, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, s);
  if (tokens <= 4) return launch_t<G32, 4, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, s);
  return launch_t<G32, 8, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, s);
}

template <int MODE>
static int gemv_entry(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n_out, int64_t k,
                      int32_t group, int64_t f, int32_t tokens, void* stream) {
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
    return launch_g<true, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, s);
  return launch_g<false, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, s);
}

}  // namespace aq

extern "C" int aq_gemv_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n, int64_t k,
                          int32_t group, int32_t tokens, int32_t add, void* stream) {
  if (add) return aq::gemv_entry<aq::kAdd>(wq, ws, x, y, n, k, group, 0, tokens, stream);
  return aq::gemv_entry<aq::kStore>(wq, ws, x, y, n, k, group, 0, tokens, stream);
}

extern "C" int aq_gate_up_q4(const uint32_t* wq, const uint16_t* ws, const float* x, float* a, int64_t f, int64_t k,
                             int32_t group, int32_t tokens, void* stream) {
  return aq::gemv_entry<aq::kGateUp>(wq, ws, x, a, f, k, group, f, tokens, stream);
}
