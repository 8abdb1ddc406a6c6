// The small kernels of a Llama decode step around the int4 GEMVs, gfx950: the embedding lookup and the attention of
// one new token (RoPE, KV-cache append and softmax-weighted sum in one launch).
//
// Reference: llama/kernels/embed.mojo:9-11, rope_kv.mojo:18-45 and attention.mojo:19-66, launched per layer by
// llama/model.mojo:142-150. Layouts follow the reference's: the fused qkv vector is q (heads x 64) | k (kv_heads x 64)
// | v (kv_heads x 64); the cache of one layer is [kv_heads, max_pos, 64]; cos/sin are host tables [max_pos, 32];
// RoPE rotates the pairs (i, i + 32) of a head (rotate_half). The KV cache here is fp16 (the reference's is fp32): the
// values are rounded once, when stored, and every read (this position's too) sees the stored fp16 values.
//
// Positions come from device memory (*pos), so a captured step can be replayed while the position advances on the
// device (see k_argmax_step).
#include "aq_common.h"

namespace aq {

constexpr int kHd = 64;     // head dimension
constexpr int kHalf = 32;   // RoPE pairs per head
constexpr int kAttnT = 512; // threads of an attention workgroup

// x[i] = table[token, i] (fp16 -> fp32); d % 8 == 0. A token outside [0, vocab) reads row 0.
__global__ __launch_bounds__(256) void k_embed(const uint16_t* __restrict__ table, int64_t vocab, int d,
                                               const int32_t* __restrict__ token, float* __restrict__ x) {
  int64_t tok = *token;
  tok = (tok < 0 || tok >= vocab) ? 0 : tok;
  const uint4* row = reinterpret_cast<const uint4*>(table + tok * d);
  for (int i = blockIdx.x * 256 + threadIdx.x; i < d / 8; i += gridDim.x * 256) {
    const uint4 h = row[i];
    float4* dst = reinterpret_cast<float4*>(x + 8 * i);
    dst[0] = make_float4(half_bits_to_float(h.x & 0xFFFF), half_bits_to_float(h.x >> 16),
                         half_bits_to_float(h.y & 0xFFFF), half_bits_to_float(h.y >> 16));
    dst[1] = make_float4(half_bits_to_float(h.z & 0xFFFF), half_bits_to_float(h.z >> 16),
                         half_bits_to_float(h.w & 0xFFFF), half_bits_to_float(h.w >> 16));
  }
}

__device__ __forceinline__ void unpack8(const uint4 h, float* v) {
  v[0] = half_bits_to_float(h.x & 0xFFFF);
  v[1] = half_bits_to_float(h.x >> 16);
  v[2] = half_bits_to_float(h.y & 0xFFFF);
  v[3] = half_bits_to_float(h.y >> 16);
  v[4] = half_bits_to_float(h.z & 0xFFFF);
  v[5] = half_bits_to_float(h.z >> 16);
  v[6] = half_bits_to_float(h.w & 0xFFFF);
  v[7] = half_bits_to_float(h.w >> 16);
}

// One workgroup per KV head g and its HPG query heads, which share every key and value row read.
//   1. The cached key and value rows s < pos of the first 512-position batch are requested at once (8 of each per
//      thread): they do not depend on this token, so their latency overlaps step 2. Row pos, written in step 2, is
//      taken from LDS instead.
//   2. RoPE on the HPG query heads (to LDS) and on the key; key and value of position pos go to the cache (fp16) and,
//      as the fp16 values stored, to LDS.
//   3. Scores s < n = pos + 1: dot(q_h, k_s) / 8, eight lanes per key row (8 dimensions each, then a DPP sum over the
//      8 lanes), all HPG heads per row read.
//   4. Softmax per head (workgroup max, exp, workgroup sum).
//   5. out_h = sum_s p_hs v_s / sum_s p_hs: a thread takes 8 dimensions of every 64th position for all HPG heads,
//      then the 64 position groups are summed (pairs by DPP, then 32 partials per output in LDS).
// Positions past 512 (max_pos > 512) run further batches, requested when they are used.
template <int HPG>
__global__ __launch_bounds__(kAttnT) void k_attn_decode(const float* __restrict__ qkv, const float* __restrict__ cosb,
                                                        const float* __restrict__ sinb, uint16_t* kc, uint16_t* vc,
                                                        const int32_t* __restrict__ pos_p, int heads, int kv_heads,
                                                        int max_pos, float* __restrict__ out) {
  constexpr int kStride = kAttnT / 8;           // 64 positions per pass of the workgroup
  constexpr int kRows = HPG >= 8 ? 4 : 8;       // rows of each kind a thread requests at once
  constexpr int kBatch = kStride * kRows;
  extern __shared__ float sc[];  // [HPG][max_pos]: scores, then unnormalised probabilities
  __shared__ float qs[HPG][kHd];
  __shared__ float cur[2][kHd];  // key (rotated) and value of position pos, as stored (fp16 values)
  __shared__ float red[kAttnT / 64][HPG];
  __shared__ float pv[kAttnT / 16][HPG][kHd];  // per (wave, row of 16 lanes) partial outputs
  const int g = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int pos = *pos_p;
  float* o = out + (size_t)g * HPG * kHd;
  if (pos < 0 || pos >= max_pos) {  // no valid position (workgroup-uniform): zeros, nothing written to the cache
    for (int i = t; i < HPG * kHd; i += kAttnT) o[i] = 0.f;
    return;
  }
  const int n = pos + 1;
  const size_t cbase = (size_t)g * max_pos * kHd;
  const int c = t & 7;    // dimensions 8c .. 8c + 7 of every row this thread reads
  const int pg = t >> 3;  // positions pg, pg + 64, ...
  const int batches = (n + kBatch - 1) / kBatch;
  const uint16_t* kbase = kc + cbase + 8 * c;
  const uint16_t* vbase = vc + cbase + 8 * c;

  // 1. rows past pos re-read row pos (in bounds; replaced or unused)
  uint4 kr[kRows], vr[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const size_t row = (size_t)min(pg + kStride * i, pos) * kHd;
    kr[i] = *reinterpret_cast<const uint4*>(kbase + row);
    vr[i] = *reinterpret_cast<const uint4*>(vbase + row);
  }

  // 2.
  if (t < HPG * kHalf) {
    const int hh = t / kHalf, i = t % kHalf;
    const float* q = qkv + (size_t)(g * HPG + hh) * kHd;
    const float a = q[i], b = q[i + kHalf];
    const float cs = cosb[pos * kHalf + i], sn = sinb[pos * kHalf + i];
    qs[hh][i] = a * cs - b * sn;
    qs[hh][i + kHalf] = b * cs + a * sn;
  } else if (t < (HPG + 1) * kHalf) {
    const int i = t - HPG * kHalf;
    const float* kp = qkv + (size_t)heads * kHd + g * kHd;
    const float* vp = qkv + (size_t)(heads + kv_heads) * kHd + g * kHd;
    const float a = kp[i], b = kp[i + kHalf];
    const float cs = cosb[pos * kHalf + i], sn = sinb[pos * kHalf + i];
    const uint16_t k0 = float_to_half_bits(a * cs - b * sn), k1 = float_to_half_bits(b * cs + a * sn);
    const uint16_t v0 = float_to_half_bits(vp[i]), v1 = float_to_half_bits(vp[i + kHalf]);
    uint16_t* kd = kc + cbase + (size_t)pos * kHd;
    uint16_t* vd = vc + cbase + (size_t)pos * kHd;
    kd[i] = k0;
    kd[i + kHalf] = k1;
    vd[i] = v0;
    vd[i + kHalf] = v1;
    cur[0][i] = half_bits_to_float(k0);
    cur[0][i + kHalf] = half_bits_to_float(k1);
    cur[1][i] = half_bits_to_float(v0);
    cur[1][i + kHalf] = half_bits_to_float(v1);
  }
  __syncthreads();

  // 3.
  float qr[HPG][8], kcur[8], vcur[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int h = 0; h < HPG; ++h) qr[h][e] = qs[h][8 * c + e];
    kcur[e] = cur[0][8 * c + e];
    vcur[e] = cur[1][8 * c + e];
  }
  float m[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) m[h] = -INFINITY;
  auto score_rows = [&](const uint4 (&rows)[kRows], int b) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int s = b * kBatch + pg + kStride * i;
      float k8[8];
      unpack8(rows[i], k8);
#pragma unroll
      for (int e = 0; e < 8; ++e) k8[e] = s == pos ? kcur[e] : k8[e];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qr[h][e], k8[e], d);
        const float v = sum8(d) * 0.125f;  // the row's 8 lanes; 1 / sqrt(64)
        if (s < n) {
          if (c == 0) sc[h * max_pos + s] = v;
          m[h] = fmaxf(m[h], v);
        }
      }
    }
  };
  score_rows(kr, 0);
  for (int b = 1; b < batches; ++b) {
    uint4 k2[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i)
      k2[i] = *reinterpret_cast<const uint4*>(kbase + (size_t)min(b * kBatch + pg + kStride * i, pos) * kHd);
    score_rows(k2, b);
  }

  // 4.
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    m[h] = wave_max(m[h]);
    if (lane == 0) red[wave][h] = m[h];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    float v = red[0][h];
#pragma unroll
    for (int w = 1; w < kAttnT / 64; ++w) v = fmaxf(v, red[w][h]);
    m[h] = v;
  }
  __syncthreads();  // red is reused below

  float l[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) l[h] = 0.f;
  for (int s = t; s < n; s += kAttnT) {
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      const float e = expf(sc[h * max_pos + s] - m[h]);
      sc[h * max_pos + s] = e;
      l[h] += e;
    }
  }
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    l[h] = wave_sum(l[h]);
    if (lane == 0) red[wave][h] = l[h];
  }
  __syncthreads();  // also publishes the probabilities
  float total[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnT / 64; ++w) v += red[w][h];
    total[h] = v;
  }

  // 5.
  float acc[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  auto accumulate = [&](const uint4 (&rows)[kRows], int b) {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int s = b * kBatch + pg + kStride * i;
      if (s >= n) break;  // positions rise with i
      float v8[8];
      unpack8(rows[i], v8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v8[e] = s == pos ? vcur[e] : v8[e];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        const float p = sc[h * max_pos + s];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, v8[e], acc[h][e]);
      }
    }
  };
  accumulate(vr, 0);
  for (int b = 1; b < batches; ++b) {
    uint4 v2[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i)
      v2[i] = *reinterpret_cast<const uint4*>(vbase + (size_t)min(b * kBatch + pg + kStride * i, pos) * kHd);
    accumulate(v2, b);
  }
  // Lanes l and l ^ 8 hold neighbouring position groups of the same 8 dimensions: add them by DPP (row_ror:8), then
  // the four rows of each wave and the 8 waves meet in LDS.
#pragma unroll
  for (int h = 0; h < HPG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] += dpp<0x128>(0.f, acc[h][e]);
  if ((lane & 8) == 0) {
    const int row = lane >> 4;
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      float4* dst = reinterpret_cast<float4*>(&pv[wave * 4 + row][h][8 * c]);
      dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  __syncthreads();
  for (int i = t; i < HPG * kHd; i += kAttnT) {
    const int h = i / kHd, d = i % kHd;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnT / 16; ++w) v += pv[w][h][d];
    o[i] = v / total[h];
  }
}

// Split attention (flash decoding): workgroup (g, sp) covers positions [sp * P, sp * P + P) of KV head g for its HPG
// query heads and writes, per head h, the partial softmax state of those positions: m = max score, l = sum exp(s - m),
// o[d] = sum exp(s - m) v[d] (unnormalised). aq_attn_out_q4 combines the splits while it stages x for the output
// projection, so the 8 KV heads spread over 8 * splits workgroups with no extra launch.
//   parts  o: [heads][splits][64] floats, then m, l: [heads][splits][2] floats
// A split past the last position writes m = -inf, l = 0, o = 0. The split holding pos does RoPE of the key and the
// cache append (and uses that row from LDS); every split rotates the queries itself. The span's first rows and the
// q, k, v values are requested before the position is read (they do not depend on it).
template <int HPG>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ qkv, const float* __restrict__ cosb,
                                                    const float* __restrict__ sinb, uint16_t* kc, uint16_t* vc,
                                                    const int32_t* __restrict__ pos_p, int heads, int kv_heads,
                                                    int max_pos, int span, float* __restrict__ parts) {
  constexpr int kT = 256;
  constexpr int kStride = kT / 8;  // 32 positions per pass
  extern __shared__ float sc[];    // [HPG][span]
  __shared__ float qs[HPG][kHd];
  __shared__ float cur[2][kHd];
  __shared__ float red[kT / 64][HPG];
  __shared__ float pv[kT / 16][HPG][kHd];
  const int g = blockIdx.x, sp = blockIdx.y, splits = gridDim.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int s0 = sp * span;
  const int c = t & 7, pg = t >> 3;
  const size_t cbase = (size_t)g * max_pos * kHd;
  const uint16_t* kbase = kc + cbase + 8 * c;
  const uint16_t* vbase = vc + cbase + 8 * c;
  // Requests that do not depend on the position go out before it is read: the span's first cached rows (two of each
  // per thread; rows past the position hold stale values and are masked below, row pos is taken from LDS) and this
  // head group's q, k, v.
  uint4 kr[2], vr[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const size_t row = (size_t)min(s0 + pg + kStride * i, max_pos - 1) * kHd;
    kr[i] = *reinterpret_cast<const uint4*>(kbase + row);
    vr[i] = *reinterpret_cast<const uint4*>(vbase + row);
  }
  const int qi = t % kHalf;
  const float* qp = qkv + (size_t)(g * HPG + min(t / kHalf, HPG - 1)) * kHd;
  const float qa = qp[qi], qb = qp[qi + kHalf];
  const float* kp = qkv + (size_t)heads * kHd + g * kHd;
  const float* vp = qkv + (size_t)(heads + kv_heads) * kHd + g * kHd;
  const float ka = kp[qi], kb = kp[qi + kHalf], va = vp[qi], vb = vp[qi + kHalf];
  const int pos = *pos_p;
  float* po = parts + (size_t)g * HPG * splits * kHd;                       // o of head g*HPG + h, split sp
  float* pml = parts + (size_t)heads * splits * kHd + (size_t)g * HPG * splits * 2;
  if (pos < 0 || pos >= max_pos || s0 > pos) {  // workgroup-uniform: no position here
    for (int i = t; i < HPG * kHd; i += kT) po[((i / kHd) * splits + sp) * kHd + i % kHd] = 0.f;
    if (t < HPG) {
      pml[(t * splits + sp) * 2] = -INFINITY;
      pml[(t * splits + sp) * 2 + 1] = 0.f;
    }
    return;
  }
  const int s1 = min(s0 + span, pos + 1);  // this split's positions: [s0, s1)
  const bool mine = pos < s0 + span;       // holds position pos: rotates and stores its key and value
  const int passes = (s1 - s0 + 2 * kStride - 1) / (2 * kStride);

  const float cs = cosb[pos * kHalf + qi], sn = sinb[pos * kHalf + qi];
  if (t < HPG * kHalf) {
    const int hh = t / kHalf;
    qs[hh][qi] = qa * cs - qb * sn;
    qs[hh][qi + kHalf] = qb * cs + qa * sn;
  }
  if (mine && t >= kT - kHalf) {  // the last 32 threads (with 8 query heads they also rotated a query pair)
    const int i = qi;
    const uint16_t k0 = float_to_half_bits(ka * cs - kb * sn), k1 = float_to_half_bits(kb * cs + ka * sn);
    const uint16_t v0 = float_to_half_bits(va), v1 = float_to_half_bits(vb);
    uint16_t* kd = kc + cbase + (size_t)pos * kHd;
    uint16_t* vd = vc + cbase + (size_t)pos * kHd;
    kd[i] = k0;
    kd[i + kHalf] = k1;
    vd[i] = v0;
    vd[i + kHalf] = v1;
    cur[0][i] = half_bits_to_float(k0);
    cur[0][i + kHalf] = half_bits_to_float(k1);
    cur[1][i] = half_bits_to_float(v0);
    cur[1][i + kHalf] = half_bits_to_float(v1);
  }
  __syncthreads();

  float qr[HPG][8], kcur[8], vcur[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int h = 0; h < HPG; ++h) qr[h][e] = qs[h][8 * c + e];
    kcur[e] = cur[0][8 * c + e];  // read only where s == pos, which only the split holding pos has
    vcur[e] = cur[1][8 * c + e];
  }
  float m[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) m[h] = -INFINITY;
  auto score_rows = [&](const uint4 (&rows)[2], int base) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = base + pg + kStride * i;
      float k8[8];
      unpack8(rows[i], k8);
#pragma unroll
      for (int e = 0; e < 8; ++e) k8[e] = s == pos ? kcur[e] : k8[e];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qr[h][e], k8[e], d);
        const float v = sum8(d) * 0.125f;  // 1 / sqrt(64)
        if (s < s1) {
          if (c == 0) sc[h * span + (s - s0)] = v;
          m[h] = fmaxf(m[h], v);
        }
      }
    }
  };
  score_rows(kr, s0);
  for (int p = 1; p < passes; ++p) {
    uint4 k2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      k2[i] = *reinterpret_cast<const uint4*>(kbase + (size_t)min(s0 + 2 * kStride * p + pg + kStride * i, pos) * kHd);
    score_rows(k2, s0 + 2 * kStride * p);
  }
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    m[h] = wave_max(m[h]);
    if (lane == 0) red[wave][h] = m[h];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < HPG; ++h) m[h] = fmaxf(fmaxf(red[0][h], red[1][h]), fmaxf(red[2][h], red[3][h]));
  __syncthreads();  // red is reused below

  float l[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) l[h] = 0.f;
  for (int s = t; s < s1 - s0; s += kT) {
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      const float e = expf(sc[h * span + s] - m[h]);
      sc[h * span + s] = e;
      l[h] += e;
    }
  }
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    l[h] = wave_sum(l[h]);
    if (lane == 0) red[wave][h] = l[h];
  }
  __syncthreads();  // also publishes the probabilities

  float acc[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  auto accumulate = [&](const uint4 (&rows)[2], int base) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = base + pg + kStride * i;
      if (s >= s1) break;  // positions rise with i
      float v8[8];
      unpack8(rows[i], v8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v8[e] = s == pos ? vcur[e] : v8[e];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        const float p = sc[h * span + (s - s0)];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, v8[e], acc[h][e]);
      }
    }
  };
  accumulate(vr, s0);
  for (int p = 1; p < passes; ++p) {
    uint4 v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      v2[i] = *reinterpret_cast<const uint4*>(vbase + (size_t)min(s0 + 2 * kStride * p + pg + kStride * i, pos) * kHd);
    accumulate(v2, s0 + 2 * kStride * p);
  }
#pragma unroll
  for (int h = 0; h < HPG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] += dpp<0x128>(0.f, acc[h][e]);  // lanes l, l ^ 8: neighbouring groups
  if ((lane & 8) == 0) {
    const int row = lane >> 4;
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      float4* dst = reinterpret_cast<float4*>(&pv[wave * 4 + row][h][8 * c]);
      dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  __syncthreads();
  for (int i = t; i < HPG * kHd; i += kT) {
    const int h = i / kHd, d = i % kHd;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kT / 16; ++w) v += pv[w][h][d];
    po[(h * splits + sp) * kHd + d] = v;
  }
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    if (t == h) {
      pml[(h * splits + sp) * 2] = m[h];
      pml[(h * splits + sp) * 2 + 1] = red[0][h] + red[1][h] + red[2][h] + red[3][h];
    }
  }
}

template <int HPG>
static int launch_split(const float* qkv, const float* cosb, const float* sinb, uint16_t* kc, uint16_t* vc,
                        const int32_t* pos, int heads, int kv_heads, int max_pos, int splits, float* parts,
                        hipStream_t s) {
  const int span = ((max_pos + splits - 1) / splits + 63) / 64 * 64;
  hipLaunchKernelGGL(k_attn_split<HPG>, dim3(kv_heads, splits), dim3(256), (size_t)HPG * span * sizeof(float), s,
                     qkv, cosb, sinb, kc, vc, pos, heads, kv_heads, max_pos, span, parts);
  return launch_status();
}

template <int HPG>
static int launch_attn(const float* qkv, const float* cosb, const float* sinb, uint16_t* kc, uint16_t* vc,
                       const int32_t* pos, int heads, int kv_heads, int max_pos, float* out, hipStream_t s) {
  const size_t lds = (size_t)HPG * max_pos * sizeof(float);
  const size_t static_lds = (size_t)HPG * kHd * 4 * (1 + kAttnT / 16) + (size_t)HPG * 4 * (kAttnT / 64) + 2 * kHd * 4;
  auto kern = k_attn_decode<HPG>;
  if (lds + static_lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return AQ_ERR_CAPACITY;
  hipLaunchKernelGGL(kern, dim3(kv_heads), dim3(kAttnT), lds, s, qkv, cosb, sinb, kc, vc, pos, heads, kv_heads,
                     max_pos, out);
  return launch_status();
}

}  // namespace aq

extern "C" int aq_embed_f16(const uint16_t* table, int64_t vocab, int64_t d, const int32_t* token, float* x,
                            void* stream) {
  if (!table || !token || !x) return AQ_ERR_NULL;
  if (vocab <= 0 || d <= 0 || d % 8 || d > (1 << 24)) return AQ_ERR_SHAPE;
  if (!aq::aligned(table, 16) || !aq::aligned(x, 16)) return AQ_ERR_ALIGN;
  const int64_t blocks = (d / 8 + 255) / 256;
  hipLaunchKernelGGL(aq::k_embed, dim3((unsigned)(blocks > 256 ? 256 : blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), table, vocab, (int)d, token, x);
  return aq::launch_status();
}

extern "C" int aq_attn_decode(const float* qkv, const float* cos_tab, const float* sin_tab, uint16_t* k_cache,
                              uint16_t* v_cache, const int32_t* pos, int32_t heads, int32_t kv_heads,
                              int32_t head_dim, int32_t max_pos, float* out, void* stream) {
  if (!qkv || !cos_tab || !sin_tab || !k_cache || !v_cache || !pos || !out) return AQ_ERR_NULL;
  if (head_dim != aq::kHd || heads <= 0 || kv_heads <= 0 || heads % kv_heads || max_pos <= 0) return AQ_ERR_SHAPE;
  const int hpg = heads / kv_heads;
  if (hpg != 1 && hpg != 2 && hpg != 4 && hpg != 8) return AQ_ERR_SHAPE;
  // LDS: the scores (hpg * max_pos floats) beside the static arrays (q, reductions, 32 partial outputs per head dim)
  const int64_t lds = (int64_t)hpg * max_pos * 4 + (int64_t)hpg * aq::kHd * 4 * (1 + aq::kAttnT / 16) +
                      (int64_t)hpg * 4 * (aq::kAttnT / 64) + 2 * aq::kHd * 4;
  if (lds > 160 * 1024) return AQ_ERR_CAPACITY;
  if (!aq::aligned(k_cache, 16) || !aq::aligned(v_cache, 16)) return AQ_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (hpg) {
    case 1: return aq::launch_attn<1>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, out, s);
    case 2: return aq::launch_attn<2>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, out, s);
    case 4: return aq::launch_attn<4>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, out, s);
    default: return aq::launch_attn<8>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, out, s);
  }
}

extern "C" int aq_attn_decode_split(const float* qkv, const float* cos_tab, const float* sin_tab, uint16_t* k_cache,
                                    uint16_t* v_cache, const int32_t* pos, int32_t heads, int32_t kv_heads,
                                    int32_t head_dim, int32_t max_pos, int32_t splits, float* parts, void* stream) {
  if (!qkv || !cos_tab || !sin_tab || !k_cache || !v_cache || !pos || !parts) return AQ_ERR_NULL;
  if (head_dim != aq::kHd || heads <= 0 || kv_heads <= 0 || heads % kv_heads || max_pos <= 0) return AQ_ERR_SHAPE;
  if (splits < 1 || splits > AQ_ATTN_MAX_SPLITS || splits > max_pos) return AQ_ERR_SHAPE;
  const int hpg = heads / kv_heads;
  if (hpg != 1 && hpg != 2 && hpg != 4 && hpg != 8) return AQ_ERR_SHAPE;
  const int64_t span = ((max_pos + splits - 1) / splits + 63) / 64 * 64;
  if (hpg * span * 4 > 64 * 1024) return AQ_ERR_CAPACITY;
  if (!aq::aligned(k_cache, 16) || !aq::aligned(v_cache, 16)) return AQ_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (hpg) {
    case 1: return aq::launch_split<1>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, splits, parts, s);
    case 2: return aq::launch_split<2>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, splits, parts, s);
    case 4: return aq::launch_split<4>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, splits, parts, s);
    default: return aq::launch_split<8>(qkv, cos_tab, sin_tab, k_cache, v_cache, pos, heads, kv_heads, max_pos, splits, parts, s);
  }
}
