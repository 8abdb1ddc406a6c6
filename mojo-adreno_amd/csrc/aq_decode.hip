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
// device (the head's launch advances it: aq_step_end.h).
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
// cache append (and uses that row from registers).
// Thread t = 8 pg + c owns dimensions 8c .. 8c + 7 of positions s0 + 64 p + pg + 32 i (pass p, i = 0, 1). Everything
// a wave needs stays in its registers until the end: each lane rotates its own dimensions of the queries (it loads
// their RoPE partners too), a score is a DPP sum over the 8 lanes of a position, and each wave keeps its own running
// maximum and rescales its sums when it grows (online softmax), so the only barrier is the final merge of the four
// waves' states through LDS. The span's first key and value rows and the q, k, v values are requested before the
// position is read (they do not depend on it).
template <int HPG>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ qkv, const float* __restrict__ cosb,
                                                    const float* __restrict__ sinb, uint16_t* kc, uint16_t* vc,
                                                    const int32_t* __restrict__ pos_p, int heads, int kv_heads,
                                                    int max_pos, int span, float* __restrict__ parts) {
  constexpr int kT = 256;
  constexpr int kStride = kT / 8;  // 32 positions per row of a pass
  __shared__ float pv[kT / 16][HPG][kHd];  // per (wave, row of 16 lanes) partial outputs
  __shared__ float2 mls[kT / 64][HPG];     // per wave (m, l)
  const int g = blockIdx.x, sp = blockIdx.y, splits = gridDim.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int s0 = sp * span;
  const int c = t & 7, pg = t >> 3;
  const size_t cbase = (size_t)g * max_pos * kHd;
  const uint16_t* kbase = kc + cbase + 8 * c;
  const uint16_t* vbase = vc + cbase + 8 * c;
  uint4 kr[2], vr[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const size_t row = (size_t)min(s0 + pg + kStride * i, max_pos - 1) * kHd;
    kr[i] = *reinterpret_cast<const uint4*>(kbase + row);
    vr[i] = *reinterpret_cast<const uint4*>(vbase + row);
  }
  // this lane's 8 dimensions d = 8c + e of q (every head), k and v, and their RoPE partners d +- 32
  const int d0 = 8 * c, dp = c < 4 ? d0 + kHalf : d0 - kHalf, qi0 = d0 & (kHalf - 1);
  float4 qa[HPG][2], qb[HPG][2];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    const float4* qp = reinterpret_cast<const float4*>(qkv + (size_t)(g * HPG + h) * kHd);
    qa[h][0] = qp[d0 / 4];
    qa[h][1] = qp[d0 / 4 + 1];
    qb[h][0] = qp[dp / 4];
    qb[h][1] = qp[dp / 4 + 1];
  }
  const float4* kp = reinterpret_cast<const float4*>(qkv + (size_t)heads * kHd + g * kHd);
  const float4* vp = reinterpret_cast<const float4*>(qkv + (size_t)(heads + kv_heads) * kHd + g * kHd);
  const float4 ka0 = kp[d0 / 4], ka1 = kp[d0 / 4 + 1], kb0 = kp[dp / 4], kb1 = kp[dp / 4 + 1];
  const float4 va0 = vp[d0 / 4], va1 = vp[d0 / 4 + 1];
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

  // RoPE (rotate_half): for d < 32, x'[d] = x[d] cos - x[d + 32] sin; for d >= 32, x'[d] = x[d] cos + x[d - 32] sin
  float cs[8], sn[8];
  {
    const float4* cp = reinterpret_cast<const float4*>(cosb + (size_t)pos * kHalf + qi0);
    const float4* sq = reinterpret_cast<const float4*>(sinb + (size_t)pos * kHalf + qi0);
    const float4 c0 = cp[0], c1 = cp[1], q0 = sq[0], q1 = sq[1];
    const float sgn = c < 4 ? -1.f : 1.f;
    cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
    sn[0] = sgn * q0.x; sn[1] = sgn * q0.y; sn[2] = sgn * q0.z; sn[3] = sgn * q0.w;
    sn[4] = sgn * q1.x; sn[5] = sgn * q1.y; sn[6] = sgn * q1.z; sn[7] = sgn * q1.w;
  }
  auto rope8 = [&](const float4 a0, const float4 a1, const float4 b0, const float4 b1, float (&out)[8]) {
    const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = a[e] * cs[e] + b[e] * sn[e];
  };
  float qr[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h) rope8(qa[h][0], qa[h][1], qb[h][0], qb[h][1], qr[h]);
  // the key and value of position pos as the cache stores them (fp16), kept in registers for that row
  float kcur[8], vcur[8];
  {
    float kf[8];
    rope8(ka0, ka1, kb0, kb1, kf);
    const float vf[8] = {va0.x, va0.y, va0.z, va0.w, va1.x, va1.y, va1.z, va1.w};
    uint32_t kw[4], vw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t k0 = float_to_half_bits(kf[2 * e]), k1 = float_to_half_bits(kf[2 * e + 1]);
      const uint16_t v0 = float_to_half_bits(vf[2 * e]), v1 = float_to_half_bits(vf[2 * e + 1]);
      kw[e] = (uint32_t)k0 | ((uint32_t)k1 << 16);
      vw[e] = (uint32_t)v0 | ((uint32_t)v1 << 16);
      kcur[2 * e] = half_bits_to_float(k0);
      kcur[2 * e + 1] = half_bits_to_float(k1);
      vcur[2 * e] = half_bits_to_float(v0);
      vcur[2 * e + 1] = half_bits_to_float(v1);
    }
    if (mine && pg == 0) {  // eight lanes store the row (16 bytes each)
      *reinterpret_cast<uint4*>(kc + cbase + (size_t)pos * kHd + d0) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
      *reinterpret_cast<uint4*>(vc + cbase + (size_t)pos * kHd + d0) = make_uint4(vw[0], vw[1], vw[2], vw[3]);
    }
  }

  // online softmax of this wave's positions: m (wave-uniform), and per lane l (lanes c == 0 count each position
  // once) and the unnormalised output acc over the lane's 8 dimensions
  float m[HPG], l[HPG], acc[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
  for (int p = 0; p < passes; ++p) {
    const int base = s0 + 2 * kStride * p;
    uint4 k2[2], v2[2];
    if (p == 0) {
      k2[0] = kr[0]; k2[1] = kr[1]; v2[0] = vr[0]; v2[1] = vr[1];
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const size_t row = (size_t)min(base + pg + kStride * i, pos) * kHd;
        k2[i] = *reinterpret_cast<const uint4*>(kbase + row);
        v2[i] = *reinterpret_cast<const uint4*>(vbase + row);
      }
    }
    float sc[2][HPG];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = base + pg + kStride * i;
      float k8[8];
      unpack8(k2[i], k8);
#pragma unroll
      for (int e = 0; e < 8; ++e) k8[e] = s == pos ? kcur[e] : k8[e];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qr[h][e], k8[e], d);
        const float v = sum8(d) * 0.125f;  // 1 / sqrt(64)
        sc[i][h] = s < s1 ? v : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      const float mn = fmaxf(m[h], wave_max(fmaxf(sc[0][h], sc[1][h])));
      // mn = -inf (wave-uniform): no position of this wave so far, and l, acc are still 0. Measuring from 0 then gives
      // r = p0 = p1 = 0 and leaves them so; without a branch the heads' maximum and exponent chains interleave.
      const float mr = mn == -INFINITY ? 0.f : mn;
      const float r = expf(m[h] - mr);  // 0 while m was -inf
      const float p0 = expf(sc[0][h] - mr), p1 = expf(sc[1][h] - mr);  // 0 for masked positions
      l[h] = l[h] * r + (c == 0 ? p0 + p1 : 0.f);
      m[h] = mn;
      float v0[8], v1[8];
      unpack8(v2[0], v0);
      unpack8(v2[1], v1);
      const int sa = base + pg, sb = base + pg + kStride;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x0 = sa == pos ? vcur[e] : v0[e], x1 = sb == pos ? vcur[e] : v1[e];
        acc[h][e] = fmaf(p1, x1, fmaf(p0, x0, acc[h][e] * r));
      }
    }
  }
  // the wave's state: its 8 position groups' sums (lanes l, l ^ 8 by DPP, then the 4 rows through LDS), m, and l
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] += dpp<0x128>(0.f, acc[h][e]);  // lanes l, l ^ 8: neighbouring groups
    const float lw = wave_sum(l[h]);
    if (lane == 0) mls[wave][h] = make_float2(m[h], lw);
  }
  if ((lane & 8) == 0) {
    const int row = lane >> 4;
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      float4* dst = reinterpret_cast<float4*>(&pv[wave * 4 + row][h][d0]);
      dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  __syncthreads();
  // merge the four waves: M = max m_w, o = sum_w e^(m_w - M) o_w, l = sum_w e^(m_w - M) l_w
  for (int i = t; i < HPG * kHd; i += kT) {
    const int h = i / kHd, d = i % kHd;
    float mw = -INFINITY;
#pragma unroll
    for (int w = 0; w < kT / 64; ++w) mw = fmaxf(mw, mls[w][h].x);
    float v = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < kT / 64; ++w) {
      const float f = mls[w][h].x == -INFINITY ? 0.f : expf(mls[w][h].x - mw);
      const float ow = (pv[4 * w][h][d] + pv[4 * w + 1][h][d]) + (pv[4 * w + 2][h][d] + pv[4 * w + 3][h][d]);
      v = fmaf(f, ow, v);
      lt = fmaf(f, mls[w][h].y, lt);
    }
    po[(h * splits + sp) * kHd + d] = v;
    if (d == 0) {
      pml[(h * splits + sp) * 2] = mw;
      pml[(h * splits + sp) * 2 + 1] = lt;
    }
  }
}

template <int HPG>
static int launch_split(const float* qkv, const float* cosb, const float* sinb, uint16_t* kc, uint16_t* vc,
                        const int32_t* pos, int heads, int kv_heads, int max_pos, int splits, float* parts,
                        hipStream_t s) {
  const int span = ((max_pos + splits - 1) / splits + 63) / 64 * 64;
  hipLaunchKernelGGL(k_attn_split<HPG>, dim3(kv_heads, splits), dim3(256), 0, s,
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
