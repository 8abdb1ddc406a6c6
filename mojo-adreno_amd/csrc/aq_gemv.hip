// int4 (Q4W) matrix-vector products for decode and few-token batches, gfx950, including the MoE decode experts.
//
// The arithmetic is the reference's gemv_q4 family (llama/kernels/gemv_q4.mojo:13-30, gemv_add_q4.mojo:13-30,
// lfm2/kernels/lk.mojo:38-72,134-167, qwen3moe/kernels/moek.mojo:30-45,200-223,273-281,496-545): per row n,
//   y[n] = sum over groups of fp16 scale * sum_k ((nib ^ 8) - 8) * x[k], accumulated in fp32.
//
// Design (HBM-bound, ~0.5625 B per weight): a 256-thread workgroup stages x (all tokens) in LDS once, then each wave
// streams R weight rows at a time: every lane takes whole 16-byte, 32-weight chunks of the rows (chunk c = lane,
// lane + 64, ...), so a wave's loads of one row are 1 KB contiguous, and applies each word to all T tokens. With a
// power-of-two group >= 32 (one scale per chunk), x is staged as signed 4-bit digits of 22-bit fixed point and every
// word meets them in v_dot8_i32_i4 as stored (stage_digits, chunk_dot): exact integer chunk sums, ~1 VALU op per
// weight. Other groups (and the MoE-down mode) decode a word as q + 8 (XOR 0x88888888, byte masks ->
// v_cvt_f32_ubyte) against fp32 x and subtract 8 * sum(x) once per chunk. Row sums end in a wave reduction.
#include "aq_common.h"
#include "aq_digits.h"
#include "aq_step_end.h"
#include "aq_moe_decode.h"

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

// Decode-step fusions. norm != NULL: every token's x is RMS-normalised on staging, x * (1 / sqrt(mean(x^2) + eps))
// * norm[k] (fp16 weights), so no separate norm kernel runs before the product.
// parts != NULL (one token): x is the attention output combined from `splits` partial softmax states (the layout of
// aq_attn_decode_split): x[h * 64 + d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c, M = max_c m_c.
// With step.cand the launch also ends the greedy step (step_end): each workgroup's best key, then the token.
struct Fuse {
  const uint16_t* norm;
  float eps;
  const float* parts;
  int splits;
  StepEnd step;  // kStore, one token (step.cand NULL: none)
};


// Weight row r of the output block starting at `base` (every mode but kMoeDown; -1 = no row, kMoeGateUp only). Rows
// past the end repeat the last output's; their sums are not written.
template <int MODE, int RO>
__device__ __forceinline__ int gemv_row(int base, int r, int n_out, int f, const MoeArgs& moe) {
  int o = base + (r % RO);
  o = o < n_out ? o : n_out - 1;
  if constexpr (MODE == kMoeGateUp) {
    const int e = o / f, j = o - e * f;
    const int ex = moe.ids[e];
    return (ex >= 0 && ex < moe.experts) ? ex * 2 * f + j + (r >= RO ? f : 0) : -1;
  } else {
    return (MODE == kGateUp && r >= RO) ? f + o : o;
  }
}

// G32: the group size is a power of two >= 32 (one scale per 32-weight chunk). Otherwise every word looks up its own.
// D: register sets of the chunk pipeline (dense G32 modes), chosen at launch from the chunks a wave has.
// XR: one token, K <= 256 * XR * 8, x given (not split-attention states): each thread requests its XR words of x
// into registers before the weights, so their staging overlaps the weights' arrival (vector memory completes in
// order: x requested after the weights would wait for them). -1: the same for split-attention states (one word of
// x, i.e. K <= 2048). 0: x is loaded while it is staged.
template <bool G32, int R, int T, int MODE, int D, int XR>
__global__ __launch_bounds__(256) void k_gemv_q4(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                 const float* __restrict__ x, float* __restrict__ y, int n_out,
                                                 int k, int group, int f, int tokens, MoeArgs moe, Fuse fz) {
  // LDS layout, conflict-free for the chunk loop (lane c reads consecutive 16-byte slots). G32 (not kMoeDown): the
  // xd / xf planes of stage_digits. Otherwise:
  //   xs4[t][p][c]  float4 p = 2j + h holds x[t, 32c + 8j + 4h .. + 3]  (T * 8 planes of nch float4)
  //   xsum[t][j][c] sum of x[t, 32c + 8j .. + 7]                        (T * 4 planes of nch floats)
  extern __shared__ float4 lds4[];
  __shared__ float red[4 * T];
  const int kw = k >> 3;
  const int nch = k >> 5;
  float4* xs4 = lds4;
  float* xsum = reinterpret_cast<float*>(lds4 + T * 8 * nch);
  uint4* xd = reinterpret_cast<uint4*>(lds4);
  float* xf = reinterpret_cast<float*>(xd + T * 6 * nch);
  // digit products (v_dot8_i32_i4) for the G32 modes but kMoeDown
  constexpr bool kDigits = G32 && MODE != kMoeDown;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int gpr = k / group;
  constexpr int RO = (MODE == kGateUp || MODE == kMoeGateUp) ? R / 2 : R;
  constexpr int SL = MODE == kMoeDown ? T : 1;  // weight rows per output (kMoeDown: one per expert slot)
  // G32 products but kMoeDown (kStore, kAdd, kGateUp, and kMoeGateUp with rows from device expert ids) stream the
  // wave's chunks, over all its row blocks, through D register sets: D chunks are in flight while one is used (with
  // D > 1 the last D requests fall past the end and carry an out-of-range offset; with D = 1 nothing is requested
  // past the end). The rest (kMoeDown, groups that are not powers of two >= 32) request each chunk when they use it.
  constexpr bool kDeep = G32 && (MODE == kStore || MODE == kAdd || MODE == kGateUp || MODE == kMoeGateUp);
  const int stride = gridDim.x * 4 * RO;
  const int cpl = (nch + kWave - 1) / kWave;  // chunks per lane and row block (the last may be partial)

  // scales travel as raw fp16 bits and are converted where used: a conversion next to its load would wait for it
  const int gsh = __builtin_ctz(group);  // G32 groups are powers of two
  auto use_chunk = [&](int c, const uint4 (&w)[R], const uint16_t (&sc)[R], float (&acc)[R][T]) {
    chunk_dot<R, T>(xd, xf, nch, c, w, sc, acc);
  };

  // The first chunk of this wave's first row block is requested before x is staged, so its latency overlaps the
  // staging instead of following it.
  const int base0 = (blockIdx.x * 4 + wave) * RO;
  uint4 wd[D][R];
  uint32_t sd[D][R];  // the aligned 4 bytes holding each scale (fp16 pairs)
  uint32_t sh[D][R];  // ... and the scale's bit offset in them (0 or 16)
  // kDeep reads W and scales and writes y through buffer resources: a chunk past the wave's last row block, a tail
  // lane past K, or a lane that stores nothing issues its instruction with an out-of-range offset (no traffic, no
  // branch). Every chunk is then the same 2R loads, so the compiler's wait counts see the full pipeline depth.
  const int wrows = MODE == kGateUp ? 2 * f : MODE == kMoeGateUp ? moe.experts * 2 * f : n_out;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(wq, (uint32_t)((size_t)wrows * kw * 4));
  // scales are read as the aligned 4 bytes holding them (a 16-bit load would be widened right after it, waiting for
  // it); the range is rounded up to whole 4-byte words, so an odd count's last scale is read with the 2 bytes after it
  const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(ws, (uint32_t)(((size_t)wrows * gpr * 2 + 3) & ~(size_t)3));
  const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(y, (uint32_t)((size_t)tokens * n_out * 4));
  int ib = base0, ic = 0;  // kDeep: the next chunk to request (row block, chunk index)
  auto issue_next = [&](uint4 (&w)[R], uint32_t (&sc)[R], uint32_t (&sb)[R]) {
    const uint32_t c = lane + ic * kWave;
    const bool ok = ib < n_out && c < (uint32_t)nch;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int grow = gemv_row<MODE, RO>(ib, r, n_out, f, moe);  // a valid row even past the end (-1: no expert)
      const bool okr = ok && (MODE != kMoeGateUp || grow >= 0);   // no expert: zero words and scales
      const uint32_t row = (uint32_t)grow;
      const uint32_t wo = (row * (uint32_t)kw + 4 * c) * 4;
      const uint32_t si = row * (uint32_t)gpr + ((32 * c) >> gsh);
      w[r] = buf_load16p<kWPolicy>(w_rsrc, okr ? wo : kOOB);
      sc[r] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, okr ? (si * 2) & ~3u : kOOB, 0, 0);
      sb[r] = (si & 1) << 4;
    }
    if (ib < n_out && ++ic == cpl) ic = 0, ib += stride;
  };
  constexpr int kXi = XR > 0 ? XR : 1;
  float4 xra[kXi], xrb[kXi];
  uint4 xrn[kXi];
  float2 pml_r[AQ_ATTN_MAX_SPLITS];  // XR < 0: (m, l) of each split of this word's head, and its 8 partial outputs
  float4 poa_r[AQ_ATTN_MAX_SPLITS], pob_r[AQ_ATTN_MAX_SPLITS];
  if constexpr (XR < 0) {
    const int S = fz.splits;
    const uint32_t wi = threadIdx.x, h = wi >> 3, d0 = (wi & 7) * 8;
    const bool ok = wi < (uint32_t)kw;
    const uint32_t o_bytes = (uint32_t)(k / 64) * S * 64 * 4;
    const __amdgpu_buffer_rsrc_t p_rsrc = make_rsrc(fz.parts, o_bytes + (uint32_t)(k / 64) * S * 2 * 4);
#pragma unroll
    for (int cc = 0; cc < AQ_ATTN_MAX_SPLITS; ++cc) {
      const bool use = ok && cc < S;
      const uint32_t oo = ((h * S + cc) * 64 + d0) * 4;
      pml_r[cc] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 p_rsrc, use ? o_bytes + (h * S + cc) * 8 : kOOB, 0, 0));
      poa_r[cc] = __builtin_bit_cast(float4, buf_load16(p_rsrc, use ? oo : kOOB));
      pob_r[cc] = __builtin_bit_cast(float4, buf_load16(p_rsrc, use ? oo + 16 : kOOB));
    }
  }
  if constexpr (XR > 0) {
    // the norm weights first: a wait for x, which comes after them, then covers them, whether or not they exist
    if (fz.norm) {
      const __amdgpu_buffer_rsrc_t n_rsrc = make_rsrc(fz.norm, (uint32_t)k * 2);
#pragma unroll
      for (int i = 0; i < kXi; ++i) {
        const uint32_t wi = threadIdx.x + 256 * i;
        xrn[i] = buf_load16(n_rsrc, wi < (uint32_t)kw ? wi * 16 : kOOB);
      }
    }
    const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(x, (uint32_t)k * 4);
#pragma unroll
    for (int i = 0; i < kXi; ++i) {
      const uint32_t wi = threadIdx.x + 256 * i;
      const bool ok = wi < (uint32_t)kw;
      xra[i] = __builtin_bit_cast(float4, buf_load16(x_rsrc, ok ? wi * 32 : kOOB));
      xrb[i] = __builtin_bit_cast(float4, buf_load16(x_rsrc, ok ? wi * 32 + 16 : kOOB));
    }
  }
  if constexpr (kDeep) {
#pragma unroll
    for (int d = 0; d < D; ++d) issue_next(wd[d], sd[d], sh[d]);
  }
  // kAdd, one or two tokens: the residual of the wave's first row block, requested now (lane 0 stores) rather than
  // after its sums, so its latency is hidden behind the weights'
  constexpr bool kYPre = kDeep && MODE == kAdd && T <= 2;
  float ypre[kYPre ? RO : 1][T];
  if constexpr (kYPre) {
#pragma unroll
    for (int r = 0; r < RO; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int o = base0 + r;
        ypre[r][t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            y_rsrc, (lane == 0 && o < n_out && t < tokens) ? ((uint32_t)t * n_out + o) * 4 : kOOB, 0, 0));
      }
  }

  // Stage x in one pass. With a norm, x * norm_w is staged and sum(x^2) gathered on the way; the row sums are then
  // scaled by 1 / sqrt(mean(x^2) + eps) (a per-token scalar), which is the RMSNorm'd product.
  float ss[T];
#pragma unroll
  for (int t = 0; t < T; ++t) ss[t] = 0.f;
  // word wi (8 values) of token t: norm, then the LDS layouts above
  auto stage = [&](int t, int wi, float4 a, float4 b, const uint4 wn) {
    const int c = wi >> 2;
    const int j = wi & 3;
    if (fz.norm) {  // workgroup-uniform
      ss[t] += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) + ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
      a.x *= half_bits_to_float(wn.x & 0xFFFF);
      a.y *= half_bits_to_float(wn.x >> 16);
      a.z *= half_bits_to_float(wn.y & 0xFFFF);
      a.w *= half_bits_to_float(wn.y >> 16);
      b.x *= half_bits_to_float(wn.z & 0xFFFF);
      b.y *= half_bits_to_float(wn.z >> 16);
      b.z *= half_bits_to_float(wn.w & 0xFFFF);
      b.w *= half_bits_to_float(wn.w >> 16);
    }
    if constexpr (kDigits) {
      stage_digits(t, c, j, a, b, xd, xf, nch);
    } else {
      xs4[(t * 8 + 2 * j) * nch + c] = a;
      xs4[(t * 8 + 2 * j + 1) * nch + c] = b;
      xsum[(t * 4 + j) * nch + c] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    }
  };
  // the attention output for 8 dimensions from the splits' states: sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c
  auto combine = [&](const float2 (&ml)[AQ_ATTN_MAX_SPLITS], const float4 (&oa)[AQ_ATTN_MAX_SPLITS],
                     const float4 (&ob)[AQ_ATTN_MAX_SPLITS], float4& a, float4& b) {
    const int S = fz.splits;
    float mx = ml[0].x;
#pragma unroll
    for (int cc = 1; cc < AQ_ATTN_MAX_SPLITS; ++cc) mx = cc < S ? fmaxf(mx, ml[cc].x) : mx;
    float den = 0.f;
    a = make_float4(0.f, 0.f, 0.f, 0.f);
    b = a;
#pragma unroll
    for (int cc = 0; cc < AQ_ATTN_MAX_SPLITS; ++cc) {
      const float w = cc < S ? expf(ml[cc].x - mx) : 0.f;  // a split with no positions has m = -inf: weight 0
      den = fmaf(w, ml[cc].y, den);
      a.x = fmaf(w, oa[cc].x, a.x); a.y = fmaf(w, oa[cc].y, a.y);
      a.z = fmaf(w, oa[cc].z, a.z); a.w = fmaf(w, oa[cc].w, a.w);
      b.x = fmaf(w, ob[cc].x, b.x); b.y = fmaf(w, ob[cc].y, b.y);
      b.z = fmaf(w, ob[cc].z, b.z); b.w = fmaf(w, ob[cc].w, b.w);
    }
    const float r = 1.0f / den;
    a.x *= r; a.y *= r; a.z *= r; a.w *= r;
    b.x *= r; b.y *= r; b.z *= r; b.w *= r;
  };
  if constexpr (XR < 0) {
    if ((int)threadIdx.x < kw) {
      float4 a, b;
      combine(pml_r, poa_r, pob_r, a, b);
      stage(0, threadIdx.x, a, b, make_uint4(0u, 0u, 0u, 0u));
    }
  } else if constexpr (XR > 0) {
#pragma unroll
    for (int i = 0; i < kXi; ++i) {
      const int wi = threadIdx.x + 256 * i;
      if (wi < kw) stage(0, wi, xra[i], xrb[i], xrn[i]);
    }
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      for (int wi = threadIdx.x; wi < kw; wi += 256) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        uint4 wn = make_uint4(0u, 0u, 0u, 0u);
        if (fz.parts) {  // workgroup-uniform; one token: dimensions 8 (wi % 8) .. + 7 of head wi / 8
          const int h = wi >> 3, d0 = (wi & 7) * 8, S = fz.splits;
          const float* po = fz.parts + (size_t)h * S * 64 + d0;
          const float* pm = fz.parts + (size_t)(k / 64) * S * 64 + (size_t)h * S * 2;
          float2 ml[AQ_ATTN_MAX_SPLITS];
          float4 oa[AQ_ATTN_MAX_SPLITS], ob[AQ_ATTN_MAX_SPLITS];
#pragma unroll
          for (int cc = 0; cc < AQ_ATTN_MAX_SPLITS; ++cc) {  // all requests first
            const int ci = cc < S ? cc : 0;
            ml[cc] = make_float2(pm[2 * ci], pm[2 * ci + 1]);
            oa[cc] = *reinterpret_cast<const float4*>(po + ci * 64);
            ob[cc] = *reinterpret_cast<const float4*>(po + ci * 64 + 4);
          }
          combine(ml, oa, ob, a, b);
        } else if (t < tokens) {
          const float4* src = reinterpret_cast<const float4*>(x + (size_t)t * k + wi * 8);
          a = src[0];
          b = src[1];
          if (fz.norm) wn = *reinterpret_cast<const uint4*>(fz.norm + wi * 8);
        }
        stage(t, wi, a, b, wn);
      }
    }
  }
  if (fz.norm) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float v = wave_sum(ss[t]);
      if (lane == 0) red[wave * T + t] = v;
    }
  }
  __syncthreads();
  float rs[T];  // per-token RMSNorm scale (1 without a norm)
#pragma unroll
  for (int t = 0; t < T; ++t)
    rs[t] = fz.norm ? 1.0f / sqrtf(((red[t] + red[T + t]) + (red[2 * T + t] + red[3 * T + t])) / (float)k + fz.eps)
                    : 1.0f;

  float best = 0.f;  // argmax candidate of this wave (kStore, token 0)
  int best_row = -1;

  // the row sums of one row block: scaled by the norm, stored (or added, or combined as silu(gate) * up) by lane 0;
  // the other lanes' accesses carry an out-of-range offset
  auto finish = [&](int base, float (&acc)[R][T]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = wave_sum(acc[r][t]) * rs[t];
#pragma unroll
    for (int r = 0; r < RO; ++r) {
      const int o = base + r;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t off = (lane == 0 && o < n_out && t < tokens) ? ((uint32_t)t * n_out + o) * 4 : kOOB;
        float v = acc[r][t];
        if constexpr (MODE == kGateUp || MODE == kMoeGateUp) v = silu(v) * acc[RO + r][t];
        if constexpr (kYPre) {
          v += base == base0 ? ypre[r][t] : __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(y_rsrc, off, 0, 0));
        } else if constexpr (MODE == kAdd) {
          v += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(y_rsrc, off, 0, 0));
        }
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), y_rsrc, off, 0, 0);
      }
      if constexpr (MODE == kStore) {  // rows arrive in ascending order, so `>` keeps the first maximum; NaN rows
                                       // never win, as in the reference's `logits[i] > logits[best]` scan
        if (o < n_out && !__builtin_isnan(acc[r][0]) && (best_row < 0 || acc[r][0] > best))
          best = acc[r][0], best_row = o;
      }
    }
  };

  if constexpr (kDeep) {
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = 0.f;
    int cb = base0, cc = 0;  // the chunk to use next
    bool more = cb < n_out;
    // Every pass of the loop requests all D register sets, also past the wave's last chunk (out-of-range offsets: no
    // traffic), so that each way round the loop leaves the same loads in flight in the same order. Requests inside
    // `more` let the loop come back to its top with only some sets requested; the compiler's wait counts, which
    // merge all ways round, then waited for every load before the use of set 0.
    while (more) {
#pragma unroll
      for (int d = 0; d < D; ++d) {  // register set d by name: set d always holds the chunk d steps ahead
        const bool act = more;       // wave-uniform
        if (act) {
          const int c = lane + cc * kWave;
          if (c < nch) {
            uint16_t s16[R];
#pragma unroll
            for (int r = 0; r < R; ++r) s16[r] = (uint16_t)(sd[d][r] >> sh[d][r]);
            use_chunk(c, wd[d], s16, acc);
          }
        }
        if (D > 1 || (act && cb + (cc + 1 == cpl ? stride : 0) < n_out)) issue_next(wd[d], sd[d], sh[d]);
        if (act && ++cc == cpl) {
          finish(cb, acc);
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = 0.f;
          cc = 0;
          cb += stride;
          more = cb < n_out;
        }
      }
    }
  }

  for (int base = base0; kDeep ? false : base < n_out; base += stride) {
    int rows[R][SL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int o = base + (r % RO);
      o = o < n_out ? o : n_out - 1;  // rows past the end repeat the last one; their sums are not written
#pragma unroll
      for (int sl = 0; sl < SL; ++sl) {
        if constexpr (MODE == kMoeDown) {
          const int ex = sl < tokens ? moe.ids[sl] : -1;
          rows[r][sl] = (ex >= 0 && ex < moe.experts) ? ex * n_out + o : -1;
        } else {
          rows[r][sl] = gemv_row<MODE, RO>(base, r, n_out, f, moe);
        }
      }
    }
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = 0.f;

    {
      for (int c = lane; c < nch; c += kWave) {
        if constexpr (MODE == kMoeDown) {
          // one row per expert slot t, applied to that slot's activations only. Every slot's 16 bytes (and scale)
          // are requested before any is used (a slot with no expert reads zeros through an out-of-range offset), so
          // the T loads are in flight together rather than one after another.
          // the stacked experts' rows (the entry point keeps them below 2 GiB)
          const uint32_t mrows = (uint32_t)moe.experts * (uint32_t)n_out;
          const auto wm_rsrc = make_rsrc(wq, mrows * (uint32_t)kw * 4u);
          const auto sm_rsrc = make_rsrc(ws, mrows * (uint32_t)gpr * 2u);
          uint4 w4s[T];
          uint32_t s4s[T];
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const int row = rows[0][t];
            w4s[t] = buf_load16(wm_rsrc, row >= 0 ? ((uint32_t)row * (uint32_t)kw + (uint32_t)c * 4u) * 4u : kOOB);
            if constexpr (G32)
              s4s[t] = __builtin_amdgcn_raw_buffer_load_b16(
                  sm_rsrc, row >= 0 ? ((uint32_t)row * (uint32_t)gpr + (uint32_t)((c * 32) >> gsh)) * 2u : kOOB, 0, 0);
          }
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const int row = rows[0][t];
            if (row < 0) continue;  // wave-uniform
            const uint4 w4 = w4s[t];
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
            if constexpr (G32) part *= half_bits_to_float((uint16_t)s4s[t]);
            acc[0][t] += part;
          }
        } else {  // a group smaller than 32 or not a multiple of it: one scale per 8-weight word
          uint4 wv[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (MODE != kMoeGateUp || rows[r][0] >= 0)
              wv[r] = *reinterpret_cast<const uint4*>(wq + (size_t)rows[r][0] * kw + c * 4);
            else
              wv[r] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
          }
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
    }

    if constexpr (MODE == kMoeDown) {
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (t < tokens) sum = fmaf(moe.rw[t], wave_sum(acc[0][t]), sum);
      if (lane == 0) y[base] = moe.add ? y[base] + sum : sum;
      continue;
    }
    finish(base, acc);
  }
  if constexpr (MODE == kStore) {
    // workgroup-uniform; lane 0 holds its wave's first maximum (rows arrive in ascending order)
    if (fz.step.cand) workgroup_step_end<4>(fz.step, best_row < 0 ? 0ull : argmax_key(best, best_row));
  }
}

// One token, power-of-two groups >= 32, no fusions (the decode down projection, and products such as C0's
// 8192 x 2048): workgroups of 16 waves, so x is staged once per CU instead of once per four-wave workgroup. The 16
// waves are RP = 16 / KS row pairs times KS slices of K: each wave requests its two rows' chunks of its K slice, then
// its words of x, and the KS partial sums of an output meet in LDS, added in slice order. KS = 4 (K >= 8192) runs
// the 2048-row down projection with 16 waves per CU instead of 4 (a plain read of its bytes by 256 workgroups of 256
// threads takes 4.1 us against 3.6 us by 1024); KS = 1 (32 rows a workgroup) takes C0 from 4.46 to 4.22 us.
template <int KS, int CPS, int MODE, bool NORM>
__global__ __launch_bounds__(1024) void k_gemv_q4_ks(const uint32_t* __restrict__ wq,
                                                         const uint16_t* __restrict__ ws,
                                                         const float* __restrict__ x, float* __restrict__ y,
                                                         int n_out, int k, int gsh, int f,
                                                         const uint16_t* __restrict__ norm, float eps) {
  constexpr int RP = 16 / KS;                              // row pairs a workgroup
  constexpr int kRows = MODE == kGateUp ? RP : 2 * RP;     // outputs a workgroup (gate|up: one per row pair)
  extern __shared__ float4 lds4[];
  __shared__ float red[KS][2 * RP];
  __shared__ float rss[16];
  const int kw = k >> 3, nch = k >> 5, gpr = k >> gsh;
  uint4* xd = reinterpret_cast<uint4*>(lds4);
  float* xf = reinterpret_cast<float*>(xd + 6 * nch);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rp = wave % RP, ks = wave / RP;  // row pair, K slice
  const int c0 = (int)(((int64_t)nch * ks) / KS), c1 = (int)(((int64_t)nch * (ks + 1)) / KS);

  // norm weights first, then x: XR words a thread, requested before the weights (vector memory completes in order,
  // so waiting for x does not wait for the weights requested after it)
  constexpr int XR = 2;  // K <= 2 * 8 * 1024
  uint4 xn[XR];
  if constexpr (NORM) {
    const __amdgpu_buffer_rsrc_t n_rsrc = make_rsrc(norm, (uint32_t)k * 2);
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const uint32_t wi = threadIdx.x + 1024 * i;
      xn[i] = buf_load16(n_rsrc, wi < (uint32_t)kw ? wi * 16 : kOOB);
    }
  }
  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(x, (uint32_t)k * 4);
  float4 xa[XR], xc[XR];
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const uint32_t wi = threadIdx.x + 1024 * i;
    const bool ok = wi < (uint32_t)kw;
    xa[i] = __builtin_bit_cast(float4, buf_load16(x_rsrc, ok ? wi * 32 : kOOB));
    xc[i] = __builtin_bit_cast(float4, buf_load16(x_rsrc, ok ? wi * 32 + 16 : kOOB));
  }
  // the pair's two rows (gate|up: gate row o and up row f + o; otherwise outputs o0, o0 + 1), their chunks of this
  // slice; rows past the end repeat the last row, and their sums are not stored
  uint32_t rows[2];
  if constexpr (MODE == kGateUp) {
    const int o = min((int)blockIdx.x * RP + rp, n_out - 1);
    rows[0] = (uint32_t)o;
    rows[1] = (uint32_t)(f + o);
  } else {
    const int o0 = blockIdx.x * kRows + 2 * rp;
    rows[0] = (uint32_t)min(o0, n_out - 1);
    rows[1] = (uint32_t)min(o0 + 1, n_out - 1);
  }
  const size_t wrows = MODE == kGateUp ? 2 * (size_t)f : (size_t)n_out;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(wq, (uint32_t)(wrows * kw * 4));
  const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(ws, (uint32_t)((wrows * gpr * 2 + 3) & ~(size_t)3));
  uint4 w[CPS][2];
  uint32_t sc[CPS][2], sh[CPS][2];
#pragma unroll
  for (int j = 0; j < CPS; ++j) {
    const uint32_t c = (uint32_t)(c0 + lane + 64 * j);
    const bool ok = c < (uint32_t)c1;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t si = rows[r] * (uint32_t)gpr + ((32 * c) >> gsh);
      w[j][r] = buf_load16p<kWPolicy>(w_rsrc, ok ? (rows[r] * (uint32_t)kw + 4 * c) * 4 : kOOB);
      sc[j][r] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, ok ? (si * 2) & ~3u : kOOB, 0, 0);
      sh[j][r] = (si & 1) << 4;
    }
  }
  // the residual (kAdd), requested now rather than after the sums, so its latency is hidden too
  float yres = 0.f;
  if constexpr (MODE == kAdd) {
    const int o = blockIdx.x * kRows + (int)threadIdx.x;
    const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(y, (uint32_t)n_out * 4);
    yres = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        y_rsrc, threadIdx.x < kRows && o < n_out ? (uint32_t)o * 4 : kOOB, 0, 0));
  }
  // K split over the waves (KS > 1): x (and the norm weights) are taken by an empty statement here, after the
  // weights are requested. Left alone, the compiler sinks their loads into the staging branch below, behind the
  // weights', and the staging's wait for x then waits for the weights too; here the wait is for x alone (vector memory
  // completes in order). Measured: the 2048 x 8192 down projection 5.06 -> 4.94 us; with KS = 1 (C0, the decode
  // gate|up) the same pin was slower (4.31 -> 4.45 and 6.31 -> 6.79 us), so those keep the compiler's order.
  if constexpr (KS > 1) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      asm volatile("" ::"v"(xa[i].x), "v"(xa[i].y), "v"(xa[i].z), "v"(xa[i].w), "v"(xc[i].x), "v"(xc[i].y),
                   "v"(xc[i].z), "v"(xc[i].w));
      if constexpr (NORM) asm volatile("" ::"v"(xn[i].x), "v"(xn[i].y), "v"(xn[i].z), "v"(xn[i].w));
    }
  }
  // K % 32 == 0, so kw % 4 == 0: whole quads stage together, as stage_digits needs. With a norm, x * norm_w is
  // staged and sum(x^2) gathered; the sums are scaled by 1 / sqrt(mean(x^2) + eps) at the end (RMSNorm).
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int wi = threadIdx.x + 1024 * i;
    if (wi < kw) {
      float4 a = xa[i], b = xc[i];
      if constexpr (NORM) {
        ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) + ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
        const uint4 wn = xn[i];
        a.x *= half_bits_to_float(wn.x & 0xFFFF);
        a.y *= half_bits_to_float(wn.x >> 16);
        a.z *= half_bits_to_float(wn.y & 0xFFFF);
        a.w *= half_bits_to_float(wn.y >> 16);
        b.x *= half_bits_to_float(wn.z & 0xFFFF);
        b.y *= half_bits_to_float(wn.z >> 16);
        b.z *= half_bits_to_float(wn.w & 0xFFFF);
        b.w *= half_bits_to_float(wn.w >> 16);
      }
      stage_digits(0, wi >> 2, wi & 3, a, b, xd, xf, nch);
    }
  }
  if constexpr (NORM) {
    const float v = wave_sum(ss);
    if (lane == 0) rss[wave] = v;
  }
  __syncthreads();

  float acc[2][1] = {{0.f}, {0.f}};
#pragma unroll
  for (int j = 0; j < CPS; ++j) {
    const int c = c0 + lane + 64 * j;
    if (c < c1) {
      const uint4 wr[2] = {w[j][0], w[j][1]};
      const uint16_t s16[2] = {(uint16_t)(sc[j][0] >> sh[j][0]), (uint16_t)(sc[j][1] >> sh[j][1])};
      chunk_dot<2, 1>(xd, xf, nch, c, wr, s16, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const float v = wave_sum(acc[r][0]);
    if (lane == 0) red[ks][2 * rp + r] = v;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int o = blockIdx.x * kRows + threadIdx.x;
    if (o < n_out) {
      float rs = 1.f;
      if constexpr (NORM) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) t += rss[q];
        rs = 1.0f / sqrtf(t / (float)k + eps);
      }
      if constexpr (MODE == kGateUp) {
        float g = red[0][2 * threadIdx.x], u = red[0][2 * threadIdx.x + 1];
#pragma unroll
        for (int q = 1; q < KS; ++q) {
          g += red[q][2 * threadIdx.x];
          u += red[q][2 * threadIdx.x + 1];
        }
        y[o] = silu(g * rs) * (u * rs);
      } else {
        float v = red[0][threadIdx.x];
#pragma unroll
        for (int q = 1; q < KS; ++q) v += red[q][threadIdx.x];
        y[o] = MODE == kAdd ? yres + v * rs : v * rs;
      }
    }
  }
}

// K slices a workgroup of the 16-wave form (0: not used), over n_out outputs: 2 at K = 4096, 4 from K = 8192 (64
// chunks a slice, one per lane) for at most 4096 outputs (512 workgroups) and K <= 16384; 1 for 8192 to 32768
// outputs over K <= 4096 (256 to 1024 workgroups of 32 outputs), and for gate|up products of 4096 to 16384 outputs
// over K <= 4096 (256 to 1024 workgroups of 16 outputs).
inline int gemv_k_slices(int64_t n_out, int64_t k, bool gate_up) {
  if (gate_up) return k <= 4096 && n_out >= 4096 && n_out <= 16384 ? 1 : 0;
  if (k <= 4096 && n_out >= 8192 && n_out <= 32768) return 1;
  if (n_out > 4096 || k < 4096 || k > 16384) return 0;
  return k < 8192 ? 2 : 4;
}

template <int KS, int MODE>
static int launch_ks(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                     int f, const uint16_t* norm, float eps, hipStream_t s) {
  const int cps = ((k / 32 + KS - 1) / KS + 63) / 64;  // chunks a lane
  const size_t lds = (size_t)k / 32 * 100;               // xd: 6 x 16 B a chunk; xf: 4 B
  const int rows = (MODE == kGateUp ? 16 : 32) / KS;    // outputs a workgroup
  const dim3 grid((unsigned)((n_out + rows - 1) / rows)), block(1024);
  const int gsh = __builtin_ctz(group);
  auto go = [&](auto kern) -> int {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return AQ_ERR_CAPACITY;
    hipLaunchKernelGGL(kern, grid, block, lds, s, wq, ws, x, y, n_out, k, gsh, f, norm, eps);
    return launch_status();
  };
  if (norm) {
    if (cps == 1) return go(k_gemv_q4_ks<KS, 1, MODE, true>);
    if (cps == 2) return go(k_gemv_q4_ks<KS, 2, MODE, true>);
  } else {
    if (cps == 1) return go(k_gemv_q4_ks<KS, 1, MODE, false>);
    if (cps == 2) return go(k_gemv_q4_ks<KS, 2, MODE, false>);
  }
  return AQ_ERR_SHAPE;
}

// Workgroups of a launch over n_out outputs, RO per wave: one pass of 4 waves each, at most 1024 (then grid-stride).
// Workgroups of a row-block GEMV launch: one row block a wave while that takes at most 1536 workgroups (six waves a
// SIMD), else 1024, each wave striding over several. A cap of 1024 for every size left the MoE decode gate|up (1536 row
// blocks) with one or two a wave: 14.4 -> 13.3 us for the C3 token with one each; a 1280 or 1536 cap for the lm_head
// (8016 row blocks) measured 32.8 and 34.0 us against 31.7.
inline int gemv_blocks(int64_t n_out, int ro) {
  const int64_t b = (n_out + 4 * ro - 1) / (4 * ro);
  return b <= 1536 ? (int)b : 1024;
}

template <bool G32, int R, int T, int MODE, int D, int XR>
static int launch_d(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, const Fuse& fz, hipStream_t s) {
  constexpr int RO = (MODE == kGateUp || MODE == kMoeGateUp) ? R / 2 : R;
  const size_t lds = (size_t)T * k * sizeof(float) + (size_t)T * (k / 8) * sizeof(float);
  auto kern = k_gemv_q4<G32, R, T, MODE, D, XR>;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return AQ_ERR_CAPACITY;
  }
  const int blocks = gemv_blocks(n_out, RO);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, wq, ws, x, y, n_out, k, group, f, tokens, moe, fz);
  return launch_status();
}

// x in registers (XR words per thread) for one token of x (not split-attention states) with K <= 8192.
template <bool G32, int R, int T, int MODE, int D>
static int launch_x(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, const Fuse& fz, hipStream_t s) {
  if constexpr (T == 1 && MODE != kMoeDown) {
    if constexpr (MODE == kAdd && G32) {  // the attention output projection
      if (fz.parts && k <= 2048) return launch_d<G32, R, T, MODE, D, -1>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
    }
    if (!fz.parts && k <= 2048) return launch_d<G32, R, T, MODE, D, 1>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
    if (!fz.parts && k <= 8192) return launch_d<G32, R, T, MODE, D, 4>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  }
  return launch_d<G32, R, T, MODE, D, 0>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
}

// Pipeline depth of the dense G32 modes: the chunks one wave streams (per lane: K/2048 per row block, times its row
// blocks), at most 2 register sets of 4 rows or 4 of 2. One chunk (most decode shapes) runs unpipelined.
template <bool G32, int R, int T, int MODE>
static int launch_t(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, const Fuse& fz, hipStream_t s) {
  constexpr bool kDeep = G32 && (MODE == kStore || MODE == kAdd || MODE == kGateUp || MODE == kMoeGateUp);
  if constexpr (kDeep) {
    constexpr int RO = (MODE == kGateUp || MODE == kMoeGateUp) ? R / 2 : R;
    const int64_t waves = 4 * (int64_t)gemv_blocks(n_out, RO);
    const int64_t items = ((k / 32 + 63) / 64) * ((n_out + waves * RO - 1) / (waves * RO));
    if constexpr (R <= 2) {  // four register sets only for one or two rows a wave (not built otherwise)
      if (items >= 4) return launch_x<G32, R, T, MODE, 4>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
    }
    if (items >= 2) return launch_x<G32, R, T, MODE, 2>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  }
  return launch_x<G32, R, T, MODE, 1>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
}

// Weight rows per wave iteration. Measured on MI355X (G = 32, K = 2048): R = 2 is fastest while the matrix has fewer
// than 16K rows (N = 5120: 4.5 us vs 5.3 us at R = 4; N = 8192: 5.0 vs 5.5 us; N = 2048, K = 8192: 7.6 vs 9.9 us),
// R = 4 from 16K rows on (N = 16384: 7.3 vs 7.4 us; N = 128256: 35.3 vs 38.1 us). kMoeDown reads one row per expert
// slot for each output instead.
inline int rows_per_wave(int64_t rows) { return rows < 16384 ? 2 : 4; }

template <bool G32, int T, int MODE>
static int launch_r(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, const Fuse& fz, hipStream_t s) {
  if constexpr (MODE == kMoeDown) {
    return launch_t<G32, 1, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  } else {
    const int64_t rows = (MODE == kGateUp || MODE == kMoeGateUp) ? 2 * (int64_t)n_out : n_out;
    if (rows_per_wave(rows) == 2) return launch_t<G32, 2, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
    return launch_t<G32, 4, T, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  }
}

template <bool G32, int MODE>
static int launch_g(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int n_out, int k, int group,
                    int f, int tokens, const MoeArgs& moe, const Fuse& fz, hipStream_t s) {
  if (tokens <= 1) return launch_r<G32, 1, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  if (tokens <= 2) return launch_r<G32, 2, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  if (tokens <= 4) return launch_r<G32, 4, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  if constexpr (MODE == kStore || MODE == kAdd) {  // few-row products up to 16 rows (speculative verify)
    if (tokens > 8) return launch_r<G32, 16, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
  }
  return launch_r<G32, 8, MODE>(wq, ws, x, y, n_out, k, group, f, tokens, moe, fz, s);
}

template <int MODE>
static int gemv_entry(const uint32_t* wq, const uint16_t* ws, const float* x, float* y, int64_t n_out, int64_t k,
                      int32_t group, int64_t f, int32_t tokens, const MoeArgs& moe, void* stream,
                      const Fuse& fz = Fuse{nullptr, 0.f, nullptr, 0, {}}) {
  if (!wq || !ws || !x || !y) return AQ_ERR_NULL;
  if (fz.norm && !aligned(fz.norm, 16)) return AQ_ERR_ALIGN;
  const int max_tokens = (MODE == kStore || MODE == kAdd) ? 16 : 8;
  if (n_out <= 0 || k <= 0 || tokens < 1 || tokens > max_tokens) return AQ_ERR_SHAPE;
  if (k % 32) return AQ_ERR_SHAPE;
  if (group <= 0 || group % 8 || k % group) return AQ_ERR_GROUP;
  const int tp = tokens <= 1 ? 1 : tokens <= 2 ? 2 : tokens <= 4 ? 4 : tokens <= 8 ? 8 : 16;
  if ((int64_t)tp * k > 32768) return AQ_ERR_CAPACITY;
  if (n_out > (int64_t)1 << 30) return AQ_ERR_SHAPE;
  // W, its scales and y are addressed through 32-bit buffer offsets below 2 GiB
  const int64_t wrows = (MODE == kGateUp || MODE == kMoeGateUp) ? 2 * n_out : n_out;
  if (wrows * k / 2 >= ((int64_t)1 << 31) || (int64_t)tokens * n_out * 4 >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;
  if (!aligned(wq, 16) || !aligned(x, 16)) return AQ_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool g32 = group >= 32 && (group & (group - 1)) == 0;
  if constexpr (MODE == kStore || MODE == kAdd || MODE == kGateUp) {
    if (g32 && tokens == 1 && !fz.step.cand && !fz.parts) {
      const int ks = gemv_k_slices(n_out, k, MODE == kGateUp);
      const int fi = (int)f;
      if (ks == 1) return launch_ks<1, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, fi, fz.norm, fz.eps, s);
      if (ks == 2) return launch_ks<2, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, fi, fz.norm, fz.eps, s);
      if (ks == 4) return launch_ks<4, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, fi, fz.norm, fz.eps, s);
    }
  }
  if (g32)
    return launch_g<true, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, moe, fz, s);
  return launch_g<false, MODE>(wq, ws, x, y, (int)n_out, (int)k, group, (int)f, tokens, moe, fz, s);
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
  // the kernel reads the stacked experts' rows through one buffer resource with 32-bit offsets (their scales, at
  // group >= 8, take fewer bytes than the words)
  if (k > 0 && experts * 2 * f * (k / 2) >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;
  const aq::MoeArgs moe{ids, nullptr, (int)experts, 0};
  return aq::gemv_entry<aq::kMoeGateUp>(wq, ws, x, a, topk * f, k, group, f, 1, moe, stream);
}

extern "C" int aq_moe_down_q4(const uint32_t* wq, const uint16_t* ws, int64_t experts, const int32_t* ids,
                              const float* weights, const float* act, float* y, int64_t d, int64_t f, int32_t group,
                              int32_t topk, int32_t add, void* stream) {
  if (!ids || !weights) return AQ_ERR_NULL;
  if (topk <= 0 || topk > 8 || d <= 0 || experts <= 0 || experts * d > INT32_MAX) return AQ_ERR_SHAPE;
  if (f > 0 && experts * d * (f / 2) >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;  // stacked W below 2 GiB
  if (aq::moe_down_dec_ok(f, group, topk) && f % group == 0) {  // one wave per expert slot, 8 lanes a row
    if (!wq || !ws || !act || !y) return AQ_ERR_NULL;
    if (!aq::aligned(wq, 16) || !aq::aligned(act, 16)) return AQ_ERR_ALIGN;
    return aq::launch_moe_down_dec(wq, ws, ids, weights, act, y, d, f, group, (int32_t)experts, topk, add,
                                   reinterpret_cast<hipStream_t>(stream));
  }
  // other groups and wider f: the expert slots are the GEMV's "tokens", act [topk, f] one activation vector per slot
  const aq::MoeArgs moe{ids, weights, (int)experts, add ? 1 : 0};
  return aq::gemv_entry<aq::kMoeDown>(wq, ws, act, y, d, f, group, 0, topk, moe, stream);
}

extern "C" int aq_rmsnorm_gemv_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w,
                                  float eps, float* y, int64_t n, int64_t k, int32_t group, int32_t tokens,
                                  void* stream) {
  if (!norm_w) return AQ_ERR_NULL;
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  return aq::gemv_entry<aq::kStore>(wq, ws, x, y, n, k, group, 0, tokens, none, stream, aq::Fuse{norm_w, eps, nullptr, 0, {}});
}

extern "C" int aq_rmsnorm_gate_up_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w,
                                     float eps, float* a, int64_t f, int64_t k, int32_t group, int32_t tokens,
                                     void* stream) {
  if (!norm_w) return AQ_ERR_NULL;
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  return aq::gemv_entry<aq::kGateUp>(wq, ws, x, a, f, k, group, f, tokens, none, stream,
                                     aq::Fuse{norm_w, eps, nullptr, 0, {}});
}

extern "C" int aq_head_argmax_q4(const uint32_t* wq, const uint16_t* ws, const float* x, const uint16_t* norm_w,
                                 float eps, float* logits, int64_t vocab, int64_t k, int32_t group, uint64_t* cand,
                                 int64_t cand_cap, int32_t* token, int32_t* pos, int32_t* hist, int32_t hist_cap,
                                 int32_t advance, void* stream) {
  if (vocab <= 0 || vocab > (int64_t)1 << 30) return AQ_ERR_SHAPE;
  // one key per workgroup, then the arrival counters
  aq::Fuse fz{norm_w, eps, nullptr, 0, {}};
  const int st = aq::make_step_end(cand, cand_cap, aq::gemv_blocks(vocab, aq::rows_per_wave(vocab)), token, pos, hist,
                                   hist_cap, advance, fz.step);
  if (st != AQ_OK) return st;
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  return aq::gemv_entry<aq::kStore>(wq, ws, x, logits, vocab, k, group, 0, 1, none, stream, fz);
}

extern "C" int aq_attn_out_q4(const uint32_t* wq, const uint16_t* ws, const float* parts, int32_t splits, float* y,
                              int64_t n, int64_t k, int32_t group, void* stream) {
  if (!parts) return AQ_ERR_NULL;
  if (splits < 1 || splits > AQ_ATTN_MAX_SPLITS || k % 64) return AQ_ERR_SHAPE;
  if (!aq::aligned(parts, 16)) return AQ_ERR_ALIGN;
  const aq::MoeArgs none{nullptr, nullptr, 0, 0};
  // x is not read (the partial states stand for it); parts is passed as x for the pointer checks
  return aq::gemv_entry<aq::kAdd>(wq, ws, parts, y, n, k, group, 0, 1, none, stream,
                                  aq::Fuse{nullptr, 0.f, parts, splits, {}});
}
