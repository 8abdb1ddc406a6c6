// Ternary (T2W) matrix-vector products and the fp16-pair (X2H) producers, gfx950.
//
// Arithmetic: y[n] = sum over 128-groups g of s[g, n] * sum_{k in g} (code(k, n) - 1) * x[k], codes of T2W words
// (uint32 [K/16, N], code of (n, k) in bits 2*(k%16) of word (k/16)*N + n), x given as fp16 pairs. This is
// bonsai/kernels/kernels.mojo:189-325 (``_group_dot8`` / ``packed_linear``) and :437-448 (``packed_reduce``); the
// reference accumulates each group in fp16 chains, this build decodes exactly and accumulates in fp32.
//
// Decode (HBM-bound: 0.27 B per weight, so ~1.5 VALU ops per weight is the budget). Two forms:
// - biased (t2_word_dot_b; the GEMVs k_t2_gemv_cols and k_t2_gemv_wide, and so the output head): four shifts of the
//   word bring each pair of code positions to bits 6-9 of both halves, one v_bitop3 per pair fills the rest with the
//   exponent of 16.0 or 4.0, giving the exact fp16 pair (B + c, B + c'); v_dot2_f32_f16 with the unscaled x pair sums
//   (B + c) x with exact products, and a per-128-group bias sum (B + 1) x, staged with x, is subtracted. 56 issue
//   cycles per 16 weights.
// - exact (t2_word_dot; k_t2_partials, the packed_linear drop-in): for code position j <= 4 of a 16-bit half,
//   (word & (0x00030003 << 2j)) | 0x64006400 is the fp16 pair (1024 + c_j * 4^j, 1024 + c_{j+8} * 4^j); subtracting
//   1024 + 4^j leaves (c - 1) * 4^j exactly, and v_dot2_f32_f16 against the x pair pre-scaled by 4^-j accumulates
//   (c - 1) * x in fp32. Positions 5..7 are the same after one shift by 10. No bias to cancel.
#include "aq_common.h"
#include "aq_step_end.h"

namespace aq {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Scale of the x pair used with code position j (0..7) of a 16-bit half.
__device__ __forceinline__ float t2_xscale(int j) {
  const int e = j <= 4 ? j : j - 5;
  return 1.0f / (float)(1 << (2 * e));
}

// sum_{j<16} (code_j - 1) * x_j for one T2W word; xp[j] = fp16 pair (x[j], x[j+8]) * 4^-e(j).
__device__ __forceinline__ float t2_word_dot(uint32_t w, const uint32_t* xp, float acc) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = j <= 4 ? j : j - 5;
    const uint32_t src = j <= 4 ? w : (w >> 10);
    const uint32_t bits = (src & (0x00030003u << (2 * e))) | 0x64006400u;
    half2v h = __builtin_bit_cast(half2v, bits);
    const _Float16 bias = (_Float16)(1024.0f + (float)(1 << (2 * e)));
    h = h - half2v{bias, bias};
    acc = __builtin_amdgcn_fdot2(h, __builtin_bit_cast(half2v, xp[j]), acc, false);
  }
  return acc;
}

// t2_word_dot with the fp16-pair exponent bits 0x64006400 passed in a VGPR (magic), so each mask-and-OR is one
// v_and_or_b32 instead of an AND and an OR with a literal.
__device__ __forceinline__ float t2_word_dot_m(uint32_t w, const uint32_t* xp, float acc, uint32_t magic) {
  const uint32_t hi = w >> 10;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = j <= 4 ? j : j - 5;
    const uint32_t bits = ((j <= 4 ? w : hi) & (0x00030003u << (2 * e))) | magic;
    const _Float16 bias = (_Float16)(1024.0f + (float)(1 << (2 * e)));
    const half2v h = __builtin_bit_cast(half2v, bits) - half2v{bias, bias};
    acc = __builtin_amdgcn_fdot2(h, __builtin_bit_cast(half2v, xp[j]), acc, false);
  }
  return acc;
}

// Biased decode (the faster form; gfx950 issues v_bitop3_b32 and shifts at twice the rate of v_and_or_b32 and
// v_pk_add_f16). The word is shifted so that code positions p = 2i, 2i + 1 (i < 4) land at bits 6-7 and 8-9 of both
// halves (w << 6, << 2, >> 2, >> 6); one v_bitop3 per pair keeps those bits and fills the rest from 0x4C00 (16.0) or
// 0x4400 (4.0), giving the exact fp16 pair (16 + c, 16 + c') for even p and (4 + c, 4 + c') for odd p. Their
// v_dot2_f32_f16 with the unscaled x pair (x[p], x[p + 8]) sums (B_k + c_k) x_k; the caller subtracts the staged bias
// sum_k (B_k + 1) x_k (B_k = 16 for even k % 8, else 4), leaving sum_k (c_k - 1) x_k. 56 issue cycles per word
// against 98 for t2_word_dot_m.
__device__ __forceinline__ uint32_t t2_pick(uint32_t a, uint32_t magic, uint32_t mask) {
  return __builtin_amdgcn_bitop3_b32(a, magic, mask, 0xE4);  // mask ? a : magic, bit by bit
}

__device__ __forceinline__ float t2_word_dot_b(uint32_t w, const uint32_t* xp, float acc, uint32_t m16, uint32_t m4) {
  const uint32_t sh[4] = {w << 6, w << 2, w >> 2, w >> 6};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, t2_pick(sh[i], m16, 0x00C000C0u)),
                                 __builtin_bit_cast(half2v, xp[2 * i]), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, t2_pick(sh[i], m4, 0x03000300u)),
                                 __builtin_bit_cast(half2v, xp[2 * i + 1]), acc, false);
  }
  return acc;
}

// Weight of x_k in the biased decode's bias: B_k + 1 for pair position p = k % 8.
__device__ __forceinline__ float t2_bias_weight(int p) { return (p & 1) ? 5.0f : 17.0f; }

// One k-row's x pairs (x[16 r + p], x[16 r + p + 8]) from its 16 fp16 (xl: x[16 r .. + 8), xh: x[16 r + 8 .. + 16)),
// and its share of the biased decode's bias, sum_p (B_p + 1) (x[16 r + p] + x[16 r + p + 8]).
__device__ __forceinline__ float t2_row_pairs(uint4 xl, uint4 xh, uint32_t (&pr)[8]) {
  const uint32_t lo[4] = {xl.x, xl.y, xl.z, xl.w}, hi[4] = {xh.x, xh.y, xh.z, xh.w};
  float bias = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    pr[2 * m] = (lo[m] & 0xFFFFu) | (hi[m] << 16);
    pr[2 * m + 1] = (lo[m] >> 16) | (hi[m] & 0xFFFF0000u);
    bias = fmaf(t2_bias_weight(2 * m), half_bits_to_float((uint16_t)lo[m]) + half_bits_to_float((uint16_t)hi[m]),
                bias);
    bias = fmaf(t2_bias_weight(2 * m + 1),
                half_bits_to_float((uint16_t)(lo[m] >> 16)) + half_bits_to_float((uint16_t)(hi[m] >> 16)), bias);
  }
  return bias;
}

// Stages x (X2H words, K/2 of them) for t2_word_dot_b: xs[8 r + p] = the pairs of k-row r, gbias[g] = the bias of
// 128-group g. Thread t of nthreads (a multiple of 64) takes rows t, t + nthreads, ...; a group is 8 consecutive
// rows, i.e. 8 consecutive threads, all staging or all idle (krows % 8 == 0), summed by DPP.
__device__ __forceinline__ void t2_stage_x(const uint32_t* __restrict__ x2h, uint32_t* xs, float* gbias, int krows,
                                           int t, int nthreads) {
  for (int r = t; r < krows; r += nthreads) {
    const uint4* row = reinterpret_cast<const uint4*>(x2h + r * 8);
    uint32_t pr[8];
    const float bias = sum8(t2_row_pairs(row[0], row[1], pr));
    *reinterpret_cast<uint4*>(xs + r * 8) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    *reinterpret_cast<uint4*>(xs + r * 8 + 4) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
    if ((r & 7) == 0) gbias[r >> 3] = bias;
  }
}

// The reference's split interface (packed_linear): workgroup (column tile ct, split sp) covers columns [256 ct, +256)
// (lane l -> columns 4l..4l+3, all four waves) and k-rows [sp * krows_wg, +krows_wg) (1024 k), divided among the four
// waves in whole 128-groups, and writes partial[sp][n].
template <bool VEC4>
__global__ __launch_bounds__(256) void k_t2_partials(const uint32_t* __restrict__ x2h, const uint32_t* __restrict__ w,
                                                     const uint16_t* __restrict__ sc, float* __restrict__ part, int N,
                                                     int K, int krows_wg, int splits) {
  extern __shared__ uint32_t xs[];  // [krows_wg][8] scaled x pairs, then [4][256] floats for the wave reduction
  float* red = reinterpret_cast<float*>(xs + krows_wg * 8);
  const int ct = blockIdx.x / splits;
  const int sp = blockIdx.x - ct * splits;
  const int kr0 = sp * krows_wg;
  const int krows_total = K >> 4;
  const int nrows = min(krows_wg, krows_total - kr0);

  // x' for this workgroup's k-rows: pair j of row r = (x[16r + j], x[16r + j + 8]) * 4^-e(j)
  for (int i = threadIdx.x; i < nrows * 8; i += 256) {
    const int r = i >> 3, j = i & 7;
    const int k = (kr0 + r) * 16 + j;
    const uint32_t lo = x2h[k >> 1], hi = x2h[(k + 8) >> 1];
    const float a = half_bits_to_float((uint16_t)(k & 1 ? lo >> 16 : lo & 0xFFFF));
    const float b = half_bits_to_float((uint16_t)((k + 8) & 1 ? hi >> 16 : hi & 0xFFFF));
    const float f = t2_xscale(j);
    xs[i] = (uint32_t)float_to_half_bits(a * f) | ((uint32_t)float_to_half_bits(b * f) << 16);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int n0 = ct * 256 + lane * 4;
  const int groups = (nrows + 7) >> 3;              // 128-groups in this workgroup
  const int gpw = (groups + 3) >> 2;                // groups per wave
  const int g0 = wave * gpw, g1 = min(groups, g0 + gpw);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(w), (short)0,
                                                                      (int)min((size_t)krows_total * N * 4,
                                                                               (size_t)0x7FFFFFFF),
                                                                      0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(sc), (short)0,
                                                                       (int)((size_t)(K >> 7) * N * 2), 0x00020000);
  float tot[4] = {0.f, 0.f, 0.f, 0.f};
  for (int g = g0; g < g1; ++g) {
    const int r0 = g * 8;
    uint4 wv[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t row = (uint32_t)(kr0 + r0 + r);
      if constexpr (VEC4) {
        const uint32_t off = n0 < N ? (row * (uint32_t)N + n0) * 4 : 0x80000000u;
        wv[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, kWPolicy));
      } else {
        uint32_t v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t off = n0 + c < N ? (row * (uint32_t)N + n0 + c) * 4 : 0x80000000u;
          v[c] = __builtin_amdgcn_raw_buffer_load_b32(wr, off, 0, kWPolicy);
        }
        wv[r] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    }
    float s4[4];
    const uint32_t grow = (uint32_t)((kr0 + r0) >> 3);  // 128-group index
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t off = n0 + c < N ? (grow * (uint32_t)N + n0 + c) * 2 : 0x80000000u;
      s4[c] = half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(srs, off, 0, 0));
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      uint32_t xp[8];
      *reinterpret_cast<uint4*>(xp) = *reinterpret_cast<const uint4*>(xs + (r0 + r) * 8);
      *reinterpret_cast<uint4*>(xp + 4) = *reinterpret_cast<const uint4*>(xs + (r0 + r) * 8 + 4);
      acc[0] = t2_word_dot(wv[r].x, xp, acc[0]);
      acc[1] = t2_word_dot(wv[r].y, xp, acc[1]);
      acc[2] = t2_word_dot(wv[r].z, xp, acc[2]);
      acc[3] = t2_word_dot(wv[r].w, xp, acc[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) tot[c] = fmaf(acc[c], s4[c], tot[c]);
  }

  // waves -> one partial per column (wave order)
  *reinterpret_cast<float4*>(red + (wave * 256 + lane * 4)) = make_float4(tot[0], tot[1], tot[2], tot[3]);
  __syncthreads();
  const int n = ct * 256 + threadIdx.x;
  float v = ((red[threadIdx.x] + red[256 + threadIdx.x]) + red[512 + threadIdx.x]) + red[768 + threadIdx.x];
  if (n < N) part[(size_t)sp * N + n] = v;
}

// Fused ternary GEMV without any cross-workgroup step. A 512-thread workgroup owns CB consecutive columns over all
// of K: lane l takes column l % CB and phase l / CB of its wave; the 8 * 64 / CB phases split the k-rows into
// contiguous runs of whole 128-groups, so a load instruction reads CB consecutive words of 64/CB rows. Phase partials
// are summed in phase order through LDS (deterministic). x pairs and the per-group biases of t2_word_dot_b are
// staged in LDS once.
template <int CB>
// step.cand != NULL: the launch also ends the greedy step (step_end), each workgroup's key the first maximum of its
// CB outputs (kNonFiniteKey if any of them is NaN or infinite).
__global__ __launch_bounds__(512) void k_t2_gemv_cols(const uint32_t* __restrict__ x2h, const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ sc, float* __restrict__ y, int N,
                                                      int K, StepEnd step) {
  constexpr int PH = 8 * 64 / CB;  // phases per workgroup
  extern __shared__ uint32_t xs[];   // [K/16][8] x pairs (x[16 r + p], x[16 r + p + 8]), then [K/128] group biases
  __shared__ float red[PH][CB];
  const int krows = K >> 4;
  float* gbias = reinterpret_cast<float*>(xs + krows * 8);
  t2_stage_x(x2h, xs, gbias, krows, threadIdx.x, 512);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int c = lane % CB;
  const int ph = wave * (64 / CB) + lane / CB;
  const int n = blockIdx.x * CB + c;
  const int groups = krows >> 3;  // 128-groups
  const int g0 = (int)(((long)groups * ph) / PH), g1 = (int)(((long)groups * (ph + 1)) / PH);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(w), (short)0, (int)min((size_t)krows * N * 4, (size_t)0x7FFFFFFF), 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(sc), (short)0,
                                                                       (int)((size_t)groups * N * 2), 0x00020000);
  uint32_t m16, m4;  // the fp16-pair fill patterns in VGPRs (the masks take the one scalar operand)
  asm volatile("v_mov_b32 %0, 0x4c004c00" : "=v"(m16));
  asm volatile("v_mov_b32 %0, 0x44004400" : "=v"(m4));
  const bool col_ok = n < N;
  float tot = 0.f;
  for (int g = g0; g < g1; ++g) {
    uint32_t wv[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
      wv[r] = __builtin_amdgcn_raw_buffer_load_b32(wr, col_ok ? ((uint32_t)(g * 8 + r) * N + n) * 4 : 0x80000000u, 0,
                                                   kWPolicy);
    const float s = half_bits_to_float(
        __builtin_amdgcn_raw_buffer_load_b16(srs, col_ok ? ((uint32_t)g * N + n) * 2 : 0x80000000u, 0, 0));
    float acc0 = -gbias[g], acc1 = 0.f;  // two chains: even and odd rows
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      uint32_t xp[8];
      *reinterpret_cast<uint4*>(xp) = *reinterpret_cast<const uint4*>(xs + (g * 8 + r) * 8);
      *reinterpret_cast<uint4*>(xp + 4) = *reinterpret_cast<const uint4*>(xs + (g * 8 + r) * 8 + 4);
      if (r & 1) acc1 = t2_word_dot_b(wv[r], xp, acc1, m16, m4);
      else acc0 = t2_word_dot_b(wv[r], xp, acc0, m16, m4);
    }
    tot = fmaf(acc0 + acc1, s, tot);
  }
  red[ph][c] = tot;
  __syncthreads();
  if (threadIdx.x < CB && blockIdx.x * CB + (int)threadIdx.x < N) {
    float v = 0.f;
#pragma unroll
    for (int p = 0; p < PH; ++p) v += red[p][threadIdx.x];
    y[blockIdx.x * CB + threadIdx.x] = v;
    if (step.cand) red[0][threadIdx.x] = v;  // each thread rereads only its own column: no barrier needed before this
  }
  if (step.cand) {  // workgroup-uniform
    __syncthreads();
    if (threadIdx.x < 64) {
      uint64_t key = 0;
      if (threadIdx.x == 0) {
        const int c0 = blockIdx.x * CB, cols = min(CB, N - c0);
        float best = red[0][0];
        int bi = 0;
        bool bad = !__builtin_isfinite(best);
        for (int j = 1; j < cols; ++j) {
          if (red[0][j] > best) best = red[0][j], bi = j;
          bad |= !__builtin_isfinite(red[0][j]);
        }
        key = bad ? kNonFiniteKey : argmax_key(best, c0 + bi);
      }
      step_end(step, key);
    }
  }
}

// Wide matrices (a vocabulary head: many columns, K <= 16384): a 256-thread workgroup owns 256 consecutive columns
// over all of K (lane l: columns 4 l .. 4 l + 3, one 16-byte load per k-row); wave w takes the 128-groups w, w + 4,
// ... Wave partials are summed in wave order through LDS. step.cand != NULL: the launch also ends the greedy step
// (step_end), each workgroup's key the first maximum of its columns (kNonFiniteKey if any of them is NaN or
// infinite). N % 4 == 0.
__global__ __launch_bounds__(256) void k_t2_gemv_wide(const uint32_t* __restrict__ x2h, const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ sc, float* __restrict__ y, int N,
                                                      int K, StepEnd step) {
  constexpr int CPL = 4, COLS = 256;
  extern __shared__ uint32_t xs[];  // [K/16][8] x pairs (x[16 r + p], x[16 r + p + 8]), then [K/128] group biases
  __shared__ float red[4][COLS];
  const int krows = K >> 4;
  const int lane = threadIdx.x & 63, wave = wave_id();
  float* gbias = reinterpret_cast<float*>(xs + krows * 8);
  const int n0 = blockIdx.x * COLS + lane * CPL;
  const bool ok = n0 < N;
  const int groups = krows >> 3;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)krows * N * 4));
  const auto sr = make_rsrc(sc, (uint32_t)((size_t)groups * N * 2));
  auto issue = [&](int g, uint4 (&wv)[8], uint32_t (&s)[2]) {
    const bool v = ok && g < groups;
#pragma unroll
    for (int r = 0; r < 8; ++r) wv[r] = buf_load16p<kWPolicy>(wr, v ? ((uint32_t)(g * 8 + r) * N + n0) * 4 : kOOB);
    const uint2 t = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(sr, v ? ((uint32_t)g * N + n0) * 2 : kOOB, 0, 0));
    s[0] = t.x, s[1] = t.y;
  };
  // x: thread r stages k-row r (two 16-byte loads of x2h: x[16 r .. 16 r + 8) and x[16 r + 8 .. 16 r + 16)); the
  // first round's loads are issued before the weights, so waiting for them does not wait for the weights
  const auto xr = make_rsrc(x2h, (uint32_t)K * 2);
  uint4 xlo = buf_load16(xr, (int)threadIdx.x < krows ? threadIdx.x * 32 : kOOB);
  uint4 xhi = buf_load16(xr, (int)threadIdx.x < krows ? threadIdx.x * 32 + 16 : kOOB);
  // two register sets in turn (no copies, which would wait for the loads in flight), both filled before x is staged
  // (the weights do not depend on it): one group's words are used while the next ones load. Both sets are used
  // unconditionally (a condition would let the compiler move their loads down to their use); past the last group
  // the loads return zero, and a zero scale adds nothing.
  uint4 wa[8], wb[8];
  uint32_t sa[2], sb[2];
  issue(wave, wa, sa);
  issue(wave + 4, wb, sb);
  // row r's pairs (x[16 r + p], x[16 r + p + 8]) and its bias sum_p (B_p + 1) (x[16 r + p] + x[16 r + p + 8]); a
  // 128-group is 8 consecutive rows, i.e. 8 consecutive threads, all staging or all idle (krows % 8 == 0). The
  // first round runs on every thread (rows past the end loaded zeros and store nothing), so its loads stay ahead of
  // the weights'.
  auto stage = [&](int r, uint4 xl, uint4 xh) {
    uint32_t pr[8];
    float bias = t2_row_pairs(xl, xh, pr);
    bias = sum8(bias);
    if (r < krows) {
      *reinterpret_cast<uint4*>(xs + r * 8) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
      *reinterpret_cast<uint4*>(xs + r * 8 + 4) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
      if ((r & 7) == 0) gbias[r >> 3] = bias;
    }
  };
  stage(threadIdx.x, xlo, xhi);
  for (int r = threadIdx.x + 256; r < krows; r += 256) stage(r, buf_load16(xr, r * 32), buf_load16(xr, r * 32 + 16));
  __syncthreads();
  uint32_t m16, m4;  // the fp16-pair fill patterns in VGPRs (the masks take the one scalar operand)
  asm volatile("v_mov_b32 %0, 0x4c004c00" : "=v"(m16));
  asm volatile("v_mov_b32 %0, 0x44004400" : "=v"(m4));
  float tot[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) tot[c] = 0.f;
  auto compute = [&](int g, const uint4 (&wv)[8], const uint32_t (&s)[2]) {
    // past the last group (its loads returned zero, scale 0) any staged group's x keeps the sum finite
    const int gx = g < groups ? g : 0;
    const float b0 = -gbias[gx];
    float acc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[c] = b0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      uint32_t xp[8];
      *reinterpret_cast<uint4*>(xp) = *reinterpret_cast<const uint4*>(xs + (gx * 8 + r) * 8);
      *reinterpret_cast<uint4*>(xp + 4) = *reinterpret_cast<const uint4*>(xs + (gx * 8 + r) * 8 + 4);
      const uint32_t* words = reinterpret_cast<const uint32_t*>(&wv[r]);
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c] = t2_word_dot_b(words[c], xp, acc[c], m16, m4);
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      tot[c] = fmaf(acc[c], half_bits_to_float((uint16_t)(s[c >> 1] >> (16 * (c & 1)))), tot[c]);
  };
  for (int g = wave; g < groups; g += 8) {
    compute(g, wa, sa);
    issue(g + 8, wa, sa);
    compute(g + 4, wb, sb);
    issue(g + 12, wb, sb);
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) red[wave][lane * CPL + c] = tot[c];
  __syncthreads();
  const int t = threadIdx.x, n = blockIdx.x * COLS + t;  // one column a thread
  const float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
  if (n < N) y[n] = v;
  if (step.cand) {  // workgroup-uniform
    const uint64_t key = n >= N ? 0ull : __builtin_isfinite(v) ? argmax_key(v, n) : kNonFiniteKey;
    workgroup_step_end<4>(step, wave_max_u64(key));
  }
}

// y[n] = sum_g partials[g][n] in g order (bonsai/kernels/kernels.mojo:437-448, packed_reduce).
__global__ __launch_bounds__(256) void k_t2_reduce(const float* __restrict__ part, float* __restrict__ y, int N,
                                                   int groups) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float acc = 0.f;
#pragma unroll 8
  for (int g = 0; g < groups; ++g) acc += part[(size_t)g * N + n];  // unrolled: eight partials requested together
  y[n] = acc;
}

// ---- X2H producers (qwen3/kernels/qwen3k.mojo:17-59) ----

__global__ void k_pack_half(const float* __restrict__ x, uint32_t* __restrict__ q, int64_t pairs) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < pairs; i += (int64_t)gridDim.x * 256)
    q[i] = (uint32_t)float_to_half_bits(x[2 * i]) | ((uint32_t)float_to_half_bits(x[2 * i + 1]) << 16);
}

// 16-byte aligned x and q: 8 floats -> 4 words a thread (two 16-byte loads, one 16-byte store); the tail of fewer than
// 8 floats goes to k_pack_half.
__global__ void k_pack_half8(const float4* __restrict__ x, uint4* __restrict__ q, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const float4 a = x[2 * i], b = x[2 * i + 1];
    uint4 o;
    o.x = (uint32_t)float_to_half_bits(a.x) | ((uint32_t)float_to_half_bits(a.y) << 16);
    o.y = (uint32_t)float_to_half_bits(a.z) | ((uint32_t)float_to_half_bits(a.w) << 16);
    o.z = (uint32_t)float_to_half_bits(b.x) | ((uint32_t)float_to_half_bits(b.y) << 16);
    o.w = (uint32_t)float_to_half_bits(b.z) | ((uint32_t)float_to_half_bits(b.w) << 16);
    q[i] = o;
  }
}

// One workgroup per row: q[row] = pack(x[row] / rms(x[row]) * w), eps as given.
__global__ __launch_bounds__(256) void k_rmsnorm_pack(const float* __restrict__ x, const float* __restrict__ w,
                                                      uint32_t* __restrict__ q, int n, float eps) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * n;
  uint32_t* qr = q + (size_t)blockIdx.x * (n / 2);
  float ss = 0.f;
#pragma unroll 8  // loads in flight together; the multiply-add order is unchanged
  for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)n + eps);
#pragma unroll 4
  for (int i = threadIdx.x; i < n / 2; i += 256)
    qr[i] = (uint32_t)float_to_half_bits(xr[2 * i] * r * w[2 * i]) |
            ((uint32_t)float_to_half_bits(xr[2 * i + 1] * r * w[2 * i + 1]) << 16);
}

// q[row] = pack(silu(gate) * up), rows of gu = gate (n) | up (n).
__global__ void k_swiglu_pack(const float* __restrict__ gu, uint32_t* __restrict__ q, int n, int rows) {
  const int64_t pairs = (int64_t)rows * (n / 2);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < pairs; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / (n / 2);
    const int c = (int)(i - row * (n / 2)) * 2;
    const float* g = gu + row * 2 * n;
    const float a = silu(g[c]) * g[n + c];
    const float b = silu(g[c + 1]) * g[n + c + 1];
    q[i] = (uint32_t)float_to_half_bits(a) | ((uint32_t)float_to_half_bits(b) << 16);
  }
}

static int t2_check(const void* x2h, const void* w, const void* s, int64_t n, int64_t k) {
  if (!x2h || !w || !s) return AQ_ERR_NULL;
  if (n <= 0 || k <= 0 || k % 128) return AQ_ERR_SHAPE;
  if (n > (1 << 26) || k > (1 << 24) || (k / 16) * n * 4 >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;
  if (!aligned(w, 16)) return AQ_ERR_ALIGN;
  return AQ_OK;
}

static int launch_t2_partials(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* part, int N, int K,
                              hipStream_t st) {
  const int krows_wg = 64;  // 1024 k
  const int splits = (K + 1023) / 1024;
  const int ctiles = (N + 255) / 256;
  const size_t lds = (size_t)krows_wg * 8 * 4 + 4 * 256 * 4;
  if (N % 4 == 0)
    hipLaunchKernelGGL(k_t2_partials<true>, dim3(ctiles * splits), dim3(256), lds, st, x2h, w, s, part, N, K, krows_wg,
                       splits);
  else
    hipLaunchKernelGGL(k_t2_partials<false>, dim3(ctiles * splits), dim3(256), lds, st, x2h, w, s, part, N, K,
                       krows_wg, splits);
  return launch_status();
}

}  // namespace aq

using namespace aq;

extern "C" int64_t aq_t2_gemv_workspace_bytes(int64_t n, int64_t k) {
  (void)n;
  (void)k;
  return 0;  // the fused kernel reduces inside each workgroup
}

namespace aq {
// Columns per workgroup: 256 (k_t2_gemv_wide) when that still gives >= 512 workgroups; else 32 (k_t2_gemv_cols)
// when that gives >= 256, else 16 (more workgroups, 64-byte segments).
inline int t2_cols_per_block(int64_t n, int64_t k) {
  if (n % 4 == 0 && (n + 255) / 256 >= 512 && k <= 16384) return 256;
  return (n + 31) / 32 >= 256 ? 32 : 16;
}

// Workgroups of the launch over N columns (also the argmax keys of a head launch).
inline int64_t t2_blocks(int64_t n, int64_t k) {
  const int cb = t2_cols_per_block(n, k);
  return (n + cb - 1) / cb;
}

static int launch_t2_gemv(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* y, int N, int K,
                          const StepEnd& step, hipStream_t sm) {
  // x staging: 8 pairs per 16-k row (2K bytes), then one bias per 128-group
  const size_t lds = (size_t)(K / 16) * 8 * 4 + (size_t)(K / 128) * 4;
  if (lds > 64 * 1024) return AQ_ERR_CAPACITY;
  const int cb = t2_cols_per_block(N, K);
  if (cb == 256)
    hipLaunchKernelGGL(k_t2_gemv_wide, dim3((unsigned)((N + 255) / 256)), dim3(256), lds, sm, x2h, w, s, y, N, K,
                       step);
  else if (cb == 32)
    hipLaunchKernelGGL(k_t2_gemv_cols<32>, dim3((unsigned)((N + 31) / 32)), dim3(512), lds, sm, x2h, w, s, y, N, K,
                       step);
  else
    hipLaunchKernelGGL(k_t2_gemv_cols<16>, dim3((unsigned)((N + 15) / 16)), dim3(512), lds, sm, x2h, w, s, y, N, K,
                       step);
  return launch_status();
}
}  // namespace aq

extern "C" int aq_t2_gemv(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* y, int64_t n, int64_t k,
                          void* workspace, int64_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  int st = t2_check(x2h, w, s, n, k);
  if (st) return st;
  if (!y) return AQ_ERR_NULL;
  return launch_t2_gemv(x2h, w, s, y, (int)n, (int)k, StepEnd{}, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int64_t aq_t2_head_candidates(int64_t n, int64_t k) {
  return n > 0 ? aq::t2_blocks(n, k) + AQ_HEAD_ARRIVAL_SLOTS : 0;  // a key per workgroup, then the counters
}

extern "C" int aq_t2_head_argmax(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* logits, int64_t n,
                                 int64_t k, uint64_t* cand, int64_t cand_cap, int32_t* token, int32_t* pos,
                                 int32_t* hist, int32_t hist_cap, int32_t advance, void* stream) {
  int st = t2_check(x2h, w, s, n, k);
  if (st) return st;
  if (!logits) return AQ_ERR_NULL;
  StepEnd step{};
  st = make_step_end(cand, cand_cap, t2_blocks(n, k), token, pos, hist, hist_cap, advance, step);
  if (st != AQ_OK) return st;
  return launch_t2_gemv(x2h, w, s, logits, (int)n, (int)k, step, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int aq_t2_packed_linear(const uint32_t* x2h, const uint32_t* w, const uint16_t* s, float* partials,
                                   int64_t n, int64_t k, void* stream) {
  int st = t2_check(x2h, w, s, n, k);
  if (st) return st;
  if (!partials) return AQ_ERR_NULL;
  return launch_t2_partials(x2h, w, s, partials, (int)n, (int)k, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int aq_t2_packed_reduce(const float* partials, float* y, int64_t n, int32_t groups, void* stream) {
  if (!partials || !y) return AQ_ERR_NULL;
  if (n <= 0 || groups <= 0 || n > (1 << 30)) return AQ_ERR_SHAPE;
  hipLaunchKernelGGL(k_t2_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), partials, y, (int)n, groups);
  return launch_status();
}

extern "C" int aq_pack_half(const float* x, uint32_t* q, int64_t count, void* stream) {
  if (!x || !q) return AQ_ERR_NULL;
  if (count <= 0 || count % 2) return AQ_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int64_t done = 0;  // floats handled by the vector kernel
  if (aligned(x, 16) && aligned(q, 16) && count >= 8) {
    const int64_t n8 = count / 8;
    int64_t blocks = (n8 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_pack_half8, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<const float4*>(x),
                       reinterpret_cast<uint4*>(q), n8);
    done = n8 * 8;
  }
  if (done < count) {
    const int64_t pairs = (count - done) / 2;
    int64_t blocks = (pairs + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_pack_half, dim3((unsigned)blocks), dim3(256), 0, s, x + done, q + done / 2, pairs);
  }
  return launch_status();
}

extern "C" int aq_rmsnorm_pack(const float* x, const float* w, uint32_t* q, int64_t rows, int64_t n, float eps,
                               void* stream) {
  if (!x || !w || !q) return AQ_ERR_NULL;
  if (rows <= 0 || n <= 0 || n % 2 || rows > (1 << 30)) return AQ_ERR_SHAPE;
  hipLaunchKernelGGL(k_rmsnorm_pack, dim3((unsigned)rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), x, w,
                     q, (int)n, eps);
  return launch_status();
}

extern "C" int aq_swiglu_pack(const float* gu, uint32_t* q, int64_t rows, int64_t n, void* stream) {
  if (!gu || !q) return AQ_ERR_NULL;
  if (rows <= 0 || n <= 0 || n % 2) return AQ_ERR_SHAPE;
  int64_t blocks = (rows * n / 2 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(k_swiglu_pack, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), gu,
                     q, (int)n, (int)rows);
  return launch_status();
}
