// Q6_K (Q6W) output head and embedding: the tied head/embedding matrix of a GGUF Q6_K model.
//
// Q6W layout: q [rows, nb = K/256, 208] bytes, one super-block of 256 weights each (ql[128]: low nibbles, qh[64]:
// 2-bit high parts, int8 scales[16], one per 16 weights), d fp16 [rows, nb]. Element 128 h + 32 j + l (h < 2, j < 4,
// l < 32) of a super-block is q = (nibble j / 2 of ql[64 h + 32 (j % 2) + l]) | (bits 2 j, 2 j + 1 of
// qh[32 h + l]) << 4, with value d * sc[8 h + 2 j + l / 16] * (q - 32).
//
// Work unit: u = (super-block b, half h, g < 2) covers the 64 weights of chunks j = g and j = g + 2 (l < 32), which
// share their 32 ql bytes (low and high nibbles) and their 32 qh bytes: 64 bytes of q plus 4 scales, 4 * nb units a
// row. A lane always owns the same unit of its rows, so the unit's 64 x values are loaded once into registers (K <=
// 4096: up to 64 units a row, UP = the next power of two of them lanes per row, 64 / UP rows per wave step) or read
// from LDS (larger K: one row per wave step, units strided over the lanes).
//
// Replaces: head_q6 / q6_chunk (lfm2/kernels/lk.mojo:88-129,179-191), the device argmax after it (:194-221) and
// embed_q6 (:224-232).
#include "aq_common.h"
#include "aq_step_end.h"

namespace aq {
namespace {

constexpr int kQ6Bytes = 208;   // bytes of a super-block in q
constexpr int kQ6Waves = 3072;  // waves of a head launch at most: 3 a SIMD (each strides over the row groups)
static_assert(kQ6Waves / 4 + AQ_HEAD_ARRIVAL_SLOTS <= AQ_HEAD_CANDIDATES, "one argmax key per workgroup");

struct Q6Raw {
  uint4 l0, l1, h0, h1;  // the unit's 32 ql bytes and 32 qh bytes
  uint2 sc;              // scales[8 h .. 8 h + 8)
  uint32_t d;            // d (fp16 bits in the low half)
};

// The loads of one unit. blk: byte offset of its super-block in q, dof: byte offset of its d (kOOB for an absent
// row: every load then returns zero).
__device__ __forceinline__ void q6_load(__amdgpu_buffer_rsrc_t qr, __amdgpu_buffer_rsrc_t dr, uint32_t blk,
                                        uint32_t dof, int h, int g, Q6Raw& r) {
  const uint32_t ql = blk + 64 * h + 32 * g, qh = blk + 128 + 32 * h;
  // default cache policy: the four 16-byte pieces of a unit share cache lines (streaming loads measured 50.8 -> 79 us
  // on the LFM2 head)
  r.l0 = buf_load16(qr, ql);
  r.l1 = buf_load16(qr, ql + 16);
  r.h0 = buf_load16(qr, qh);
  r.h1 = buf_load16(qr, qh + 16);
  r.sc = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(qr, blk + 192 + 8 * h, 0, 0));
  r.d = __builtin_amdgcn_raw_buffer_load_b16(dr, dof, 0, 0);
}

// The four 6-bit values of ql/qh word w of chunk g (qa) and of chunk g + 2 (qb), one per byte.
__device__ __forceinline__ void q6_bytes(uint32_t ql, uint32_t qh, int g, uint32_t& qa, uint32_t& qb) {
  qa = (ql & 0x0F0F0F0Fu) | ((qh << (4 - 2 * g)) & 0x30303030u);
  qb = ((ql >> 4) & 0x0F0F0F0Fu) | ((qh >> (2 * g)) & 0x30303030u);
}

__device__ __forceinline__ float sbyte(uint32_t w, int i) { return (float)(int8_t)(uint8_t)(w >> (8 * i)); }

// d * sum over the unit of sc * (q - 32) * x. xa: x of chunk g (32 values), xb: of chunk g + 2; sx: 32 * the sums of
// xa[0, 16), xa[16, 32), xb[0, 16), xb[16, 32) (the -32 offset, applied once per 16 weights).
__device__ __forceinline__ float q6_dot(const Q6Raw& r, const float* xa, const float* xb, float4 sx, int g) {
  const uint32_t ql[8] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w, r.l1.x, r.l1.y, r.l1.z, r.l1.w};
  const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
  float a[2] = {0.f, 0.f}, b[2] = {0.f, 0.f};
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t qa, qb;
    q6_bytes(ql[w], qh[w], g, qa, qb);
    float& A = a[w >> 2];
    float& B = b[w >> 2];
    A = fmaf((float)(qa & 0xFFu), xa[4 * w], A);
    A = fmaf((float)((qa >> 8) & 0xFFu), xa[4 * w + 1], A);
    A = fmaf((float)((qa >> 16) & 0xFFu), xa[4 * w + 2], A);
    A = fmaf((float)(qa >> 24), xa[4 * w + 3], A);
    B = fmaf((float)(qb & 0xFFu), xb[4 * w], B);
    B = fmaf((float)((qb >> 8) & 0xFFu), xb[4 * w + 1], B);
    B = fmaf((float)((qb >> 16) & 0xFFu), xb[4 * w + 2], B);
    B = fmaf((float)(qb >> 24), xb[4 * w + 3], B);
  }
  // chunk g's scales are bytes 2 g, 2 g + 1 of the 8, chunk g + 2's bytes 2 g + 4, 2 g + 5
  const uint32_t wa = g ? r.sc.x >> 16 : r.sc.x, wb = g ? r.sc.y >> 16 : r.sc.y;
  float acc = sbyte(wa, 0) * (a[0] - sx.x);
  acc = fmaf(sbyte(wa, 1), a[1] - sx.y, acc);
  acc = fmaf(sbyte(wb, 0), b[0] - sx.z, acc);
  acc = fmaf(sbyte(wb, 1), b[1] - sx.w, acc);
  return half_bits_to_float((uint16_t)r.d) * acc;
}

// Sum over each aligned group of UP lanes (UP = 4 .. 64), complete in the group's last lane.
template <int UP>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1>(0.f, v);
  v += dpp<0x4E>(0.f, v);
  if constexpr (UP >= 8) v += dpp<0x141>(0.f, v);
  if constexpr (UP >= 16) v += dpp<0x140>(0.f, v);
  if constexpr (UP >= 32) v += dpp<0x142, 0xA>(0.f, v);
  if constexpr (UP >= 64) v += dpp<0x143, 0xC>(0.f, v);
  return v;
}

// The first maximum among the lanes' (value, row) pairs (row < 0: none) as an argmax key, in every lane.
__device__ __forceinline__ uint64_t wave_key_max(float best, int best_row) {
  return wave_max_u64(best_row < 0 ? 0ull : argmax_key(best, best_row));
}

struct Q6Args {
  const uint8_t* q;
  const uint16_t* d;
  const float* x;
  const uint16_t* norm;  // RMSNorm weights [K] (NULL: x as given)
  float eps;
  float* y;
  int rows, nb;
  StepEnd step;    // the greedy step's end in the same launch (step.cand NULL: none)
};

// K <= 4096: UP lanes per row (the unit count rounded up to a power of two), 64 / UP rows a step, x in registers;
// the next three steps' loads are in flight during a step's arithmetic.
template <int UP>
__global__ __launch_bounds__(256) void k_head_q6(Q6Args a) {
  constexpr int RPW = 64 / UP;
  const int lane = threadIdx.x & 63;
  const int U = 4 * a.nb, K = 256 * a.nb;
  const int u = lane % UP, sub = lane / UP;
  const bool live = u < U;
  const int b = u >> 2, h = (u >> 1) & 1, g = u & 1;
  const int xo = 256 * b + 128 * h + 32 * g;  // x of chunk g; chunk g + 2 at xo + 64

  float xa[32], xb[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 va = live ? reinterpret_cast<const float4*>(a.x + xo)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 vb = live ? reinterpret_cast<const float4*>(a.x + xo + 64)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    xa[4 * i] = va.x, xa[4 * i + 1] = va.y, xa[4 * i + 2] = va.z, xa[4 * i + 3] = va.w;
    xb[4 * i] = vb.x, xb[4 * i + 1] = vb.y, xb[4 * i + 2] = vb.z, xb[4 * i + 3] = vb.w;
  }
  float rs = 1.f;
  if (a.norm) {  // every row group of the wave holds all of x: its sum of squares is the group's
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) ss = fmaf(xa[i], xa[i], fmaf(xb[i], xb[i], ss));
    ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum<UP>(ss)), UP - 1));
    rs = 1.0f / sqrtf(ss / (float)K + a.eps);
    if (live) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        xa[i] *= half_bits_to_float(a.norm[xo + i]);
        xb[i] *= half_bits_to_float(a.norm[xo + 64 + i]);
      }
    }
  }
  float4 sx = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) sx.x += xa[i], sx.y += xa[16 + i], sx.z += xb[i], sx.w += xb[16 + i];
  sx.x *= 32.f, sx.y *= 32.f, sx.z *= 32.f, sx.w *= 32.f;

  const auto qr = make_rsrc(a.q, (uint32_t)((int64_t)a.rows * a.nb * kQ6Bytes));
  const auto dr = make_rsrc(a.d, (uint32_t)((int64_t)a.rows * a.nb * 2));
  const int groups = (a.rows + RPW - 1) / RPW;
  const int wave = blockIdx.x * 4 + wave_id(), waves = gridDim.x * 4;
  auto issue = [&](int rg, Q6Raw& r) {
    const int row = rg * RPW + sub;
    const bool ok = live && rg < groups && row < a.rows;
    const uint32_t ub = (uint32_t)(row * a.nb + b);
    q6_load(qr, dr, ok ? ub * kQ6Bytes : kOOB, ok ? ub * 2 : kOOB, h, g, r);
  };
  float best = 0.f;
  int best_row = -1;
  auto process = [&](int rg, const Q6Raw& r) {
    const float v = group_sum<UP>(q6_dot(r, xa, xb, sx, g)) * rs;
    const int row = rg * RPW + sub;
    if (u == UP - 1 && row < a.rows) {
      a.y[row] = v;
      // rows arrive in ascending order, so `>` keeps the first maximum; NaN never wins
      if (!__builtin_isnan(v) && (best_row < 0 || v > best)) best = v, best_row = row;
    }
  };
  // three register sets in turn, all in flight ahead of their use (a copy from one to another would wait for the
  // loads): a step's loads are issued three steps before its arithmetic. Every set is processed unconditionally so
  // that its loads stay where they are issued; past the last row group they returned zero and nothing is stored.
  Q6Raw ra, rb, rc;
  issue(wave, ra);
  issue(wave + waves, rb);
  issue(wave + 2 * waves, rc);
  for (int rg = wave; rg < groups; rg += 3 * waves) {
    process(rg, ra);
    issue(rg + 3 * waves, ra);
    process(rg + waves, rb);
    issue(rg + 4 * waves, rb);
    process(rg + 2 * waves, rc);
    issue(rg + 5 * waves, rc);
  }
  if (a.step.cand) workgroup_step_end<4>(a.step, wave_key_max(best, best_row));  // workgroup-uniform
}

// Any K (% 256): x (times the norm weights) and the per-unit offsets sx staged in LDS; one row a wave step, the
// row's units strided over the 64 lanes.
__global__ __launch_bounds__(256) void k_head_q6_lds(Q6Args a) {
  extern __shared__ float xs[];  // K floats, then 4 * (K / 64) floats of sx
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wv = wave_id();
  const int U = 4 * a.nb, K = 256 * a.nb;
  float4* sxs = reinterpret_cast<float4*>(xs + K);
  float ss = 0.f;
  for (int i = threadIdx.x; i < K; i += 256) {
    const float v = a.x[i];
    ss = fmaf(v, v, ss);
    xs[i] = a.norm ? v * half_bits_to_float(a.norm[i]) : v;
  }
  float rs = 1.f;
  if (a.norm) {
    ss = wave_sum(ss);
    if (lane == 0) red[wv] = ss;
  }
  __syncthreads();
  if (a.norm) rs = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)K + a.eps);
  for (int u = threadIdx.x; u < U; u += 256) {
    const int xo = 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * (u & 1);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = 0; i < 16; ++i)
      s.x += xs[xo + i], s.y += xs[xo + 16 + i], s.z += xs[xo + 64 + i], s.w += xs[xo + 80 + i];
    sxs[u] = make_float4(32.f * s.x, 32.f * s.y, 32.f * s.z, 32.f * s.w);
  }
  __syncthreads();

  const auto qr = make_rsrc(a.q, (uint32_t)((int64_t)a.rows * a.nb * kQ6Bytes));
  const auto dr = make_rsrc(a.d, (uint32_t)((int64_t)a.rows * a.nb * 2));
  const int wave = blockIdx.x * 4 + wv, waves = gridDim.x * 4;
  float best = 0.f;
  int best_row = -1;
  for (int row = wave; row < a.rows; row += waves) {
    float acc = 0.f;
    for (int u = lane; u < U; u += 64) {
      const int b = u >> 2, h = (u >> 1) & 1, g = u & 1;
      const uint32_t ub = (uint32_t)(row * a.nb + b);
      Q6Raw r;
      q6_load(qr, dr, ub * kQ6Bytes, ub * 2, h, g, r);
      const float* xa = xs + 256 * b + 128 * h + 32 * g;
      float xra[32], xrb[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) xra[i] = xa[i], xrb[i] = xa[64 + i];
      acc += q6_dot(r, xra, xrb, sxs[u], g);
    }
    const float v = wave_sum(acc) * rs;
    if (lane == 0) {
      a.y[row] = v;
      if (!__builtin_isnan(v) && (best_row < 0 || v > best)) best = v, best_row = row;
    }
  }
  if (a.step.cand) workgroup_step_end<4>(a.step, wave_key_max(best, best_row));  // workgroup-uniform
}

// x[t] = the dequantized row ids[t] (rows outside [0, rows) read row 0): (d * sc) * (q - 32) in fp32, a thread a
// unit, workgroup row blockIdx.y.
__global__ __launch_bounds__(256) void k_embed_q6(const uint8_t* __restrict__ q, const uint16_t* __restrict__ d,
                                                  int rows, int nb, const int32_t* __restrict__ ids,
                                                  float* __restrict__ x) {
  const int t = blockIdx.y;
  int64_t tok = ids[t];
  tok = (tok < 0 || tok >= rows) ? 0 : tok;
  const int U = 4 * nb, K = 256 * nb;
  for (int u = blockIdx.x * 256 + threadIdx.x; u < U; u += gridDim.x * 256) {
    const int b = u >> 2, h = (u >> 1) & 1, g = u & 1;
    const uint8_t* blk = q + (tok * nb + b) * kQ6Bytes;
    const uint4* ql = reinterpret_cast<const uint4*>(blk + 64 * h + 32 * g);
    const uint4* qh = reinterpret_cast<const uint4*>(blk + 128 + 32 * h);
    const uint2 sc = *reinterpret_cast<const uint2*>(blk + 192 + 8 * h);
    const float dd = half_bits_to_float(d[tok * nb + b]);
    const uint32_t wa = g ? sc.x >> 16 : sc.x, wb = g ? sc.y >> 16 : sc.y;
    const float da[2] = {dd * sbyte(wa, 0), dd * sbyte(wa, 1)}, db[2] = {dd * sbyte(wb, 0), dd * sbyte(wb, 1)};
    const uint4 l0 = ql[0], l1 = ql[1], h0 = qh[0], h1 = qh[1];
    const uint32_t lw[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    float* xa = x + (int64_t)t * K + 256 * b + 128 * h + 32 * g;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t qa, qb;
      q6_bytes(lw[w], hw[w], g, qa, qb);
      const float sa = da[w >> 2], sb = db[w >> 2];
      reinterpret_cast<float4*>(xa)[w] =
          make_float4(sa * (float)((int)(qa & 0xFFu) - 32), sa * (float)((int)((qa >> 8) & 0xFFu) - 32),
                      sa * (float)((int)((qa >> 16) & 0xFFu) - 32), sa * (float)((int)(qa >> 24) - 32));
      reinterpret_cast<float4*>(xa + 64)[w] =
          make_float4(sb * (float)((int)(qb & 0xFFu) - 32), sb * (float)((int)((qb >> 8) & 0xFFu) - 32),
                      sb * (float)((int)((qb >> 16) & 0xFFu) - 32), sb * (float)((int)(qb >> 24) - 32));
    }
  }
}

int q6_check(const void* q, const void* d, int64_t rows, int64_t cols) {
  if (!q || !d) return AQ_ERR_NULL;
  if (rows <= 0 || cols <= 0 || cols % 256) return AQ_ERR_SHAPE;
  if (rows * (cols / 256) * kQ6Bytes >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;
  if (!aligned(q, 16) || !aligned(d, 2)) return AQ_ERR_ALIGN;
  return AQ_OK;
}

// Waves a head launch over rows x cols uses (a multiple of 4: workgroups of 4 waves).
int q6_waves(int64_t rows, int64_t cols) {
  const int64_t units = cols / 64;
  int64_t per_step = 1;
  if (units <= 64) {
    int up = 4;
    while (up < units) up *= 2;
    per_step = 64 / up;
  }
  const int64_t groups = (rows + per_step - 1) / per_step;
  const int64_t w = groups < kQ6Waves ? groups : kQ6Waves;
  return (int)((w + 3) / 4 * 4);
}

int launch_head_q6(const Q6Args& a, int64_t cols, hipStream_t s) {
  const int units = (int)(cols / 64);
  const dim3 grid((unsigned)(q6_waves(a.rows, cols) / 4)), block(256);
  switch (units <= 4 ? 4 : units <= 8 ? 8 : units <= 16 ? 16 : units <= 32 ? 32 : units <= 64 ? 64 : 0) {
    case 4: hipLaunchKernelGGL(k_head_q6<4>, grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL(k_head_q6<8>, grid, block, 0, s, a); break;
    case 16: hipLaunchKernelGGL(k_head_q6<16>, grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL(k_head_q6<32>, grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL(k_head_q6<64>, grid, block, 0, s, a); break;
    default: {
      const size_t lds = (size_t)cols * 4 + (size_t)units * 16;
      if (lds > 64 * 1024) return AQ_ERR_CAPACITY;
      hipLaunchKernelGGL(k_head_q6_lds, grid, block, lds, s, a);
    }
  }
  return launch_status();
}

}  // namespace
}  // namespace aq

extern "C" int64_t aq_head_q6_candidates(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % 256) return 0;
  return aq::q6_waves(rows, cols) / 4 + AQ_HEAD_ARRIVAL_SLOTS;  // a key per workgroup, then the counters
}

extern "C" int aq_gemv_q6(const uint8_t* q, const uint16_t* d, const float* x, float* y, int64_t rows, int64_t cols,
                          void* stream) {
  int st = aq::q6_check(q, d, rows, cols);
  if (st) return st;
  if (!x || !y) return AQ_ERR_NULL;
  if (!aq::aligned(x, 16)) return AQ_ERR_ALIGN;
  const aq::Q6Args a{q, d, x, nullptr, 0.f, y, (int)rows, (int)(cols / 256), {}};
  return aq::launch_head_q6(a, cols, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int aq_head_argmax_q6(const uint8_t* q, const uint16_t* d, const float* x, const uint16_t* norm_w,
                                 float eps, float* logits, int64_t rows, int64_t cols, uint64_t* cand,
                                 int64_t cand_cap, int32_t* token, int32_t* pos, int32_t* hist, int32_t hist_cap,
                                 int32_t advance, void* stream) {
  int st = aq::q6_check(q, d, rows, cols);
  if (st) return st;
  if (!x || !logits) return AQ_ERR_NULL;
  if (!aq::aligned(x, 16) || (norm_w && !aq::aligned(norm_w, 2))) return AQ_ERR_ALIGN;
  aq::Q6Args a{q, d, x, norm_w, eps, logits, (int)rows, (int)(cols / 256), {}};
  st = aq::make_step_end(cand, cand_cap, aq::q6_waves(rows, cols) / 4, token, pos, hist, hist_cap, advance, a.step);
  if (st != AQ_OK) return st;
  return aq::launch_head_q6(a, cols, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int aq_embed_q6(const uint8_t* q, const uint16_t* d, int64_t rows, int64_t cols, const int32_t* ids,
                           int32_t ntok, float* x, void* stream) {
  int st = aq::q6_check(q, d, rows, cols);
  if (st) return st;
  if (!ids || !x) return AQ_ERR_NULL;
  if (ntok <= 0 || ntok > 65535) return AQ_ERR_SHAPE;
  if (!aq::aligned(x, 16)) return AQ_ERR_ALIGN;
  const int units = (int)(cols / 64);
  const dim3 grid((unsigned)((units + 255) / 256), (unsigned)ntok);
  hipLaunchKernelGGL(aq::k_embed_q6, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), q, d, (int)rows,
                     (int)(cols / 256), ids, x);
  return aq::launch_status();
}
