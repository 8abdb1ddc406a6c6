// MoE decode down projection (one token), gfx950: y[r] = (add ? y[r] : 0) + sum over expert slots s < topk, in slot
// order, of rw[s] * (W[ids[s] * d + r] . a[s]), Q4W W stacked by expert [experts * d, f/8], fp32 a [topk, f].
// The arithmetic of qwen3moe/kernels/moek.mojo:213-223 (moe_down) and lfm2moe/kernels/mk.mojo:107-118.
//
// Design (HBM-bound: 8 expert rows of f/2 bytes for every output; Qwen3-30B-A3B moves 7.1 MB a token):
// - a 512-thread workgroup owns RW = 8 outputs; wave s takes expert slot s, so every wave streams the 8 rows of one
//   expert and stages only that slot's activations (a KB each), not all eight;
// - 8 lanes a row: lane (row r = l / 8, sub = l % 8) takes the 32-weight chunks c = 8 j + sub, j < CPL, of its row
//   (CPL = f / 256 rounded up: 3 at f = 768, so every lane is busy), all requested at once; the slot's activations
//   (a word of 8 values a lane and pass) are requested before them, so the staging overlaps the weights' flight;
// - the slot's activations are staged as signed 4-bit digits of per-chunk fixed point (stage_digits), and a chunk's
//   four words meet them in v_dot8_i32_i4 as stored (chunk_dot), times its fp16 scale (one per chunk: a power-of-two
//   group >= 32);
// - each row's 8 lane sums meet by DPP, and the 8 slots' sums by LDS: thread r < RW folds them in slot order, so the
//   result does not depend on scheduling.
#include "aq_common.h"
#include "aq_digits.h"
#include "aq_moe_decode.h"

namespace aq {

constexpr int kDownRows = 8;    // outputs a workgroup
constexpr int kDownSlots = 8;   // waves a workgroup: expert slots (topk <= 8)

template <int CPL>
__global__ __launch_bounds__(512) void k_moe_down_dec(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                      const int32_t* __restrict__ ids, const float* __restrict__ rw,
                                                      const float* __restrict__ act, float* __restrict__ y, int d,
                                                      int f, int gsh, int experts, int topk, int add) {
  extern __shared__ uint4 xd[];  // stage_digits planes of the 8 slots ([slot][6][f / 32]), then their factors
  __shared__ float red[kDownSlots][kDownRows];
  const int lane = threadIdx.x & 63;
  const int s = wave_id();  // expert slot of this wave
  const int r0 = blockIdx.x * kDownRows;
  const int row = lane >> 3, sub = lane & 7;
  const int kw = f >> 3, nch = f >> 5, gpr = f >> gsh;
  float* xf = reinterpret_cast<float*>(xd + kDownSlots * 6 * nch);

  // this slot's activations first, a word (8 values) a lane and pass: they do not depend on the expert id, so their
  // arrival (and the staging below) overlaps the id's load and the weights' flight; vector memory completes in
  // order, so waiting for them does not wait for the weights requested after them
  constexpr int XP = (CPL * 8 * 4 + 63) / 64;  // passes: f / 8 words over 64 lanes (f <= 256 CPL)
  float4 xa[XP], xb[XP];
  const bool slot = s < topk;  // wave-uniform
  {
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(act, (uint32_t)topk * (uint32_t)f * 4u);
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const uint32_t wi = (uint32_t)(lane + 64 * j);  // word within the slot's row
      const uint32_t off = slot && wi < (uint32_t)kw ? ((uint32_t)s * (uint32_t)f + 8u * wi) * 4u : kOOB;
      xa[j] = __builtin_bit_cast(float4, buf_load16(a_rsrc, off));
      xb[j] = __builtin_bit_cast(float4, buf_load16(a_rsrc, off == kOOB ? kOOB : off + 16u));
    }
  }
  const int e = slot ? ids[s] : -1;
  const bool live = e >= 0 && e < experts;  // wave-uniform
  // the stacked experts' rows and scales: below 2 GiB (checked by the entry point)
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(wq, (uint32_t)experts * (uint32_t)d * (uint32_t)kw * 4u);
  const __amdgpu_buffer_rsrc_t s_rsrc =
      make_rsrc(ws, ((uint32_t)experts * (uint32_t)d * (uint32_t)gpr * 2u + 3u) & ~3u);
  const int r = min(r0 + row, d - 1);  // rows past d repeat the last one; their sums are not stored
  const uint32_t wrow = (uint32_t)e * (uint32_t)d + (uint32_t)r;
  uint4 w[CPL];
  uint32_t sc[CPL];  // the aligned 4 bytes holding each chunk's scale (a 16-bit load would be widened, and so
  uint32_t sh[CPL];  // waited for, right after it) and the scale's bit offset in them
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = 8 * j + sub;
    const bool ok = live && c < nch;
    w[j] = buf_load16p<kWPolicy>(w_rsrc, ok ? (wrow * (uint32_t)kw + 4u * (uint32_t)c) * 4u : kOOB);
    const uint32_t si = wrow * (uint32_t)gpr + (uint32_t)((32 * c) >> gsh);
    sc[j] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, ok ? (si * 2u) & ~3u : kOOB, 0, 0);
    sh[j] = (si & 1u) << 4;
  }

  // stage the slot's digits (f % 32 == 0: kw % 4 == 0, so a pass holds whole chunks and a chunk's 4 lanes are all in
  // range or all out, as stage_digits needs)
  if (live) {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int wi = lane + 64 * j;
      if (wi < kw) stage_digits(s, wi >> 2, wi & 3, xa[j], xb[j], xd, xf, nch);
    }
  }
  __syncthreads();

  float acc[1][1] = {{0.f}};
  if (live) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = 8 * j + sub;
      if (c < nch) {
        const uint4 wr[1] = {w[j]};
        const uint16_t s16[1] = {(uint16_t)(sc[j] >> sh[j])};
        chunk_dot<1, 1>(xd + s * 6 * nch, xf + s * nch, nch, c, wr, s16, acc);
      }
    }
  }
  const float a = sum8(acc[0][0]);
  if (sub == 0) red[s][row] = live ? a : 0.f;
  __syncthreads();
  if (threadIdx.x < kDownRows) {
    const int o = r0 + threadIdx.x;
    if (o < d) {
      float sum = 0.f;
      for (int t = 0; t < topk; ++t) sum = fmaf(rw[t], red[t][threadIdx.x], sum);
      y[o] = add ? y[o] + sum : sum;
    }
  }
}

bool moe_down_dec_ok(int64_t f, int32_t group, int32_t topk) {
  return topk >= 1 && topk <= kDownSlots && f >= 32 && f % 32 == 0 && f <= 32 * 8 * 8 && group >= 32 &&
         (group & (group - 1)) == 0;
}

int launch_moe_down_dec(const uint32_t* wq, const uint16_t* ws, const int32_t* ids, const float* rw,
                        const float* act, float* y, int64_t d, int64_t f, int32_t group, int32_t experts,
                        int32_t topk, int32_t add, hipStream_t st) {
  const int cpl = (int)((f / 32 + 7) / 8);
  const size_t lds = (size_t)kDownSlots * (size_t)(f / 32) * (6 * 16 + 4);  // digit planes and factors
  const dim3 grid((unsigned)((d + kDownRows - 1) / kDownRows)), block(512);
  const int gsh = __builtin_ctz(group);
#define AQ_DOWN_CASE(C)                                                                                              \
  case C:                                                                                                            \
    if (lds > 64 * 1024 && hipFuncSetAttribute(reinterpret_cast<const void*>(k_moe_down_dec<C>),                    \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) \
      return AQ_ERR_CAPACITY;                                                                                        \
    hipLaunchKernelGGL(k_moe_down_dec<C>, grid, block, lds, st, wq, ws, ids, rw, act, y, (int)d, (int)f, gsh,       \
                       experts, topk, add);                                                                          \
    break;
  switch (cpl) {
    AQ_DOWN_CASE(1)
    AQ_DOWN_CASE(2)
    AQ_DOWN_CASE(3)
    AQ_DOWN_CASE(4)
    AQ_DOWN_CASE(5)
    AQ_DOWN_CASE(6)
    AQ_DOWN_CASE(7)
    AQ_DOWN_CASE(8)
    default:
      return AQ_ERR_SHAPE;
  }
#undef AQ_DOWN_CASE
  return launch_status();
}

}  // namespace aq
