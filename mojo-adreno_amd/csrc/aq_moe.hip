// Mixture-of-experts plumbing around the grouped int4 GEMM, gfx950: top-k routing, deterministic expert grouping
// (histogram, padded prefix sum, stable permute, work tiles), the weighted combine and the fp32 router GEMV. The
// decode-time expert GEMVs are modes of the int4 GEMV (aq_gemv.hip).
//
// Reference: qwen3moe/kernels/moek.mojo (route :156-197, p_route :385-425, moe_gate_up :200-210, moe_down :213-223,
// gemv_f32 :143-153, p_expert_lists :432-442, p_expert_items :548-557, p_moe_sum :479-488) and
// lfm2moe/kernels/mk.mojo (p_group :123-161, p_combine :189-199). Every index this file produces is a pure function
// of the routing ids (no atomics decide an order), so routing, lists, slots and tiles are bit-for-bit reproducible.
#include "aq_common.h"

namespace aq {

// ---- routing: top-k of E logits per token, lowest index among equals; weights = softmax over the k winners ----
// One wave per token, lane l holding logits l, l + 64, ... (PER_LANE of them). Round r: the wave maximum m of the
// logits not yet taken (DPP), then the lowest index holding m among them (one ballot per slot: slot j's indices
// 64 j .. 64 j + 63 are all below slot j + 1's), which is taken: the reference's iterated argmax (moek.mojo:164-186).
// The weights are exp(v_r - v_0) / sum_{r < k} exp(v_r - v_0), summed in rank order. With xq, the wave also rounds
// its token's row of x (d fp32, d % 8 == 0) to fp16 pairs for the grouped GEMM, issued first so the two overlap.
template <int PER_LANE>
__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                               float* __restrict__ weights, int tokens, int E, int topk,
                                               const float* __restrict__ x, uint32_t* __restrict__ xq, int d) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave_id();
  if (t >= tokens) return;  // wave-uniform; the kernel has no barrier
  if (xq) {
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)t * d);
    uint4* qr = reinterpret_cast<uint4*>(xq + (size_t)t * (d / 2));
#pragma unroll 4  // several words' loads in flight together
    for (int i = lane; i < d / 8; i += 64) {
      const float4 a = xr[2 * i], b = xr[2 * i + 1];
      qr[i] = make_uint4((uint32_t)float_to_half_bits(a.x) | ((uint32_t)float_to_half_bits(a.y) << 16),
                         (uint32_t)float_to_half_bits(a.z) | ((uint32_t)float_to_half_bits(a.w) << 16),
                         (uint32_t)float_to_half_bits(b.x) | ((uint32_t)float_to_half_bits(b.y) << 16),
                         (uint32_t)float_to_half_bits(b.z) | ((uint32_t)float_to_half_bits(b.w) << 16));
    }
  }
  float v[PER_LANE];
  bool taken[PER_LANE];
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? logits[(size_t)t * E + e] : -INFINITY;
    taken[j] = e >= E;  // padding slots are never candidates
  }
  float top0 = 0.f, le = 0.f, total = 0.f;  // le: exp(v_r - v_0) of this lane's round r = lane
  for (int r = 0; r < topk; ++r) {
    float best = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) best = taken[j] ? best : fmaxf(best, v[j]);
    const float m = wave_max(best);
    int win = -1;
#pragma unroll
    for (int j = PER_LANE - 1; j >= 0; --j) {  // the lowest slot with a match decides
      const uint64_t bal = __ballot(!taken[j] && v[j] == m);
      if (bal) win = 64 * j + __builtin_ctzll(bal);
    }
    if (win < 0) {  // no candidate equals m (NaN logits only): the lowest index not yet taken
#pragma unroll
      for (int j = PER_LANE - 1; j >= 0; --j) {
        const uint64_t bal = __ballot(!taken[j]);
        if (bal) win = 64 * j + __builtin_ctzll(bal);
      }
    }
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j)
      if (lane + 64 * j == win) taken[j] = true;
    if (r == 0) top0 = m;
    const float ex = expf(m - top0);
    total += ex;
    if (lane == r) le = ex;
    if (lane == 0) ids[(size_t)t * topk + r] = win;
  }
  if (lane < topk) weights[(size_t)t * topk + lane] = le / total;
}

// ---- grouping: one 1024-thread workgroup --------------------------------------------------------------------------
// Entry i = t * topk + k chose expert ids[i]. Per expert e: cnt[e] entries; segments in expert order, each padded to
// a multiple of tm rows, start at offs[e] (exclusive prefix sum of the padded counts); entry i's row slot[i] is
// offs[e] + its rank among e's entries in ascending i; src[row] = its token (-1 on padding rows); work tiles
// (e, offs[e] + c) for c = 0, tm, ... < cnt[e], in expert order, and their number. Optionally the qwen3moe lists
// (lists[e * cap + r] = i of rank r) and items ((e, c) every `items_tt` entries).
// Ranks without atomics deciding any order: bit t of expert e's token bitmap is set (LDS atomic OR, order-free) when
// token t chose e. While a token chooses an expert at most once (top-k of distinct experts), the rank of entry i is
// the number of set bits below t: a per-word prefix popcount plus the popcount of the bits below t in its word. An
// OR that finds its bit already set shows a token that chose one expert twice; the whole launch then takes the
// reference's ordered scan instead (p_group: one thread per expert walks the entries in ascending i, here in chunks
// staged in LDS), which counts every entry and ranks repeated ones in ascending i.
struct GroupOut {
  int32_t* counts;   // [E]
  int32_t* offs;     // [E + 1]
  int32_t* slot;     // [n]
  int32_t* src;      // [max_rows]
  int32_t* tiles;    // [2 * max_tiles]
  int32_t* ntiles;   // [1]
  int32_t* lists;    // [E * cap] or null
  int32_t* items;    // [2 * max_items] or null
  int32_t* nitems;   // [1] or null
  int cap, items_tt, max_rows, max_tiles, max_items;
};

constexpr int kGroupChunk = 1024;  // entries staged per round of the ordered scan

__global__ __launch_bounds__(1024) void k_moe_group(const int32_t* __restrict__ ids, int n, int topk, int E, int tm,
                                                    GroupOut o) {
  extern __shared__ unsigned long long bits[];  // [E][W] token bitmaps
  const int T = n / topk;
  const int W = (T + 63) >> 6;
  int32_t* pre = reinterpret_cast<int32_t*>(bits + (size_t)E * W);  // [E][W] set bits before each word
  int32_t* eoff = pre + E * W;   // [E + 1] first row of expert e's segment
  int32_t* tbase = eoff + E + 1; // [E + 1] first work tile of expert e
  int32_t* ibase = tbase + E + 1;// [E + 1] first work item of expert e (lists mode)
  int32_t* chunk = ibase + E + 1;// [kGroupChunk] entries of one round of the ordered scan
  __shared__ int32_t wtot[16][3];
  __shared__ int repeated;       // some token chose one expert twice: ordered scan
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  if (threadIdx.x == 0) repeated = 0;
  for (int i = threadIdx.x; i < E * W; i += 1024) bits[i] = 0ull;
  for (int r = threadIdx.x; r < o.max_rows; r += 1024) o.src[r] = -1;  // padding rows; real rows are set below
  __syncthreads();
  // this thread's first kIdReg ids stay in registers for the placement below (a second read would wait on memory)
  constexpr int kIdReg = 4;
  int idr[kIdReg];
#pragma unroll
  for (int q = 0; q < kIdReg; ++q) {
    const int i = threadIdx.x + 1024 * q;
    idr[q] = i < n ? ids[i] : -1;
  }
  for (int i = threadIdx.x; i < n; i += 1024) {
    const int q = i >> 10;
    const int e = q < kIdReg ? idr[q < kIdReg ? q : 0] : ids[i];
    if (e >= 0 && e < E) {
      const unsigned long long bit = 1ull << ((i / topk) & 63);
      if (atomicOr(&bits[(size_t)e * W + ((i / topk) >> 6)], bit) & bit) repeated = 1;
    }
  }
  __syncthreads();
  const bool scan = repeated != 0;  // workgroup-uniform
  const int e = threadIdx.x;
  // The ordered scan: every thread stages the entries [base, base + kGroupChunk) into LDS, then thread e (< E) walks
  // them in ascending i and calls visit(i) for each entry of its expert. Barriers are workgroup-uniform.
  auto ordered_scan = [&](auto visit) {
    for (int base = 0; base < n; base += kGroupChunk) {
      const int len = min(kGroupChunk, n - base);
      for (int j = threadIdx.x; j < len; j += 1024) chunk[j] = ids[base + j];
      __syncthreads();
      if (e < E)
        for (int j = 0; j < len; ++j)
          if (chunk[j] == e) visit(base + j);
      __syncthreads();
    }
  };
  // one thread per expert: count, padded rows, tiles, items; then exclusive scans over the experts (16 waves x 64)
  int c = 0, rows = 0, nt = 0, ni = 0;
  if (scan) {
    ordered_scan([&](int) { ++c; });
  } else if (e < E) {
    for (int w = 0; w < W; ++w) {
      pre[e * W + w] = c;
      c += __popcll(bits[(size_t)e * W + w]);
    }
  }
  if (e < E) {
    nt = (c + tm - 1) / tm;
    rows = nt * tm;
    ni = o.items ? (c + o.items_tt - 1) / o.items_tt : 0;
  }
  int sr = rows, st = nt, si = ni;  // inclusive wave scans
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int ur = __shfl_up(sr, d, 64), ut = __shfl_up(st, d, 64), ui = __shfl_up(si, d, 64);
    if (lane >= d) {
      sr += ur;
      st += ut;
      si += ui;
    }
  }
  if (lane == 63) {
    wtot[wave][0] = sr;
    wtot[wave][1] = st;
    wtot[wave][2] = si;
  }
  __syncthreads();
  int br = 0, bt = 0, bi = 0;
  for (int v = 0; v < wave; ++v) {
    br += wtot[v][0];
    bt += wtot[v][1];
    bi += wtot[v][2];
  }
  if (e < E) {
    eoff[e] = br + sr - rows;
    tbase[e] = bt + st - nt;
    ibase[e] = bi + si - ni;
    o.counts[e] = c;
    o.offs[e] = eoff[e];
    for (int j = 0; j < nt; ++j)
      if (tbase[e] + j < o.max_tiles) {
        o.tiles[2 * (tbase[e] + j)] = e;
        o.tiles[2 * (tbase[e] + j) + 1] = eoff[e] + j * tm;
      }
    if (o.items)
      for (int j = 0; j < ni; ++j)
        if (ibase[e] + j < o.max_items) {
          o.items[2 * (ibase[e] + j)] = e;
          o.items[2 * (ibase[e] + j) + 1] = j * o.items_tt;
        }
    if (e == E - 1) {
      o.offs[E] = br + sr;
      o.ntiles[0] = bt + st;
      if (o.nitems) o.nitems[0] = bi + si;
    }
  }
  __syncthreads();
  // entry i of expert ex at rank r among ex's entries
  auto place = [&](int i, int ex, int rank) {
    const int row = eoff[ex] + rank;
    o.slot[i] = row;
    if (row < o.max_rows) o.src[row] = i / topk;
    if (o.lists && rank < o.cap) o.lists[(size_t)ex * o.cap + rank] = i;
  };
  for (int i = threadIdx.x; i < n; i += 1024) {
    const int q = i >> 10;
    const int ex = q < kIdReg ? idr[q < kIdReg ? q : 0] : ids[i];
    if (ex < 0 || ex >= E) {
      o.slot[i] = -1;  // an id outside [0, E) is in no group
      continue;
    }
    if (scan) continue;  // placed by the ordered scan below
    const int t = i / topk;
    const unsigned long long word = bits[(size_t)ex * W + (t >> 6)];
    place(i, ex, pre[ex * W + (t >> 6)] + __popcll(word & ((1ull << (t & 63)) - 1ull)));
  }
  if (scan) {
    int rank = 0;
    ordered_scan([&](int i) { place(i, e, rank++); });
  }
}

// ---- combine: y[t, c] = (add ? y[t, c] : 0) + sum_k w[t, k] * yd[slot[t*topk + k], c], k in order ----
// KT: a compile-time bound on topk (0: any topk, one entry at a time). With KT, every entry's slot and weight and then
// every row's 16 bytes are requested before the first is used, so the eight row reads are in flight together.
template <int KT>
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ yd, const int32_t* __restrict__ slot,
                                                     const float* __restrict__ w, float* __restrict__ y, int tokens,
                                                     int d, int topk, int add, int yd_rows) {
  const int d4 = d >> 2;
  const int64_t total = (int64_t)tokens * d4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int t = (int)(i / d4);
    const int c = (int)(i - (int64_t)t * d4);
    float4 acc = add ? reinterpret_cast<const float4*>(y + (size_t)t * d)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (KT > 0) {
      int r[KT];
      float wk[KT];
#pragma unroll
      for (int k = 0; k < KT; ++k) {
        const int rr = k < topk ? (slot ? slot[t * topk + k] : t * topk + k) : -1;
        r[k] = (rr >= 0 && rr < yd_rows) ? rr : -1;  // an entry in no group contributes nothing
        wk[k] = k < topk ? w[t * topk + k] : 0.f;
      }
      float4 v[KT];
#pragma unroll
      for (int k = 0; k < KT; ++k)
        v[k] = r[k] >= 0 ? reinterpret_cast<const float4*>(yd + (size_t)r[k] * d)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int k = 0; k < KT; ++k) {
        if (r[k] < 0) continue;  // as in the loop below: a skipped entry adds nothing (not even 0 * NaN)
        acc.x = fmaf(wk[k], v[k].x, acc.x);
        acc.y = fmaf(wk[k], v[k].y, acc.y);
        acc.z = fmaf(wk[k], v[k].z, acc.z);
        acc.w = fmaf(wk[k], v[k].w, acc.w);
      }
    } else {
      for (int k = 0; k < topk; ++k) {
        const int r = slot ? slot[t * topk + k] : t * topk + k;
        if (r < 0 || r >= yd_rows) continue;  // an entry in no group contributes nothing
        const float wk = w[t * topk + k];
        const float4 v = reinterpret_cast<const float4*>(yd + (size_t)r * d)[c];
        acc.x = fmaf(wk, v.x, acc.x);
        acc.y = fmaf(wk, v.y, acc.y);
        acc.z = fmaf(wk, v.z, acc.z);
        acc.w = fmaf(wk, v.w, acc.w);
      }
    }
    reinterpret_cast<float4*>(y + (size_t)t * d)[c] = acc;
  }
}

// ---- router: y[t, r] = W[r] . x[t] with fp32 W: one wave per (row, token) ----
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ y, int n, int k, int tokens) {
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * 4 + wave_id();
  if (o >= n * tokens) return;
  const int t = o / n, r = o - t * n;
  const float* wr = w + (size_t)r * k;
  const float* xr = x + (size_t)t * k;
  float acc = 0.f;
  if ((k & 3) == 0) {
#pragma unroll 8  // eight rows' words requested together (the multiply-add order is unchanged)
    for (int c = lane; c < (k >> 2); c += 64) {
      const float4 a = reinterpret_cast<const float4*>(wr)[c];
      const float4 b = reinterpret_cast<const float4*>(xr)[c];
      acc = fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, fmaf(a.w, b.w, acc))));
    }
  } else {
    for (int c = lane; c < k; c += 64) acc = fmaf(wr[c], xr[c], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[(size_t)t * n + r] = acc;
}

}  // namespace aq

using namespace aq;

static int launch_route(const float* logits, int32_t* ids, float* weights, int64_t tokens, int32_t experts,
                        int32_t topk, const float* x, uint32_t* xq, int d, hipStream_t s) {
  using namespace aq;
  const dim3 grid((unsigned)((tokens + 3) / 4));
  if (experts <= 64)
    hipLaunchKernelGGL(k_route<1>, grid, dim3(256), 0, s, logits, ids, weights, (int)tokens, experts, topk, x, xq, d);
  else if (experts <= 128)
    hipLaunchKernelGGL(k_route<2>, grid, dim3(256), 0, s, logits, ids, weights, (int)tokens, experts, topk, x, xq, d);
  else
    hipLaunchKernelGGL(k_route<4>, grid, dim3(256), 0, s, logits, ids, weights, (int)tokens, experts, topk, x, xq, d);
  return launch_status();
}

extern "C" int aq_moe_route(const float* logits, int32_t* ids, float* weights, int64_t tokens, int32_t experts,
                            int32_t topk, void* stream) {
  if (!logits || !ids || !weights) return AQ_ERR_NULL;
  if (tokens <= 0 || experts <= 0 || experts > 256 || topk <= 0 || topk > 8 || topk > experts) return AQ_ERR_SHAPE;
  return launch_route(logits, ids, weights, tokens, experts, topk, nullptr, nullptr, 0,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int aq_moe_route_pack(const float* logits, int32_t* ids, float* weights, int64_t tokens, int32_t experts,
                                 int32_t topk, const float* x, uint32_t* xq, int64_t d, void* stream) {
  if (!logits || !ids || !weights || !x || !xq) return AQ_ERR_NULL;
  if (tokens <= 0 || experts <= 0 || experts > 256 || topk <= 0 || topk > 8 || topk > experts) return AQ_ERR_SHAPE;
  if (d <= 0 || d % 8 || tokens * d >= ((int64_t)1 << 31)) return AQ_ERR_SHAPE;
  if (!aq::aligned(x, 16) || !aq::aligned(xq, 16)) return AQ_ERR_ALIGN;
  return launch_route(logits, ids, weights, tokens, experts, topk, x, xq, (int)d, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int64_t aq_moe_group_max_rows(int64_t tokens, int32_t topk, int32_t experts, int32_t tm) {
  if (tokens <= 0 || topk <= 0 || experts <= 0 || tm <= 0) return 0;
  return (tokens * topk + (int64_t)experts * (tm - 1) + tm - 1) / tm * tm;
}

extern "C" int32_t aq_moe_group_max_tiles(int64_t tokens, int32_t topk, int32_t experts, int32_t tm) {
  if (tokens <= 0 || topk <= 0 || experts <= 0 || tm <= 0) return 0;
  return (int32_t)((tokens * topk + (int64_t)experts * (tm - 1)) / tm);
}

static size_t group_lds(int64_t tokens, int E) {
  const int64_t W = (tokens + 63) / 64;
  return (size_t)E * W * 12 + (size_t)3 * (E + 1) * 4 + (size_t)aq::kGroupChunk * 4;
}

extern "C" int aq_moe_group(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts, int32_t tm,
                            int32_t* counts, int32_t* offs, int32_t* slot, int32_t* src, int64_t max_rows,
                            int32_t* tiles, int32_t max_tiles, int32_t* ntiles, void* stream) {
  if (!ids || !counts || !offs || !slot || !src || !tiles || !ntiles) return AQ_ERR_NULL;
  if (tokens <= 0 || topk <= 0 || experts <= 0 || experts > 1024 || tm <= 0) return AQ_ERR_SHAPE;
  if (max_rows < aq_moe_group_max_rows(tokens, topk, experts, tm) ||
      max_tiles < aq_moe_group_max_tiles(tokens, topk, experts, tm))
    return AQ_ERR_CAPACITY;
  const int64_t n = tokens * topk;
  const size_t lds = group_lds(tokens, experts);
  if (lds > 160 * 1024) return AQ_ERR_CAPACITY;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_moe_group), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return AQ_ERR_CAPACITY;
  GroupOut o{};
  o.counts = counts; o.offs = offs; o.slot = slot; o.src = src; o.tiles = tiles; o.ntiles = ntiles;
  o.max_rows = (int)max_rows; o.max_tiles = max_tiles;
  hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), lds, reinterpret_cast<hipStream_t>(stream), ids, (int)n, topk,
                     experts, tm, o);
  return launch_status();
}

extern "C" int aq_moe_expert_lists(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts, int32_t cap,
                                   int32_t* lists, int32_t* counts, int32_t items_tt, int32_t* items,
                                   int32_t max_items, int32_t* nitems, int32_t* scratch, int64_t scratch_ints,
                                   void* stream) {
  if (!ids || !lists || !counts || !scratch) return AQ_ERR_NULL;
  if (tokens <= 0 || topk <= 0 || experts <= 0 || experts > 1024 || cap < tokens) return AQ_ERR_SHAPE;
  if (items && (items_tt <= 0 || !nitems)) return AQ_ERR_ARG;
  const int64_t n = tokens * topk;
  // the lists are the grouping with tm = 1 (no padding); its offsets, slots, src and tiles go to the scratch ints
  const int64_t need = (experts + 1) + n + n + 2 * n + 1;
  if (scratch_ints < need) return AQ_ERR_CAPACITY;
  const size_t lds = group_lds(tokens, experts);
  if (lds > 160 * 1024) return AQ_ERR_CAPACITY;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_moe_group), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return AQ_ERR_CAPACITY;
  GroupOut o{};
  o.counts = counts;
  o.offs = scratch;
  o.slot = scratch + (experts + 1);
  o.src = o.slot + n;
  o.tiles = o.src + n;
  o.ntiles = o.tiles + 2 * n;
  o.max_rows = (int)n;
  o.max_tiles = (int)n;
  o.lists = lists;
  o.cap = cap;
  o.items = items;
  o.items_tt = items_tt;
  o.nitems = nitems;
  o.max_items = max_items;
  hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), lds, reinterpret_cast<hipStream_t>(stream), ids, (int)n, topk,
                     experts, 1, o);
  return launch_status();
}

extern "C" int aq_moe_combine(const float* yd, int64_t yd_rows, const int32_t* slot, const float* weights, float* y,
                              int64_t tokens, int64_t d, int32_t topk, int32_t add, void* stream) {
  if (!yd || !weights || !y) return AQ_ERR_NULL;
  if (tokens <= 0 || d <= 0 || d % 4 || topk <= 0 || yd_rows <= 0 || yd_rows > (1 << 30)) return AQ_ERR_SHAPE;
  if (!aligned(yd, 16) || !aligned(y, 16)) return AQ_ERR_ALIGN;
  int64_t blocks = (tokens * d / 4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (topk <= 8)
    hipLaunchKernelGGL(k_moe_combine<8>, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       yd, slot, weights, y, (int)tokens, (int)d, topk, add, (int)yd_rows);
  else
    hipLaunchKernelGGL(k_moe_combine<0>, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       yd, slot, weights, y, (int)tokens, (int)d, topk, add, (int)yd_rows);
  return launch_status();
}

extern "C" int aq_gemv_f32(const float* w, const float* x, float* y, int64_t n, int64_t k, int32_t tokens,
                           void* stream) {
  if (!w || !x || !y) return AQ_ERR_NULL;
  if (n <= 0 || k <= 0 || tokens <= 0 || n * tokens > (1 << 30)) return AQ_ERR_SHAPE;
  if ((k & 3) == 0 && (!aligned(w, 16) || !aligned(x, 16))) return AQ_ERR_ALIGN;
  hipLaunchKernelGGL(k_gemv_f32, dim3((unsigned)((n * tokens + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w, x, y, (int)n, (int)k, tokens);
  return launch_status();
}
