// int4 (Q4W) and ternary (T2W) prefill GEMMs on CDNA4 matrix cores (v_mfma_f32_16x16x32_f16), gfx950.
//
// Y[M, N] (+)= X[M, K] . deq(W)^T, W in Q4W (uint32 [N, K/8], fp16 scale per `group` weights of a row), X fp16 or
// fp32 [M, K] (fp32 is rounded to fp16 when staged), Y fp32 [M, N], accumulation in fp32. This is the arithmetic of
// llama/kernels/prefill/p_gemm_q4.mojo:106-142 (G = 64) and lfm2/kernels/lk.mojo:458-495 (G = 32); the reference
// dequantises W to fp32 in shared memory and multiplies fp32 cooperative matrices, this kernel dequantises to fp16 in
// registers and multiplies on MFMA.
//
// Tiling. A 256-thread workgroup (4 waves) owns BM = 16*MB rows and BN = 4 * 16*NB columns; wave w owns the column
// strip [16*NB*w, +16*NB) for all BM rows (accumulators MB x NB 16x16 tiles). K advances in super-steps of 128 = four
// MFMA k-steps of 32, with k permuted inside a super-step so that each lane's B operand is one contiguous 16-byte
// load: lane l (column l%16, block b = l/16) takes k = 32b + 8s + {0..7} at MFMA step s, i.e. exactly the four words
// b*4 .. b*4+3 of its row. Each word is dequantised straight into the MFMA B fragment: nibbles t and t+4 of the word
// become one half2 (1024 + (nib ^ 8), via mask and OR with 0x6400), minus 1032, times the fp16 scale. The A operand (X)
// is staged once per workgroup in LDS in fragment order with the same k permutation (halves 0,4,1,5,2,6,3,7 of each
// 8-chunk), so a fragment is one ds_read_b128 per lane; slots are XOR-swizzled to keep staging writes 2-way. LDS is
// double-buffered: the next super-step's X and W are fetched into registers while this one is multiplied.
#include <algorithm>
#include <mutex>

#include "aq_gemm.h"

namespace aq {

// Swizzled LDS slot (16 bytes each) of the A fragment of (row-block mb, step s, lane l).
__device__ __forceinline__ int a_slot(int mb, int s, int l) {
  const int sw = s | (((l >> 4) & 1) << 2);
  return (mb * 4 + s) * 64 + (l ^ sw);
}

// Natural 8 fp16 (as 4 dwords: pairs (0,1),(2,3),(4,5),(6,7)) -> permuted pairs (0,4),(1,5),(2,6),(3,7).
__device__ __forceinline__ uint4 permute8(uint4 d) {
  uint4 e;
  e.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  e.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  e.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  e.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return e;
}

// One Q4W word -> MFMA B fragment (8 fp16 in the permuted k order) scaled by s2 = (scale, scale).
__device__ __forceinline__ half8 dequant_word(uint32_t w, half2v s2) {
  const uint32_t u = w ^ 0x88888888u;
  const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
  half8 out;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t bits = ((u >> (4 * t)) & 0x000F000Fu) | 0x64006400u;
    half2v h = __builtin_bit_cast(half2v, bits);
    h = (h - bias) * s2;
    out[2 * t] = h[0];
    out[2 * t + 1] = h[1];
  }
  return out;
}

// One workgroup computes the BM x (4*NW) tile over super-steps [ks0, ks1). With SPLIT it writes its fp32 partial to
// part[split][M][N]; otherwise to y (store or accumulate).
//
// T2W (FMT = kT2): lane (column n, block b) loads the two words (k-rows (k0 + 32b)/16 and +1) of its column; MFMA
// step s takes word s/2, code positions j = 4(s%2) + t and j + 8 (t = 0..3) as fp16 pairs (1024 + c, via mask and
// OR), minus 1025, times the column's fp16 scale for this 128-group. X is staged with the same pairing: 8-k chunks
// A (k 0..7 of a 16-k word) and B (k 8..15) interleave as (A[4h+t], B[4h+t]).
template <int FMT, int MB, int NB, bool G32, bool XF32, bool ADD, bool SPLIT, int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs ga) {
  const void* __restrict__ xv = ga.x;
  const uint32_t* __restrict__ wq = ga.w;
  const uint16_t* __restrict__ ws = ga.s;
  float* __restrict__ y = ga.y;
  float* __restrict__ part = ga.part;
  const int M = ga.M, N = ga.N, K = ga.K, group = ga.group, mtiles = ga.mtiles, ntiles = ga.ntiles;
  const int splits = ga.splits, sup_per_split = ga.sup_per_split;
  constexpr int BM = 16 * MB;
  constexpr int NW = 16 * NB;                      // columns per wave
  constexpr int UPR = FMT == kT2 ? 8 : 16;          // staging units per row per super-step (16 or 8 k each)
  constexpr int UNITS = BM * UPR;
  constexpr int UPT = (UNITS + 255) / 256;          // units per thread
  constexpr int UL = (FMT == kT2 ? 2 : 1) * (XF32 ? 2 : 1);  // 16-byte loads per unit
  extern __shared__ uint4 lds[];                    // 2 stages x MB*4*64 fragment slots

  int sp = 0, nt, m0, expert = 0;
  if (!tile_of<MODE>(ga, BM, sp, nt, m0, expert)) return;
  const int nsup = (K + kSuper - 1) / kSuper;
  const int ks0 = sp * sup_per_split;
  const int ks1 = min(nsup, ks0 + sup_per_split);
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  // this wave's first column; SwiGLU: gate columns j0 .. j0 + NW/2 - 1 and up columns F + j0 ..
  const int nw0 = MODE == kGroupedSwiglu ? nt * (2 * NW) + wave * (NW / 2) : nt * (4 * NW) + wave * NW;
  const int kw = K >> 3;                       // Q4W words per row
  const int gpr = K / group;

  const __amdgpu_buffer_rsrc_t xr_rsrc = make_rsrc(xv, (uint32_t)((size_t)M * K * (XF32 ? 4 : 2)));
  const size_t wrows = MODE == kDense ? (size_t)N : (size_t)ga.n_per_expert * (size_t)ga.mtiles;  // mtiles = experts
  const __amdgpu_buffer_rsrc_t w_rsrc =
      make_rsrc(wq, (uint32_t)(FMT == kT2 ? (size_t)(K >> 4) * N * 4 : wrows * kw * 4));
  const __amdgpu_buffer_rsrc_t s_rsrc =
      make_rsrc(ws, (uint32_t)(FMT == kT2 ? (size_t)(K >> 7) * N * 2 : wrows * gpr * 2));

  // ---- per-lane B source: NB columns (16 apart) ----
  const int bcol = lane & 15;
  const int bblk = lane >> 4;
  int ncol[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {  // columns past N read zeros and are not stored
    if constexpr (MODE == kGroupedSwiglu)
      ncol[nb] = nb < NB / 2 ? nw0 + nb * 16 + bcol : ga.F + nw0 + (nb - NB / 2) * 16 + bcol;
    else
      ncol[nb] = nw0 + nb * 16 + bcol;
    if (MODE == kGroupedSwiglu && nw0 + (nb % (NB / 2)) * 16 + bcol >= ga.F) ncol[nb] = N;  // past F: invalid
  }
  const uint32_t wrow0 = (uint32_t)expert * (uint32_t)ga.n_per_expert;  // first W row of this tile's expert

  auto load_b = [&](int ks, uint4 (&wv)[NB], float (&sc)[NB][G32 ? 1 : 4]) {
    const int k = ks * kSuper + 32 * bblk;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = ncol[nb];
      const bool ok = k < K && n < N;
      if constexpr (FMT == kT2) {
        const uint32_t kr = (uint32_t)(k >> 4);
        wv[nb].x = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, ok ? (kr * N + n) * 4 : kOOB, 0, 0);
        wv[nb].y = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, ok ? ((kr + 1) * N + n) * 4 : kOOB, 0, 0);
        wv[nb].z = wv[nb].w = 0;
        sc[nb][0] = buf_load_half(s_rsrc, ok ? ((uint32_t)(k >> 7) * N + n) * 2 : kOOB);
      } else {
        const uint32_t wrow = wrow0 + (uint32_t)n;
        const uint32_t row = wrow * kw * 4;
        wv[nb] = buf_load16(w_rsrc, ok ? row + (uint32_t)(k >> 3) * 4 : kOOB);
        if constexpr (G32) {
          sc[nb][0] = buf_load_half(s_rsrc, ok ? wrow * gpr * 2 + (uint32_t)(k / group) * 2 : kOOB);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            sc[nb][j] = buf_load_half(s_rsrc, ok ? wrow * gpr * 2 + (uint32_t)((k + 8 * j) / group) * 2 : kOOB);
        }
      }
    }
  };

  // B fragment of MFMA step s for column block nb.
  auto dequant = [&](int s, const uint4& w4, float scale) -> half8 {
    const _Float16 h = (_Float16)scale;
    const half2v s2 = {h, h};
    if constexpr (FMT == kT2) {
      const uint32_t w = s < 2 ? w4.x : w4.y;
      const half2v bias = {(_Float16)1025.0f, (_Float16)1025.0f};
      half8 out;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 4 * (s & 1) + t;
        const uint32_t bits = ((w >> (2 * j)) & 0x00030003u) | 0x64006400u;
        half2v v = (__builtin_bit_cast(half2v, bits) - bias) * s2;
        out[2 * t] = v[0];
        out[2 * t + 1] = v[1];
      }
      return out;
    } else {
      const uint32_t w = s == 0 ? w4.x : s == 1 ? w4.y : s == 2 ? w4.z : w4.w;
      return dequant_word(w, s2);
    }
  };

  // ---- X staging: unit u = t + 256 i: row r = u / UPR, k offset ku * (16 or 8) ----
  // X row of each staging unit (fixed for the whole K loop): the tile row, or its token through src
  int xrow[UPT];
#pragma unroll
  for (int i = 0; i < UPT; ++i) {
    const int u = threadIdx.x + 256 * i;
    const int g = m0 + u / UPR;
    int m = g;
    if constexpr (MODE != kDense) m = g < ga.rows_total ? (ga.src ? ga.src[g] : g) : -1;
    xrow[i] = ((UNITS % 256 == 0 || u < UNITS) && m >= 0 && m < M) ? m : -1;
  }
  auto load_x = [&](int ks, uint4 (&xr)[UPT][UL]) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = threadIdx.x + 256 * i;
      const int ku = u % UPR;
      const int m = xrow[i];
      const int k = ks * kSuper + ku * (FMT == kT2 ? 16 : 8);
      const bool ok = m >= 0 && k < K;
      const uint32_t e = ((uint32_t)m * K + k) * (XF32 ? 4 : 2);  // byte offset
#pragma unroll
      for (int q = 0; q < UL; ++q) xr[i][q] = buf_load16(xr_rsrc, ok ? e + 16 * q : kOOB);
    }
  };
  auto store_x = [&](int buf, const uint4 (&xr)[UPT][UL]) {
    uint4* base = lds + buf * (MB * 256);
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = threadIdx.x + 256 * i;
      if (UNITS % 256 == 0 || u < UNITS) {
        const int r = u / UPR;
        const int ku = u % UPR;
        uint4 c[FMT == kT2 ? 2 : 1];  // fp16 8-k chunks of this unit
#pragma unroll
        for (int q = 0; q < (FMT == kT2 ? 2 : 1); ++q) {
          if constexpr (XF32) {
            const uint4 a = xr[i][2 * q], b = xr[i][2 * q + 1];
            c[q].x = pack_half2(__uint_as_float(a.x), __uint_as_float(a.y));
            c[q].y = pack_half2(__uint_as_float(a.z), __uint_as_float(a.w));
            c[q].z = pack_half2(__uint_as_float(b.x), __uint_as_float(b.y));
            c[q].w = pack_half2(__uint_as_float(b.z), __uint_as_float(b.w));
          } else {
            c[q] = xr[i][q];
          }
        }
        if constexpr (FMT == kT2) {
          const int l = (ku >> 1) * 16 + (r & 15);
          const int s0 = 2 * (ku & 1);
          const uint4 A = c[0], B = c[1];
          uint4 f0, f1;
          f0.x = __builtin_amdgcn_perm(B.x, A.x, 0x05040100u);
          f0.y = __builtin_amdgcn_perm(B.x, A.x, 0x07060302u);
          f0.z = __builtin_amdgcn_perm(B.y, A.y, 0x05040100u);
          f0.w = __builtin_amdgcn_perm(B.y, A.y, 0x07060302u);
          f1.x = __builtin_amdgcn_perm(B.z, A.z, 0x05040100u);
          f1.y = __builtin_amdgcn_perm(B.z, A.z, 0x07060302u);
          f1.z = __builtin_amdgcn_perm(B.w, A.w, 0x05040100u);
          f1.w = __builtin_amdgcn_perm(B.w, A.w, 0x07060302u);
          base[a_slot(r >> 4, s0, l)] = f0;
          base[a_slot(r >> 4, s0 + 1, l)] = f1;
        } else {
          const int l = (ku >> 2) * 16 + (r & 15);
          base[a_slot(r >> 4, ku & 3, l)] = permute8(c[0]);
        }
      }
    }
  };

  float4v acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};

  uint4 xr[UPT][UL];
  uint4 wv[NB];
  float sc[NB][G32 ? 1 : 4];
  load_x(ks0, xr);
  load_b(ks0, wv, sc);
  store_x(0, xr);
  __syncthreads();

  // The loop body is one basic block: on the last step the prefetch re-reads the current slice and its LDS store goes
  // to the idle buffer, which nothing reads again.
  for (int ks = ks0; ks < ks1; ++ks) {
    const int buf = (ks - ks0) & 1;
    uint4 wn[NB];
    float sn[NB][G32 ? 1 : 4];
    const int kn = ks + 1 < ks1 ? ks + 1 : ks;  // the last step re-fetches its own slice (in bounds, unused)
    load_x(kn, xr);
    load_b(kn, wn, sn);
    const uint4* abase = lds + buf * (MB * 256);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 a[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a[mb] = __builtin_bit_cast(half8, abase[a_slot(mb, s, lane)]);
      half8 bf[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bf[nb] = dequant(s, wv[nb], sc[nb][G32 ? 0 : s]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mb], bf[nb], acc[mb][nb], 0, 0, 0);
    }
    store_x(buf ^ 1, xr);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      wv[nb] = wn[nb];
#pragma unroll
      for (int j = 0; j < (G32 ? 1 : 4); ++j) sc[nb][j] = sn[nb][j];
    }
    __syncthreads();
  }

  gemm_store<MB, NB, ADD, SPLIT, MODE>(ga, acc, m0, nw0, sp, lane);
}

// y[i] = (add ? y[i] : 0) + sum_{s < splits} part[s][i], summed in split order (deterministic).
// S > 0: the split count at compile time, so every partial of a thread's four outputs is requested before the first
// add (a loop over a run-time count waited for each load before requesting the next). S = 0: any count. The sums
// run in split order either way.
template <int S>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, float* __restrict__ y,
                                                       int64_t count, int splits, int add) {
  const int64_t n4 = count >> 2;
  const float4* p4 = reinterpret_cast<const float4*>(part);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    float4 acc = add ? y4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (S > 0) {
      float4 v[S];
#pragma unroll
      for (int s = 0; s < S; ++s) v[s] = p4[(int64_t)s * n4 + i];
#pragma unroll
      for (int s = 0; s < S; ++s) acc.x += v[s].x, acc.y += v[s].y, acc.z += v[s].z, acc.w += v[s].w;
    } else {
#pragma unroll 8
      for (int s = 0; s < splits; ++s) {
        const float4 v = p4[(int64_t)s * n4 + i];
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
    }
    y4[i] = acc;
  }
  for (int64_t i = (n4 << 2) + blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
    float acc = add ? y[i] : 0.f;
    for (int s = 0; s < splits; ++s) acc += part[(int64_t)s * count + i];
    y[i] = acc;
  }
}

struct GemmPlan {
  int mb, nb, mtiles, ntiles, splits, sup_per_split;
};

// Tiles of at most max_mb 16-row blocks (the fewest that cover M with that many tiles: 431 -> 4 x 112 at 7) and
// `cols` columns; K split while the workgroups stay within `fill`, each split keeping >= 2 super-steps.
constexpr int kMaxMB = 7;  // accumulators and operands of a wave stay in 256 VGPRs
static GemmPlan plan_tiles(int M, int N, int K, int max_mb, int cols, int fill) {
  GemmPlan p;
  const int blocks16 = (M + 15) / 16;
  p.nb = cols / 64;
  p.mtiles = (blocks16 + max_mb - 1) / max_mb;
  p.mb = (blocks16 + p.mtiles - 1) / p.mtiles;
  p.ntiles = (N + cols - 1) / cols;
  const int nsup = (K + kSuper - 1) / kSuper;
  const int tiles = p.mtiles * p.ntiles;
  int s = 1;
  while (tiles * s * 2 <= fill && nsup / (s * 2) >= 2) s *= 2;
  p.sup_per_split = (nsup + s - 1) / s;
  p.splits = (nsup + p.sup_per_split - 1) / p.sup_per_split;
  return p;
}

// 256-column tiles of up to 112 rows, K split to cover the 256 CUs (up to 320 workgroups). For the direct-to-LDS
// kernel (narrow_ok), shapes whose splits would hold only a few super-steps take 128-column tiles instead, which
// need fewer splits (and fp32 partials): with <= 4 super-steps a split, tiles of 2, 3 or 4 row blocks, whichever
// gives the most workgroups within one per CU (fewer splits on a tie); with <= 8, tiles of up to 7 blocks.
// Same-process A/B on MI355X at M = 431: q|k|v (3072 x 2048) 23.4 -> 15.9 us (3 blocks, no split), o (2048 x 2048)
// 22.0 -> 12.8 (2 blocks, no split; 4 blocks and 2 splits: 16.2), down (2048 x 8192) 30.3 -> 28.3 (7 blocks,
// 4 splits). Longer splits lose: the ternary 4096 x 12288 at M = 412 went from 48 to 54 us with 7 blocks and 64
// with 4.
static GemmPlan plan_gemm(int M, int N, int K, bool narrow_ok) {
  GemmPlan p = plan_tiles(M, N, K, kMaxMB, 256, 320);
  // One pass that leaves CUs idle: tiles of 6 or 5 row blocks when they fill more of the chip without a split (the
  // ternary 12288 x 4096 at M = 412: 4 x 48 -> 5 x 48 workgroups, 51.9 -> 47.9 us).
  if (p.splits == 1 && p.mtiles * p.ntiles < 256) {
    for (int mb = kMaxMB - 1; mb >= kMaxMB - 2; --mb) {
      const GemmPlan c = plan_tiles(M, N, K, mb, 256, 320);
      const int t = c.mtiles * c.ntiles;
      if (c.splits == 1 && t <= 256 && t > p.mtiles * p.ntiles) p = c;
    }
  }
  if (!narrow_ok || p.splits == 1 || p.sup_per_split > 8) return p;
  if (p.sup_per_split > 4) return plan_tiles(M, N, K, kMaxMB, 128, 256);
  GemmPlan best = plan_tiles(M, N, K, 4, 128, 256);
  for (int mb = 2; mb < 4; ++mb) {  // more workgroups within one per CU; fewer splits on a tie
    const GemmPlan c = plan_tiles(M, N, K, mb, 128, 256);
    const int wc = c.mtiles * c.ntiles * c.splits, wb = best.mtiles * best.ntiles * best.splits;
    if (wc <= 256 && (wc > wb || (wc == wb && c.splits < best.splits))) best = c;
  }
  return best;
}

static int64_t gemm_workspace_bytes(const GemmPlan& p, int M, int N) {
  return p.splits > 1 ? (int64_t)p.splits * M * N * 4 : 0;
}

template <int FMT, int MB, bool G32, bool XF32, bool ADD, bool SPLIT>
static int launch_gemm(const void* x, const uint32_t* wq, const uint16_t* ws, float* y, float* part, int M, int N,
                       int K, int group, const GemmPlan& p, hipStream_t s) {
  constexpr int NB = 4;
  int blocks = p.mtiles * p.ntiles * p.splits;
  blocks = (blocks + 7) / 8 * 8;  // extra workgroups exit at once; a multiple of 8 enables the XCD mapping
  GemmArgs ga{};
  ga.x = x; ga.w = wq; ga.s = ws; ga.y = y; ga.part = part;
  ga.M = M; ga.N = N; ga.K = K; ga.group = group; ga.mtiles = p.mtiles; ga.ntiles = p.ntiles;
  ga.splits = p.splits; ga.sup_per_split = p.sup_per_split;
  if constexpr (FMT == kQ4 && G32 && !XF32) {
    if (x16_shape_ok(K, group)) return launch_gemm_x16(ga, kQ4, MB, p.nb, ADD, SPLIT, kDense, blocks, s);
  }
  if constexpr (FMT == kT2 && !XF32) return launch_gemm_x16(ga, kT2, MB, p.nb, ADD, SPLIT, kDense, blocks, s);
  const size_t lds = 2 * (size_t)MB * 256 * 16;
  auto kern = k_gemm<FMT, MB, NB, G32, XF32, ADD, SPLIT, kDense>;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return AQ_ERR_CAPACITY;
  }
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, ga);
  return launch_status();
}

template <int FMT, bool G32, bool XF32, bool ADD, bool SPLIT>
static int gemm_mb(const void* x, const uint32_t* wq, const uint16_t* ws, float* y, float* part, int M, int N,
                   int K, int group, const GemmPlan& p, hipStream_t s) {
  switch (p.mb) {
    case 1: return launch_gemm<FMT, 1, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    case 2: return launch_gemm<FMT, 2, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    case 3: return launch_gemm<FMT, 3, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    case 4: return launch_gemm<FMT, 4, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    case 5: return launch_gemm<FMT, 5, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    case 6: return launch_gemm<FMT, 6, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
    default: return launch_gemm<FMT, 7, G32, XF32, ADD, SPLIT>(x, wq, ws, y, part, M, N, K, group, p, s);
  }
}

template <int FMT, bool G32, bool XF32>
static int gemm_dispatch(const void* x, const uint32_t* wq, const uint16_t* ws, float* y, float* part, int M, int N,
                         int K, int group, int add, const GemmPlan& p, hipStream_t s) {
  if (p.splits > 1) {
    int st = gemm_mb<FMT, G32, XF32, false, true>(x, wq, ws, y, part, M, N, K, group, p, s);
    if (st != AQ_OK) return st;
    const int64_t count = (int64_t)M * N;
    int64_t blocks = (count / 4 + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    if (blocks < 1) blocks = 1;
    const dim3 grid((unsigned)blocks), block(256);
    switch (p.splits) {
      case 2: hipLaunchKernelGGL(k_splitk_reduce<2>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 3: hipLaunchKernelGGL(k_splitk_reduce<3>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 4: hipLaunchKernelGGL(k_splitk_reduce<4>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 5: hipLaunchKernelGGL(k_splitk_reduce<5>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 6: hipLaunchKernelGGL(k_splitk_reduce<6>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 7: hipLaunchKernelGGL(k_splitk_reduce<7>, grid, block, 0, s, part, y, count, p.splits, add); break;
      case 8: hipLaunchKernelGGL(k_splitk_reduce<8>, grid, block, 0, s, part, y, count, p.splits, add); break;
      default: hipLaunchKernelGGL(k_splitk_reduce<0>, grid, block, 0, s, part, y, count, p.splits, add);
    }
    return launch_status();
  }
  return add ? gemm_mb<FMT, G32, XF32, true, false>(x, wq, ws, y, part, M, N, K, group, p, s)
             : gemm_mb<FMT, G32, XF32, false, false>(x, wq, ws, y, part, M, N, K, group, p, s);
}

static int noalloc_scratch(hipStream_t s, void** ptr);

// noalloc (aq_gemm_q4_noalloc): the split-K partials go to this file's static scratch array, whose size ws_bytes
// gives, and a shape whose partials exceed it is refused instead of running in one pass.
template <int FMT>
static int gemm_entry(const void* x, int xf32, const uint32_t* wq, const uint16_t* ws, float* y, int64_t m,
                      int64_t n, int64_t k, int32_t group, int32_t add, void* workspace, int64_t ws_bytes,
                      void* stream, bool noalloc = false) {
  if (!x || !wq || !ws || !y) return AQ_ERR_NULL;
  if (m <= 0 || n <= 0 || k <= 0 || k % (FMT == kT2 ? 128 : 32)) return AQ_ERR_SHAPE;
  if (m > (1 << 24) || n > (1 << 24) || k > (1 << 24)) return AQ_ERR_SHAPE;
  if (FMT == kQ4 && (group <= 0 || group % 8 || k % group)) return AQ_ERR_GROUP;
  // buffer offsets are 32-bit: each operand (X, W, Y and each split's partial slab of M x N floats) stays under 2 GiB
  if (m * k * (xf32 ? 4 : 2) >= ((int64_t)1 << 31) || n * k / (FMT == kT2 ? 4 : 2) >= ((int64_t)1 << 31) ||
      m * n * 4 >= ((int64_t)1 << 31))
    return AQ_ERR_CAPACITY;
  if (!aligned(wq, 16) || !aligned(x, 16) || !aligned(y, 16)) return AQ_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int M = (int)m, N = (int)n, K = (int)k;
  const bool g32 = FMT == kT2 || group % 32 == 0;
  if (FMT == kT2) group = 128;
  GemmPlan p = plan_gemm(M, N, K, !xf32 && g32 && x16_shape_ok(K, group));
  if (noalloc) {
    workspace = nullptr;
    if (p.splits > 1) {
      if (gemm_workspace_bytes(p, M, N) > ws_bytes) return AQ_ERR_CAPACITY;
      const int st = noalloc_scratch(s, &workspace);
      if (st != AQ_OK) return st;
    }
  }
  if (p.splits > 1 && (!workspace || ws_bytes < gemm_workspace_bytes(p, M, N) || !aligned(workspace, 16))) {
    p.splits = 1;  // no (or too small a) workspace: one pass over K
    p.sup_per_split = (K + kSuper - 1) / kSuper;
  }
  float* part = static_cast<float*>(workspace);
  if (xf32) return g32 ? gemm_dispatch<FMT, true, true>(x, wq, ws, y, part, M, N, K, group, add, p, s)
                       : gemm_dispatch<FMT, false, true>(x, wq, ws, y, part, M, N, K, group, add, p, s);
  return g32 ? gemm_dispatch<FMT, true, false>(x, wq, ws, y, part, M, N, K, group, add, p, s)
             : gemm_dispatch<FMT, false, false>(x, wq, ws, y, part, M, N, K, group, add, p, s);
}

// ---- grouped (MoE) GEMM ----------------------------------------------------------------------------------------
// Grouped tiles are 128 columns wide (64 of gate and 64 of up in the SwiGLU form): twice the workgroups of 256-column
// tiles, which hides more of the weight stream's latency. C3 (T = 404, 48-row tiles): 0.183 -> 0.153 ms a block.
constexpr int kGroupedNB = 2;
template <int MB, bool G32, bool XF32, int MODE>
static int launch_grouped(const GemmArgs& ga0, int max_tiles, hipStream_t s) {
  constexpr int NB = 4;
  const size_t lds = 2 * (size_t)MB * 256 * 16;
  auto kern = k_gemm<kQ4, MB, NB, G32, XF32, false, false, MODE>;
  GemmArgs ga = ga0;
  const bool x16 = G32 && !XF32 && x16_shape_ok(ga.K, ga.group);
  const int nbx = x16 ? kGroupedNB : NB;
  ga.ntiles = MODE == kGroupedSwiglu ? (ga.F + 2 * 16 * nbx - 1) / (2 * 16 * nbx) : (ga.N + 64 * nbx - 1) / (64 * nbx);
  ga.splits = 1;
  ga.sup_per_split = (ga.K + kSuper - 1) / kSuper;
  const int blocks = ga.ntiles * max_tiles;
  if (blocks <= 0) return AQ_OK;
  if (x16) return launch_gemm_x16(ga, kQ4, MB, nbx, false, false, MODE, blocks, s);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, ga);
  return launch_status();
}

template <bool G32, bool XF32, int MODE>
static int grouped_mb(const GemmArgs& ga, int mb, int max_tiles, hipStream_t s) {
  switch (mb) {
    case 1: return launch_grouped<1, G32, XF32, MODE>(ga, max_tiles, s);
    case 2: return launch_grouped<2, G32, XF32, MODE>(ga, max_tiles, s);
    case 3: return launch_grouped<3, G32, XF32, MODE>(ga, max_tiles, s);
    case 4: return launch_grouped<4, G32, XF32, MODE>(ga, max_tiles, s);
    case 5: return launch_grouped<5, G32, XF32, MODE>(ga, max_tiles, s);
    case 6: return launch_grouped<6, G32, XF32, MODE>(ga, max_tiles, s);
    default: return launch_grouped<7, G32, XF32, MODE>(ga, max_tiles, s);
  }
}

}  // namespace aq

// Grouped int4 GEMM over experts (see include/aq.h).
extern "C" int aq_moe_gemm_q4(const void* x, int32_t x_is_f32, int64_t x_rows, const int32_t* src,
                              const uint32_t* wq, const uint16_t* ws, int64_t experts, int64_t n, int64_t k,
                              int32_t group, const int32_t* tiles, const int32_t* ntiles, int32_t max_tiles,
                              int32_t tm, int64_t rows_total, int32_t swiglu, void* out, void* stream) {
  using namespace aq;
  if (!x || !wq || !ws || !tiles || !ntiles || !out) return AQ_ERR_NULL;
  if (x_rows <= 0 || experts <= 0 || n <= 0 || k <= 0 || k % 32 || max_tiles < 0 || rows_total <= 0)
    return AQ_ERR_SHAPE;
  if (tm % 16 || tm < 16 || tm > 16 * kMaxMB) return AQ_ERR_SHAPE;
  if (swiglu && n % 2) return AQ_ERR_SHAPE;
  if (group <= 0 || group % 8 || k % group) return AQ_ERR_GROUP;
  if (experts * n * k / 2 >= ((int64_t)1 << 31) || x_rows * k * (x_is_f32 ? 4 : 2) >= ((int64_t)1 << 31) ||
      rows_total * n * 4 >= ((int64_t)1 << 31))
    return AQ_ERR_CAPACITY;
  if (!aligned(wq, 16) || !aligned(x, 16)) return AQ_ERR_ALIGN;
  GemmArgs ga{};
  ga.x = x; ga.w = wq; ga.s = ws;
  ga.y = static_cast<float*>(out);
  ga.act = static_cast<uint16_t*>(out);
  ga.tiles = tiles; ga.ntiles_dev = ntiles; ga.src = src;
  ga.M = (int)x_rows; ga.N = (int)n; ga.K = (int)k; ga.group = group;
  ga.mtiles = (int)experts;  // grouped launches keep the expert count here (W rows = experts * n)
  ga.n_per_expert = (int)n; ga.F = (int)(n / 2); ga.rows_total = (int)rows_total;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int mb = tm / 16;
  const bool g32 = group % 32 == 0;
  if (swiglu) {
    if (x_is_f32) return g32 ? grouped_mb<true, true, kGroupedSwiglu>(ga, mb, max_tiles, st)
                             : grouped_mb<false, true, kGroupedSwiglu>(ga, mb, max_tiles, st);
    return g32 ? grouped_mb<true, false, kGroupedSwiglu>(ga, mb, max_tiles, st)
               : grouped_mb<false, false, kGroupedSwiglu>(ga, mb, max_tiles, st);
  }
  if (x_is_f32) return g32 ? grouped_mb<true, true, kGrouped>(ga, mb, max_tiles, st)
                           : grouped_mb<false, true, kGrouped>(ga, mb, max_tiles, st);
  return g32 ? grouped_mb<true, false, kGrouped>(ga, mb, max_tiles, st)
             : grouped_mb<false, false, kGrouped>(ga, mb, max_tiles, st);
}

namespace aq {
}  // namespace aq

// ---- the allocation-free variant of aq_gemm_q4 ------------------------------------------------------------------
// Its split-K partials live in `scratch`, one array per GPU (the device code object's copy, held until the process
// ends); calls on one GPU share it, so calls that overlap there race. Host code never passes the array's name (a
// host-side stand-in, not a device address) to a kernel: the device address comes from hipGetSymbolAddress, once per
// device with that device current, and is kept per device.
static __device__ __align__(256) uint8_t scratch[AQ_GEMM_NOALLOC_SCRATCH_BYTES];

namespace aq {

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int noalloc_scratch(hipStream_t s, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return AQ_ERR_LAUNCH;
  if (s) {  // the stream's device must be the current one: the symbol is looked up on the current device
    int sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess) return AQ_ERR_LAUNCH;
    if (sdev != dev) return AQ_ERR_ARG;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return AQ_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return AQ_OK;
}

}  // namespace aq

extern "C" int aq_gemm_q4_noalloc(const void* x, int32_t x_is_f32, const uint32_t* wq, const uint16_t* ws, float* y,
                                  int64_t m, int64_t n, int64_t k, int32_t group, int32_t add, void* stream) {
  return aq::gemm_entry<aq::kQ4>(x, x_is_f32, wq, ws, y, m, n, k, group, add, nullptr, AQ_GEMM_NOALLOC_SCRATCH_BYTES,
                                 stream, true);
}

extern "C" int aq_gemm_q4(const void* x, int32_t x_is_f32, const uint32_t* wq, const uint16_t* ws, float* y,
                          int64_t m, int64_t n, int64_t k, int32_t group, int32_t add, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  return aq::gemm_entry<aq::kQ4>(x, x_is_f32, wq, ws, y, m, n, k, group, add, workspace, workspace_bytes, stream);
}

extern "C" int aq_gemm_t2(const void* x, int32_t x_is_f32, const uint32_t* w, const uint16_t* s, float* y, int64_t m,
                          int64_t n, int64_t k, int32_t add, void* workspace, int64_t workspace_bytes, void* stream) {
  return aq::gemm_entry<aq::kT2>(x, x_is_f32, w, s, y, m, n, k, 128, add, workspace, workspace_bytes, stream);
}

extern "C" int64_t aq_gemm_t2_workspace_bytes(int64_t m, int64_t n, int64_t k);
extern "C" int64_t aq_gemm_q4_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || m > (1 << 24) || n > (1 << 24) || k > (1 << 24)) return 0;
  // the larger of the two tilings' needs: which one runs depends on X's type and the group
  const aq::GemmPlan a = aq::plan_gemm((int)m, (int)n, (int)k, false), b = aq::plan_gemm((int)m, (int)n, (int)k, true);
  return std::max(aq::gemm_workspace_bytes(a, (int)m, (int)n), aq::gemm_workspace_bytes(b, (int)m, (int)n));
}

extern "C" int64_t aq_gemm_t2_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  return aq_gemm_q4_workspace_bytes(m, n, k);
}
