// int4 (Q4W) prefill GEMM for fp16 X with one scale per 32-k chunk (group % 32 == 0) on CDNA4 matrix cores, gfx950:
// the same product as aq_gemm.hip (llama/kernels/prefill/p_gemm_q4.mojo:106-142, lfm2/kernels/lk.mojo:458-495,
// lfm2moe grouped p_gemm_q4g), with X staged by direct global-to-LDS loads. Built without the VGPR-form MFMA flag:
// the accumulators live in AGPRs, which leaves the VGPRs to the operands.
#include "aq_gemm.h"

namespace aq {

// ---- int4 GEMM for fp16 X, K % 128 == 0, group a power of two >= 32: direct-to-LDS staging ----------------------
//
// The MFMA k slots follow X's natural order: at step s of a super-step, lane l (row or column l%16, block b = l/16)
// holds k = k0 + 32b + 8s + {0..7}. The A fragment of (row block mb, step s) is therefore 64 contiguous 16-byte pieces
// of X, one per lane, and is fetched by one buffer_load_dwordx4 ... lds straight into fragment order (no registers,
// no VALU, conflict-free ds_read_b128). Wave w fetches the fragments of step w for every row block. The B side is
// the lane's word s of its 32-k chunk: byte t of the word holds k = 2t (low nibble) and 2t+1 (high nibble). One
// v_perm_b32 copies byte t under the exponent bytes 0x64 (low half) and 0x54 (high half); masking the other nibble and
// flipping bit 3 of the kept one (v_bitop3) gives the fp16 pair (1024 + q_lo, 64 + q_hi) with q = nib ^ 8, since the
// mantissa LSB weighs 1 at 1024 and 1/16 at 64. Minus (1032, 72) this is the signed nibble exactly, times the scale.
// Two named LDS buffers alternate, so the direct loads into one never alias the fragment reads of the other.
__device__ __forceinline__ half8 dequant_q4_natural(uint32_t w, uint32_t s2bits) {
  const uint32_t magic = 0x00005464u;  // bytes 4, 5 of the v_perm source pair: 0x64, 0x54
  const half2v s2 = __builtin_bit_cast(half2v, s2bits);
  const half2v bias = {(_Float16)1032.0f, (_Float16)72.0f};
  half8 out;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t sel = 0x05000400u | ((uint32_t)t << 16) | (uint32_t)t;
    const uint32_t x = (__builtin_amdgcn_perm(magic, w, sel) & 0xFFF0FF0Fu) ^ 0x00800008u;
    const half2v h = (__builtin_bit_cast(half2v, x) - bias) * s2;
    out[2 * t] = h[0];
    out[2 * t + 1] = h[1];
  }
  return out;
}

// 16 bytes per lane from `r` at byte offset `off` into LDS at dst + 16 * lane (dst wave-uniform). A device-only
// function: the address-space cast must not appear in host-visible code such as a lambda.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint4* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, 0);
}

// T2W (ternary) word w holds the 2-bit codes of 16 consecutive k of one column, code i at bits 2i; half h (k 8h .. 8h + 7)
// is one MFMA step's B operand. Pair t = (code 2t, 2t + 1) sits in byte 2h + t/2 at bits 4(t % 2) and 4(t % 2) + 2.
// v_perm copies that byte under two exponent bytes whose mantissa LSB makes the code's bits weigh 1: 0x64 (1024) and
// 0x5C (256) for bits 0 and 2, 0x54 (64) and 0x4C (16) for bits 4 and 6; masking the other codes gives (1024 + c,
// 256 + c') or (64 + c, 16 + c'), minus (1025, 257) / (65, 17) is (c - 1, c' - 1) exactly, times the scale.
__device__ __forceinline__ half8 dequant_t2_natural(uint32_t w, int h, uint32_t s2bits) {
  const uint32_t magic = 0x4C545C64u;  // bytes 4..7 of the v_perm source pair: 0x64, 0x5C, 0x54, 0x4C
  const half2v s2 = __builtin_bit_cast(half2v, s2bits);
  half8 out;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t b = (uint32_t)(2 * h + (t >> 1));
    const uint32_t sel = ((t & 1) ? 0x07000600u : 0x05000400u) | (b << 16) | b;
    const uint32_t mask = (t & 1) ? 0xFFC0FF30u : 0xFF0CFF03u;
    const half2v bias = (t & 1) ? half2v{(_Float16)65.0f, (_Float16)17.0f} : half2v{(_Float16)1025.0f, (_Float16)257.0f};
    const uint32_t x = __builtin_amdgcn_perm(magic, w, sel) & mask;
    const half2v v = (__builtin_bit_cast(half2v, x) - bias) * s2;
    out[2 * t] = v[0];
    out[2 * t + 1] = v[1];
  }
  return out;
}

// FMT kQ4: Q4W rows [N, K/8] with fp16 scales [N, K/group]; kT2: T2W words [K/16, N] with scales [K/128, N] (dense
// mode only). T2W is column-contiguous, so its loads are coalesced in the MFMA B layout directly (no ds_bpermute).
// W8: 512 threads, two groups of four waves run the same tile over the two halves of the workgroup's super-steps
// (each with its own pair of X buffers), and their accumulators are summed through LDS at the end. A SIMD then holds
// two waves, so one wave's dequantisation issues while the other's MFMAs run: with one wave per SIMD in-order issue
// leaves most of the VALU work outside the MFMA shadow. The caller gives W8 an even number of super-steps.
// NB = 2 (narrow tiles, four waves, dense only): each wave takes 32 columns, a workgroup 128, so shapes with few
// 256-column tiles need fewer K splits (and fp32 partials) to fill the chip.
// The lane index computed where it is used (not merged with an earlier computation), so that nothing derived from
// the thread index has to stay in a register across the main loop.
__device__ __forceinline__ int fresh_lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

template <int FMT, int MB, int NB, bool ADD, bool SPLIT, int MODE, bool W8>
__global__ __launch_bounds__(W8 ? 512 : 256) void k_gemm_x16(GemmArgs ga) {
  const uint32_t* __restrict__ wq = ga.w;
  const uint16_t* __restrict__ ws = ga.s;
  const int M = ga.M, N = ga.N, K = ga.K, group = ga.group;
  constexpr int BM = 16 * MB;
  constexpr int NW = 16 * NB;
  constexpr int FR = MB * 4 * 64;  // uint4 slots per buffer: MB row blocks x 4 steps x 64 lanes
  static_assert(NB == 4 || (NB == 2 && (MODE == kDense || !W8)), "W prefetch: one column block per MFMA step");
  __shared__ uint4 xbuf[(W8 ? 4 : 2) * FR];

  int sp = 0, nt, m0, expert = 0;
  if (!tile_of<MODE>(ga, BM, sp, nt, m0, expert)) return;
  const int nsup = (K + kSuper - 1) / kSuper;
  int ks0 = sp * ga.sup_per_split;
  int ks1 = min(nsup, ks0 + ga.sup_per_split);
  const int lane = threadIdx.x & 63;
  // wave-uniform, in scalar registers: the epilogue needs them after the loop, and no vector register has to hold
  // them (or the thread index) through it
  const int grp = W8 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8)) : 0;  // this group's half of the K range
  const int wave = __builtin_amdgcn_readfirstlane((int)((threadIdx.x >> 6) & 3));     // the wave within its group
  if constexpr (W8) {
    const int half = (ks1 - ks0) >> 1;
    ks0 += grp * half;
    ks1 = ks0 + half;
  }
  uint4* const xa = xbuf + 2 * grp * FR;
  uint4* const xb = xa + FR;
  const int nw0 = MODE == kGroupedSwiglu ? nt * (2 * NW) + wave * (NW / 2) : nt * (4 * NW) + wave * NW;
  const int kw = K >> 3;
  const int gpr = K / group;
  const int gsh = 31 - __builtin_clz(group);  // group is a power of two >= 32 here (128 for T2W)

  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(ga.x, (uint32_t)((size_t)M * K * 2));
  const size_t wrows = MODE == kDense ? (size_t)N : (size_t)ga.n_per_expert * (size_t)ga.mtiles;
  const __amdgpu_buffer_rsrc_t w_rsrc =
      make_rsrc(wq, (uint32_t)(FMT == kT2 ? (size_t)(K >> 4) * N * 4 : wrows * kw * 4));
  const __amdgpu_buffer_rsrc_t s_rsrc =
      make_rsrc(ws, (uint32_t)(FMT == kT2 ? (size_t)(K >> 7) * N * 2 : wrows * gpr * 2));

  // ---- staging. LDS block (mb, j) (1 KB) holds rows 16mb .. +15 of the tile over the j-th 32-k chunk of the
  // super-step: row r's four 8-k pieces s sit in slots 4r + (s ^ sw(r)), sw(r) = (r >> 2) & 3, which makes the
  // fragment reads below conflict-free. Wave w fetches chunk j = w of every row block; lane L takes row L/4 and slot
  // L%4, so four consecutive lanes read one row's 64 contiguous bytes.
  const int srow = lane >> 2;
  const int spiece = (lane & 3) ^ ((srow >> 2) & 3);
  uint32_t xoff[MB];  // byte offset of this lane's X row (kOOB past the end) plus its piece
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int g = m0 + mb * 16 + srow;
    int m = g;
    if constexpr (MODE != kDense) m = g < ga.rows_total ? (ga.src ? ga.src[g] : g) : -1;
    xoff[mb] = ((m >= 0 && m < M) ? (uint32_t)m * (uint32_t)K * 2u : kOOB) + (uint32_t)spiece * 16u;
  }
  const int wave_u = wave;
  auto stage = [&](int ks, uint4* dst, int mb) {
    const int k = ks * kSuper + 32 * wave_u;  // K % 128 == 0: always inside the row
    lds_load16(x_rsrc, dst + (mb * 4 + wave_u) * 64, xoff[mb] + (uint32_t)k * 2u);
  };
  // fragment (mb, s) of this lane: block (mb, lane / 16), row lane % 16, piece s
  const int arow = lane & 15;
  const int aslot = (lane >> 4) * 64 + 4 * arow;
  const int asw = (arow >> 2) & 3;

  // ---- B source. Loads use a coalesced lane pattern: loader lane L = 4r + p fetches piece p (16 bytes: 32 k) of
  // the super-step's 64 bytes of row r of a 16-column block, and its row's scale p & smask, so four consecutive lanes
  // read contiguous memory. ds_bpermute then moves each word to the MFMA B layout (lane l = column l % 16, piece
  // l / 16): the source of lane l is loader lane 4 (l % 16) + l / 16, and for its scale 4 (l % 16) + its group's index
  // within the super-step.
  const int lrow = lane >> 2;
  const int lpiece = lane & 3;
  const int smask = max((kSuper >> gsh) - 1, 0);  // scales per row and super-step, minus one (3, 1 or 0)
  // Columns past the end read the last valid row instead (their sums are never stored), so the loads in the loop
  // need no condition: a select there is turned into branches around the loads, with waits between them.
  uint32_t wrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int n;
    if constexpr (MODE == kGroupedSwiglu) {
      const int j = min(nw0 + (nb % (NB / 2)) * 16 + lrow, ga.F - 1);
      n = nb < NB / 2 ? j : ga.F + j;
    } else {
      n = min(nw0 + nb * 16 + (FMT == kT2 ? (lane & 15) : lrow), N - 1);
    }
    wrow[nb] = (uint32_t)expert * (uint32_t)ga.n_per_expert + (uint32_t)n;  // T2W: the column
  }
  const int waddr = 16 * (lane & 15) + 4 * (lane >> 4);
  const int saddr = 16 * (lane & 15) + 4 * ((32 * (lane >> 4)) >> gsh);
  // raw (loader-layout) W piece and scale bits of column block nb for super-step ks
  auto load_b = [&](int ks, uint4 (&wr)[NB], uint32_t (&sr)[NB], int nb) {
    if constexpr (FMT == kT2) {  // the two words (32 k) of block l / 16 and the column's scale, B layout as loaded
      const uint32_t r = (uint32_t)(ks * (kSuper / 16) + 2 * (lane >> 4));
      wr[nb].x = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, (r * (uint32_t)N + wrow[nb]) * 4u, 0, 0);
      wr[nb].y = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, ((r + 1) * (uint32_t)N + wrow[nb]) * 4u, 0, 0);
      sr[nb] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, ((uint32_t)ks * (uint32_t)N + wrow[nb]) * 2u, 0, 0);
    } else {
      const int k = ks * kSuper + 32 * lpiece;  // K % 128 == 0: always inside the row
      wr[nb] = buf_load16(w_rsrc, wrow[nb] * (uint32_t)kw * 4u + (uint32_t)(k >> 3) * 4u);
      const uint32_t g = (uint32_t)((ks * kSuper) >> gsh) + (uint32_t)(lpiece & smask);
      sr[nb] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, (wrow[nb] * (uint32_t)gpr + g) * 2u, 0, 0);
    }
  };
  auto bperm = [&](int addr, uint32_t v) -> uint32_t {  // T2W arrives in the B layout already
    if constexpr (FMT == kT2) return v;
    else return (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v);
  };

  struct WSet {
    uint4 w[NB];
    uint32_t s[NB];
  };
  float4v acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = float4v{0.f, 0.f, 0.f, 0.f};

  // One super-step: multiply the current slice from `cur` while fetching X of the next one into `nxt` (first, so the
  // barrier can wait for it alone); load_w(s) issues the W loads that belong to MFMA step s. The A fragments and B
  // words of MFMA step s + 1 are read (LDS, ds_bpermute) during step s. Fetches past the end re-read the last slice:
  // the X copy goes to the idle buffer, which nothing reads again. The caller waits and synchronises afterwards.
  auto step = [&](const uint4* cur, uint4* nxt, const WSet& cw, int ks, auto&& load_w) {
    const int kn = ks + 1 < ks1 ? ks + 1 : ks;
    const uint4(&wr)[NB] = cw.w;
    const uint32_t(&sr)[NB] = cw.s;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) stage(kn, nxt, mb);
    uint32_t s2[NB];
    uint32_t bw[2][NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      s2[nb] = bperm(saddr, sr[nb]) * 0x00010001u;  // (scale, scale): the 16-bit load zero-extends
      bw[0][nb] = bperm(waddr, wr[nb].x);
    }
    half8 a[2][MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a[0][mb] = __builtin_bit_cast(half8, cur[mb * 256 + aslot + asw]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      load_w(s);
      if (s < 3) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          a[(s + 1) & 1][mb] = __builtin_bit_cast(half8, cur[mb * 256 + aslot + ((s + 1) ^ asw)]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          bw[(s + 1) & 1][nb] = FMT == kT2 ? (s + 1 < 2 ? wr[nb].x : wr[nb].y)
                                           : bperm(waddr, s == 0 ? wr[nb].y : s == 1 ? wr[nb].z : wr[nb].w);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const half8 b = FMT == kT2 ? dequant_t2_natural(bw[s & 1][nb], s & 1, s2[nb])
                                   : dequant_q4_natural(bw[s & 1][nb], s2[nb]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s & 1][mb], b, acc[mb][nb], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Vector memory loads complete in issue order: waiting until at most N loads issued after this super-step's X loads
  // remain leaves those X loads landed; the barrier makes that true of every wave. vmcnt(N), expcnt and lgkmcnt as
  // they are.
#define AQ_WAIT_X_SYNC(N)                                     \
  do {                                                        \
    __builtin_amdgcn_s_waitcnt(0x0F70 | ((N) & 15) | (((N) >> 4) << 14)); \
    __syncthreads();                                          \
  } while (0)
  const auto no_w = [](int) {};
  if constexpr (MODE != kDense && FMT == kQ4) {
    // Grouped (MoE) tiles stream every weight row once, 64 bytes a super-step, and their short super-steps wait on
    // load latency. Here W is requested in pairs of super-steps: pair (ks + 2, ks + 3) during super-step ks (the two
    // halves of a row's 128-byte line back to back), into the register pair that super-steps ks - 2 and ks - 1 used,
    // so every second super-step's W is requested three ahead with four register sets; the loop is unrolled by 4.
    // Measured on MI355X, C3 at 404 tokens: 0.1547 -> 0.1406 ms a block.
    WSet pa0, pa1, pb0, pb1;
    auto clampk = [&](int k) { return k < ks1 ? k : ks0; };
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) stage(ks0, xa, mb);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      load_b(ks0, pa0.w, pa0.s, nb);
      load_b(clampk(ks0 + 1), pa1.w, pa1.s, nb);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    constexpr int kPairLoads = 4 * NB;  // two super-steps of (piece, scale) per column block
    for (int ks = ks0; ks < ks1; ks += 4) {
      step(xa, xb, pa0, ks, [&](int s) {
        if (s < NB) {
          load_b(clampk(ks + 2), pb0.w, pb0.s, s);
          load_b(clampk(ks + 3), pb1.w, pb1.s, s);
        }
      });
      AQ_WAIT_X_SYNC(kPairLoads);
      if (ks + 1 < ks1) {
        step(xb, xa, pa1, ks + 1, no_w);
        AQ_WAIT_X_SYNC(0);
      }
      if (ks + 2 < ks1) {
        step(xa, xb, pb0, ks + 2, [&](int s) {
          if (s < NB) {
            load_b(clampk(ks + 4), pa0.w, pa0.s, s);
            load_b(clampk(ks + 5), pa1.w, pa1.s, s);
          }
        });
        AQ_WAIT_X_SYNC(kPairLoads);
      }
      if (ks + 3 < ks1) {
        step(xb, xa, pb1, ks + 3, no_w);
        AQ_WAIT_X_SYNC(0);
      }
    }
  } else {
    // Three W register sets rotate by name (the loop below is unrolled by 6 = lcm of 2 X buffers and 3 W sets), so no
    // register that a load is still writing is ever copied: super-step ks multiplies one set while ks + 1's has
    // landed and ks + 2's is in flight, its loads spread over the MFMA steps (one column block each). T2W issues
    // 3 NB loads a super-step, so waiting for 2 NB also waits for some of them.
    WSet w0, w1, w2;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) stage(ks0, xa, mb);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) load_b(ks0, w0.w, w0.s, nb);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) load_b(ks0 + 1 < ks1 ? ks0 + 1 : ks0, w1.w, w1.s, nb);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    auto ahead = [&](WSet& fw, int ks) {
      const int kf = ks + 2 < ks1 ? ks + 2 : ks;
      return [&fw, kf, &load_b](int s) {
        if (s < NB) load_b(kf, fw.w, fw.s, s);
      };
    };
    for (int ks = ks0; ks < ks1; ks += 6) {
      step(xa, xb, w0, ks, ahead(w2, ks));
      AQ_WAIT_X_SYNC(2 * NB);
      if (ks + 1 < ks1) { step(xb, xa, w1, ks + 1, ahead(w0, ks + 1)); AQ_WAIT_X_SYNC(2 * NB); }
      if (ks + 2 < ks1) { step(xa, xb, w2, ks + 2, ahead(w1, ks + 2)); AQ_WAIT_X_SYNC(2 * NB); }
      if (ks + 3 < ks1) { step(xb, xa, w0, ks + 3, ahead(w2, ks + 3)); AQ_WAIT_X_SYNC(2 * NB); }
      if (ks + 4 < ks1) { step(xa, xb, w1, ks + 4, ahead(w0, ks + 4)); AQ_WAIT_X_SYNC(2 * NB); }
      if (ks + 5 < ks1) { step(xb, xa, w2, ks + 5, ahead(w1, ks + 5)); AQ_WAIT_X_SYNC(2 * NB); }
    }
  }
#undef AQ_WAIT_X_SYNC
  if constexpr (W8) {
    // The two groups' sums meet in LDS, each group finishing half of the columns: group 0 column blocks 0 .. NB/2 - 1,
    // group 1 the rest; each first leaves the other's half in LDS. (One group finishing all of them left the other
    // idle through the final stores.) The last step's barrier follows its wait for the X loads: LDS is quiescent and
    // no wave reads it any more. Register arrays are indexed by constants only, so the group picks by selects.
    constexpr int H = NB / 2;
    float4v* red = reinterpret_cast<float4v*>(xbuf);  // [group][wave][MB][H][64]: 4 * FR slots
    const bool g1 = grp != 0;
    const int el = fresh_lane_id();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int h = 0; h < H; ++h)
        red[(((grp * 4 + wave) * MB + mb) * H + h) * 64 + el] = g1 ? acc[mb][h] : acc[mb][H + h];
    __syncthreads();
    float4v out[MB][H];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int h = 0; h < H; ++h)
        out[mb][h] = (g1 ? acc[mb][H + h] : acc[mb][h]) + red[((((1 - grp) * 4 + wave) * MB + mb) * H + h) * 64 + el];
    gemm_store<MB, H, ADD, SPLIT, MODE>(ga, out, m0, nw0 + grp * 16 * H, sp, el);
  } else {
    gemm_store<MB, NB, ADD, SPLIT, MODE>(ga, acc, m0, nw0, sp, fresh_lane_id());
  }
}

template <int FMT, int MB, int NB, int MODE, bool W8>
static void launch_mb(const GemmArgs& ga, bool add, bool split, int blocks, hipStream_t s) {
  const dim3 block(W8 ? 512 : 256);
  if constexpr (MODE != kDense && W8) {
    return;  // not built: grouped launches keep four waves (launch_gemm_x16 takes eight only for dense tiles)
  } else if constexpr (MODE == kDense) {
    if (split) hipLaunchKernelGGL((k_gemm_x16<FMT, MB, NB, false, true, MODE, W8>), dim3(blocks), block, 0, s, ga);
    else if (add) hipLaunchKernelGGL((k_gemm_x16<FMT, MB, NB, true, false, MODE, W8>), dim3(blocks), block, 0, s, ga);
    else hipLaunchKernelGGL((k_gemm_x16<FMT, MB, NB, false, false, MODE, W8>), dim3(blocks), block, 0, s, ga);
  } else {
    hipLaunchKernelGGL((k_gemm_x16<FMT, MB, NB, false, false, MODE, W8>), dim3(blocks), block, 0, s, ga);
  }
}

template <int FMT, int NB, int MODE, bool W8>
static void launch_mode(const GemmArgs& ga, int mb, bool add, bool split, int blocks, hipStream_t s) {
  switch (mb) {
    case 1: return launch_mb<FMT, 1, NB, MODE, W8>(ga, add, split, blocks, s);
    case 2: return launch_mb<FMT, 2, NB, MODE, W8>(ga, add, split, blocks, s);
    case 3: return launch_mb<FMT, 3, NB, MODE, W8>(ga, add, split, blocks, s);
    case 4: return launch_mb<FMT, 4, NB, MODE, W8>(ga, add, split, blocks, s);
    case 5: return launch_mb<FMT, 5, NB, MODE, W8>(ga, add, split, blocks, s);
    case 6: return launch_mb<FMT, 6, NB, MODE, W8>(ga, add, split, blocks, s);
    default: return launch_mb<FMT, 7, NB, MODE, W8>(ga, add, split, blocks, s);
  }
}

template <bool W8>
static void launch_fmt(const GemmArgs& ga, int fmt, int mb, bool add, bool split, int mode, int blocks, hipStream_t s) {
  if (fmt == kT2) launch_mode<kT2, 4, kDense, W8>(ga, mb, add, split, blocks, s);
  else if (mode == kDense) launch_mode<kQ4, 4, kDense, W8>(ga, mb, add, split, blocks, s);
  else if (mode == kGrouped) launch_mode<kQ4, 4, kGrouped, W8>(ga, mb, false, false, blocks, s);
  else launch_mode<kQ4, 4, kGroupedSwiglu, W8>(ga, mb, false, false, blocks, s);
}

// Grouped modes take neither `add` nor split-K, and Q4W only. The caller has checked x16_shape_ok. Every
// workgroup's super-step range has the same even length when sup_per_split is even and divides the super-step count.
// The 8-wave form runs for dense ranges of >= 16 super-steps (same-process A/B: C1's int4 gate|up 40.1 -> 37.8 us,
// C2's ternary GEMM 5-12% faster; with 2-8 super-steps a group, C1's split-K projections lose 5-10%, and C3's
// grouped gate|up goes from 84 to 94 us, so those keep four waves). Narrow tiles follow the same rule (C1's q|k|v
// with 16 super-steps a workgroup: 16.1 -> 15.0 us).
// The eight-wave form takes a whole CU (512 threads, up to 112 KB of LDS); above one workgroup per CU, four waves let
// two workgroups share a CU instead of running a second, partial round: C2's fused ternary gate|up (24576 x 4096 at
// M = 412, 384 workgroups) 96.0 -> 84.6 us.
constexpr int kW8MaxBlocks = 256;
int launch_gemm_x16(const GemmArgs& ga, int fmt, int mb, int nb, bool add, bool split, int mode, int blocks,
                    hipStream_t s) {
  const int nsup = (ga.K + kSuper - 1) / kSuper;
  const int per = ga.sup_per_split;
  const bool w8 = per >= 16 && per % 2 == 0 && nsup % per == 0 && blocks <= kW8MaxBlocks;
  if (nb == 2) {  // narrow tiles
    if (mode == kGrouped) launch_mode<kQ4, 2, kGrouped, false>(ga, mb, false, false, blocks, s);
    else if (mode == kGroupedSwiglu) launch_mode<kQ4, 2, kGroupedSwiglu, false>(ga, mb, false, false, blocks, s);
    else if (w8) {
      if (fmt == kT2) launch_mode<kT2, 2, kDense, true>(ga, mb, add, split, blocks, s);
      else launch_mode<kQ4, 2, kDense, true>(ga, mb, add, split, blocks, s);
    } else {
      if (fmt == kT2) launch_mode<kT2, 2, kDense, false>(ga, mb, add, split, blocks, s);
      else launch_mode<kQ4, 2, kDense, false>(ga, mb, add, split, blocks, s);
    }
    return launch_status();
  }
  if (mode == kDense && w8)
    launch_fmt<true>(ga, fmt, mb, add, split, mode, blocks, s);
  else launch_fmt<false>(ga, fmt, mb, add, split, mode, blocks, s);
  return launch_status();
}

}  // namespace aq
