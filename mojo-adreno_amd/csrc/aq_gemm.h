// Shared pieces of the MFMA GEMM kernels (aq_gemm.hip, aq_gemm_x16.hip): operand types, buffer-resource loads, the
// kernel argument block, the tile decode and the epilogue.
#pragma once
#include "aq_common.h"

namespace aq {

constexpr int kSuper = 128;  // k per super-step

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  return (uint32_t)float_to_half_bits(a) | ((uint32_t)float_to_half_bits(b) << 16);
}

enum { kQ4 = 0, kT2 = 1 };  // weight formats: Q4W rows [N, K/8] / T2W transposed words [K/16, N]

// Kernel arguments (by value). Dense: X [M, K] -> y [M, N]. Grouped (MoE): work tile `it` of tiles[] is (expert e,
// first grouped row m0); X row of grouped row g is src[g] (a token; -1 = padding, zeros) or g itself when src is
// null; W rows of expert e start at e * n_per_expert; output rows are grouped rows (rows_total of them).
struct GemmArgs {
  const void* x;
  const uint32_t* w;
  const uint16_t* s;
  float* y;
  float* part;
  uint16_t* act;           // SwiGLU epilogue output (fp16 bits) [rows_total, F]
  const int* tiles;        // grouped: (expert, first row) pairs
  const int* ntiles_dev;   // grouped: number of valid tiles (device)
  const int* src;          // grouped: token of each grouped row, or null
  int M, N, K, group, mtiles, ntiles, splits, sup_per_split;
  int n_per_expert, F, rows_total;
};

enum { kDense = 0, kGrouped = 1, kGroupedSwiglu = 2 };

// Work tile of this workgroup. Dense: ids are split into (xcd = id % 8, local = id / 8) when the grid is a multiple of
// 8, so each XCD works through a contiguous run; within a run the m-tiles of one (n-tile, split) are adjacent (they
// share W). Grouped: tile it of tiles[] = (expert, first grouped row). Returns false for workgroups with no tile.
template <int MODE>
__device__ __forceinline__ bool tile_of(const GemmArgs& ga, int BM, int& sp, int& nt, int& m0, int& expert) {
  int id = blockIdx.x;
  const int nblk = gridDim.x;
  if constexpr (MODE == kDense) {
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    const int mt = id % ga.mtiles;
    const int rest = id / ga.mtiles;
    sp = rest % ga.splits;
    nt = rest / ga.splits;
    m0 = mt * BM;
    return nt < ga.ntiles;
  } else {
    nt = id % ga.ntiles;
    const int it = id / ga.ntiles;
    if (it >= *ga.ntiles_dev) return false;
    expert = ga.tiles[2 * it];
    m0 = ga.tiles[2 * it + 1];
    return true;
  }
}

// Epilogue shared by the GEMM kernels: lane l holds D[4*(l/16) + r][l%16] of each 16x16 tile; buffer stores drop rows
// and columns past the end.
// Cache policy of the dense GEMM's final fp32 output stores: sc1 | nt (streaming, device scope); the output is
// written once at the end of a one-pass launch. bench.py on MI355X, alternating libraries: C1 gate|up 42.3 -> 41.5 us,
// C2's ternary GEMM 159 -> 154 us a triple. Split-K partials (read back by k_splitk_reduce) and the grouped outputs
// (read back by the combine: the C3 block was 3% slower with nt) keep the default policy.
constexpr int kYPolicy = 18;
template <int MB, int NB, bool ADD, bool SPLIT, int MODE>
__device__ __forceinline__ void gemm_store(const GemmArgs& ga, const float4v (&acc)[MB][NB], int m0, int nw0, int sp,
                                           int lane) {
  const int M = ga.M, N = ga.N;
  float* __restrict__ y = ga.y;
  float* __restrict__ part = ga.part;
  const int bcol = lane & 15;
  const int rq = (lane >> 4) * 4;
  if constexpr (MODE == kGroupedSwiglu) {
    const int F = ga.F;
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(ga.act, (uint32_t)((size_t)ga.rows_total * F * 2));
#pragma unroll
    for (int nb = 0; nb < NB / 2; ++nb) {
      const int j = nw0 + nb * 16 + bcol;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int g = m0 + mb * 16 + rq + r;
          const uint32_t off = j < F ? ((uint32_t)g * F + j) * 2 : kOOB;
          const float v = silu(acc[mb][nb][r]) * acc[mb][nb + NB / 2][r];
          __builtin_amdgcn_raw_buffer_store_b16(float_to_half_bits(v), a_rsrc, off, 0, 0);
        }
      }
    }
  } else {
    const int rows_out = MODE == kDense ? M : ga.rows_total;
    float* out = SPLIT ? part + (size_t)sp * M * N : y;
    const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(out, (uint32_t)((size_t)rows_out * N * 4));
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = nw0 + nb * 16 + bcol;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + mb * 16 + rq + r;
          const uint32_t off = n < N ? ((uint32_t)m * N + n) * 4 : kOOB;
          float v = acc[mb][nb][r];
          if constexpr (ADD && !SPLIT)
            v += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(y_rsrc, off, 0, 0));
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), y_rsrc, off, 0,
                                                (MODE == kDense && !SPLIT) ? kYPolicy : 0);
        }
      }
    }
  }
}

// Launch the direct-to-LDS GEMM (fp16 X; Q4W with a power-of-two group >= 32, or T2W) for MB row blocks, in
// aq_gemm_x16.hip.
// Shapes it takes: K a multiple of 128 (whole super-steps) and a power-of-two group >= 32 (one scale per 32-k chunk).
inline bool x16_shape_ok(int K, int group) {
  return K > 0 && K % 128 == 0 && group >= 32 && (group & (group - 1)) == 0;
}
// nb = 4: 256-column tiles (four or eight waves of 64 columns); nb = 2 (dense only): 128-column tiles.
int launch_gemm_x16(const GemmArgs& ga, int fmt, int mb, int nb, bool add, bool split, int mode, int blocks,
                    hipStream_t s);

}  // namespace aq
