// Streaming read, gfx950: the XOR of every 32-bit word of a buffer, each 16 bytes loaded once with the weights' nt
// (streaming) cache policy. It does no other work, so the time of a launch over the bytes of a weight matrix is the
// ceiling the matrix-vector kernels over that matrix are measured against (same bytes, same launch overhead, same
// memory latency, nothing to decode).
//
// The buffer is cut into pages of 256 * kReadUnroll 16-byte vectors; workgroup b reads pages b, b + blocks, ...,
// thread t the vectors t, t + 256, ... of a page, all kReadUnroll of them requested before any is used (a workgroup's
// loads of a page are one contiguous 8 KB). Wave w of workgroup b writes the XOR of its words to sink[4 b + w].
#include "aq_common.h"

namespace aq {

constexpr int kReadUnroll = 2;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_xor(uint32_t v) {
  return v ^ (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}

__global__ __launch_bounds__(256) void k_stream_read(const void* __restrict__ p, uint32_t n16,
                                                     uint32_t* __restrict__ sink) {
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(p, n16 * 16u);
  const uint32_t pages = (n16 + 256 * kReadUnroll - 1) / (256 * kReadUnroll);
  uint32_t acc = 0;
  for (uint32_t pg = blockIdx.x; pg < pages; pg += gridDim.x) {
    uint4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint32_t idx = pg * (256 * kReadUnroll) + (uint32_t)u * 256 + threadIdx.x;
      v[u] = buf_load16p<kWPolicy>(rsrc, idx < n16 ? idx * 16u : kOOB);
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= (v[u].x ^ v[u].y) ^ (v[u].z ^ v[u].w);
  }
  // XOR over the wave by DPP (as wave_sum does for sums): within rows of 16, then across rows into lane 63
  acc = dpp_xor<0xB1, 0xF>(acc);
  acc = dpp_xor<0x4E, 0xF>(acc);
  acc = dpp_xor<0x141, 0xF>(acc);
  acc = dpp_xor<0x140, 0xF>(acc);
  acc = dpp_xor<0x142, 0xA>(acc);
  acc = dpp_xor<0x143, 0xC>(acc);
  if ((threadIdx.x & 63) == 63) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

}  // namespace aq

extern "C" int aq_stream_read(const void* p, int64_t bytes, int32_t blocks, uint32_t* sink, void* stream) {
  if (!p || !sink) return AQ_ERR_NULL;
  if (bytes <= 0 || bytes % 16) return AQ_ERR_SHAPE;
  if (bytes >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;  // 32-bit buffer offsets
  if (blocks < 0 || blocks > AQ_STREAM_READ_MAX_BLOCKS) return AQ_ERR_ARG;
  if (!aq::aligned(p, 16)) return AQ_ERR_ALIGN;
  const uint32_t n16 = (uint32_t)(bytes / 16);
  if (blocks == 0) {  // one page a workgroup, at most AQ_STREAM_READ_MAX_BLOCKS
    const int64_t b = ((int64_t)n16 + 256 * aq::kReadUnroll - 1) / (256 * aq::kReadUnroll);
    blocks = (int32_t)(b < AQ_STREAM_READ_MAX_BLOCKS ? b : AQ_STREAM_READ_MAX_BLOCKS);
  }
  hipLaunchKernelGGL(aq::k_stream_read, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p,
                     n16, sink);
  return aq::launch_status();
}
