// Streaming read, gfx950: the XOR of every 32-bit word of a buffer, each 16 bytes loaded once with the weights' nt
// (streaming) cache policy. It does no other work, so the time of a launch over the bytes of a weight matrix is the
// ceiling the matrix-vector kernels over that matrix are measured against (same bytes, same launch overhead, same
// memory latency, nothing to decode).
//
// Thread g of G = blocks * 256 reads the 16-byte vectors g, g + G, g + 2G, ... (every wave's loads are 1 KB
// contiguous), U of them requested before any is used; workgroup b writes the XOR of its share to sink[b].
#include "aq_common.h"

namespace aq {

constexpr int kReadUnroll = 4;

__global__ __launch_bounds__(256) void k_stream_read(const void* __restrict__ p, uint32_t n16,
                                                     uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[4];
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(p, n16 * 16u);
  const uint32_t G = gridDim.x * 256u;
  uint32_t acc = 0;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n16; i += kReadUnroll * G) {
    uint4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint32_t idx = i + (uint32_t)u * G;
      v[u] = buf_load16p<kWPolicy>(rsrc, idx < n16 ? idx * 16u : kOOB);
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= (v[u].x ^ v[u].y) ^ (v[u].z ^ v[u].w);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, s, kWave);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = (red[0] ^ red[1]) ^ (red[2] ^ red[3]);
}

}  // namespace aq

extern "C" int aq_stream_read(const void* p, int64_t bytes, int32_t blocks, uint32_t* sink, void* stream) {
  if (!p || !sink) return AQ_ERR_NULL;
  if (bytes <= 0 || bytes % 16) return AQ_ERR_SHAPE;
  if (bytes >= ((int64_t)1 << 31)) return AQ_ERR_CAPACITY;  // 32-bit buffer offsets
  if (blocks < 0 || blocks > AQ_STREAM_READ_MAX_BLOCKS) return AQ_ERR_ARG;
  if (!aq::aligned(p, 16)) return AQ_ERR_ALIGN;
  const uint32_t n16 = (uint32_t)(bytes / 16);
  if (blocks == 0) {  // one pass of kReadUnroll vectors a thread, at most 1024 workgroups
    const int64_t b = ((int64_t)n16 + 256 * aq::kReadUnroll - 1) / (256 * aq::kReadUnroll);
    blocks = (int32_t)(b < 1024 ? b : 1024);
  }
  hipLaunchKernelGGL(aq::k_stream_read, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p,
                     n16, sink);
  return aq::launch_status();
}
