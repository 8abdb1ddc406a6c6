// Greedy-decode step end inside an output head's launch (the int4, Q6_K and ternary heads): every workgroup leaves
// its best argmax key (argmax_key, or kNonFiniteKey) in cand[block] and counts itself; the workgroup that arrives
// last (every other key is then stored) takes the largest key and writes *token (-1 for kNonFiniteKey), hist[*pos]
// (when 0 <= *pos < hist_cap) and *pos += advance, as the reference's host scan over the logits does
// (llama/llama.mojo:72-75, lfm2/kernels/lk.mojo:194-221, bonsai/bonsai_vk.c:506-515).
//
// The keys are stored and read with device-coherent (sc1) accesses and the counters are device-scope atomics, so no
// cache writeback or fence is needed: a key has reached device scope before its workgroup counts itself. The count
// is two-level, so that no counter takes more than a small share of the launch's atomics at once (1024 workgroups
// finishing together on one counter queue on its address): workgroup b counts on group b % 16's counter, the
// group's last member counts on the top counter and sets its group's back to zero, and the last on the top counter
// sets that one back to zero. Every counter is zero again when the launch ends.
#pragma once
#include "aq_common.h"

namespace aq {

struct StepEnd {
  uint64_t* cand;      // one key per workgroup (NULL: no step end)
  uint32_t* arrivals;  // AQ_HEAD_ARRIVAL_SLOTS 8-byte slots: the top counter in slot 0, group g's in slot g + 1
  int32_t* token;
  int32_t* pos;
  int32_t* hist;
  int hist_cap;
  int advance;
};

constexpr int kArrivalGroups = AQ_HEAD_ARRIVAL_SLOTS - 1;

// Called by all 64 lanes of wave 0 of every workgroup of the launch, with the workgroup's key in lane 0.
__device__ __forceinline__ void step_end(const StepEnd& e, uint64_t key) {
  const int lane = threadIdx.x & 63;
  const uint32_t nb = gridDim.x;
  const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(e.cand, nb * 8u);
  uint32_t last = 0;
  if (lane == 0) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, key), c_rsrc, blockIdx.x * 8u, 0, kSc1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the key has reached device scope
    const uint32_t ng = nb < (uint32_t)kArrivalGroups ? nb : (uint32_t)kArrivalGroups, g = blockIdx.x % ng;
    const uint32_t members = (nb - g + ng - 1) / ng;
    uint32_t* gc = e.arrivals + 2 * (g + 1);
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == members - 1) {
      __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // every member has counted
      last = __hip_atomic_fetch_add(e.arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1;
    }
  }
  if (!__builtin_amdgcn_readfirstlane(last)) return;
  // the last workgroup: every key, 16 a lane per pass, then the wave's maximum
  constexpr int kPer = 16;
  uint64_t m = 0;
  for (uint32_t b0 = 0; b0 < nb; b0 += kPer * kWave) {
    uint64_t kv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t b = b0 + lane + kWave * i;
      kv[i] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(c_rsrc, b < nb ? b * 8u : kOOB, 0, kSc1));
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) m = kv[i] > m ? kv[i] : m;
  }
  m = wave_max_u64(m);
  if (lane == 0) {
    const int idx = m == kNonFiniteKey ? -1 : m ? (int)~(uint32_t)m : 0;
    const int p = *e.pos;
    *e.token = idx;
    if (e.hist && p >= 0 && p < e.hist_cap) e.hist[p] = idx;
    *e.pos = p + e.advance;
    __hip_atomic_store(e.arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Called by every thread of a workgroup of WAVES waves, each wave's key in its lane 0: the workgroup's key is their
// maximum, and wave 0 ends the step with it. Contains a barrier.
template <int WAVES>
__device__ __forceinline__ void workgroup_step_end(const StepEnd& e, uint64_t key) {
  __shared__ uint64_t wkey[WAVES];
  if ((threadIdx.x & 63) == 0) wkey[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x < 64) {
    uint64_t m = wkey[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) m = wkey[w] > m ? wkey[w] : m;
    step_end(e, m);
  }
}

// The StepEnd of a head launch of `blocks` workgroups over cand [cand_cap] (8-byte aligned; its last
// AQ_HEAD_ARRIVAL_SLOTS slots hold the counters): AQ_OK, or the status that refuses the arguments.
inline int make_step_end(uint64_t* cand, int64_t cand_cap, int64_t blocks, int32_t* token, int32_t* pos,
                         int32_t* hist, int32_t hist_cap, int32_t advance, StepEnd& e) {
  if (!cand || !token || !pos) return AQ_ERR_NULL;
  if (hist_cap < 0) return AQ_ERR_SHAPE;
  if (cand_cap < blocks + AQ_HEAD_ARRIVAL_SLOTS) return AQ_ERR_CAPACITY;
  if (!aligned(cand, 8)) return AQ_ERR_ALIGN;
  e = StepEnd{cand, reinterpret_cast<uint32_t*>(cand + (cand_cap - AQ_HEAD_ARRIVAL_SLOTS)), token, pos, hist,
              hist_cap, advance};
  return AQ_OK;
}

}  // namespace aq
