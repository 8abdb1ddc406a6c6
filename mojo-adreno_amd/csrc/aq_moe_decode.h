// The MoE decode down projection kernel (aq_moe_decode.hip), launched by aq_moe_down_q4 (aq_gemv.hip).
#pragma once
#include "aq_common.h"

namespace aq {

// Shapes the kernel takes: topk <= 8 slots, f % 32 == 0 and f <= 2048, a power-of-two group >= 32.
bool moe_down_dec_ok(int64_t f, int32_t group, int32_t topk);

// y[r] = (add ? y[r] : 0) + sum_{s < topk, in order} rw[s] * W[ids[s] * d + r] . act[s] for r < d. The caller has
// checked the pointers (wq and act 16-byte aligned), f % group == 0 and the stacked W below 2 GiB.
int launch_moe_down_dec(const uint32_t* wq, const uint16_t* ws, const int32_t* ids, const float* rw,
                        const float* act, float* y, int64_t d, int64_t f, int32_t group, int32_t experts,
                        int32_t topk, int32_t add, hipStream_t st);

}  // namespace aq
