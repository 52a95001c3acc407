// The exact integer attention and its operand producers (attn.hip): argument block and launchers.
#pragma once
#include "vk_common.h"

namespace vk {

// k_fused_attention's operands (src/kernels.h:73-77): Q/K planes [G * Tqp|Tkp x 64] with per-row
// e and sums, transposed V planes [G * 64 x Tkp] with per-(g, d) e, the exp table, the output.
struct AttnArgs {
    const int8_t *qh, *ql;
    const int32_t* eq;
    const long long *qhs, *qls;
    const int8_t *kh, *kl;
    const int32_t* ek;
    const long long* ksum;
    const int8_t *vth, *vtl;
    const int32_t* ev;
    int heads, Tq, Tqp, Tk, Tkp, causal;
    const long long* Lexp;
    int C;
    int32_t* out;
    uint32_t* rowmax;
};

hipError_t launch_attention(hipStream_t st, const AttnArgs& a, int G);
hipError_t launch_quant_heads(hipStream_t st, const int32_t* X, int B, int T, int C, int heads, int Tp, int8_t* hi, int8_t* lo, int32_t* e, long long* hs,
                              long long* ls, long long* tsum);
hipError_t launch_quant_heads_pad(hipStream_t st, int G, int T, int Tp, int8_t* hi, int8_t* lo, int32_t* e, long long* hs, long long* ls, long long* tsum);
hipError_t launch_quant_v(hipStream_t st, const int32_t* X, int B, int Tk, int C, int heads, int Tkp, int8_t* vth, int8_t* vtl, int32_t* ev, long long* vsum);

}  // namespace vk
