// kernels/moe.hpp -- MoE routing (dispatch and combine) on the MI355X backend.
//
// Drop-in for two functions of the reference header src/kernels/moe.hpp,
// with its MoEConfig (moe.hpp:39-49):
//   moe_dispatch (moe.hpp:63-78)  counting sort of the (token, slot) pairs by
//                                 expert, stable in slot order, and the row
//                                 copy into expert-major order;
//   moe_combine  (moe.hpp:96-102) the gate-weighted sum of the expert outputs
//                                 back per token, in the reference's
//                                 summation order (bit-exact).
// The reference's router, fp32 expert MLP and moe_forward are not provided:
// on this backend the expert MLP runs on W4A16 experts through the C ABI
// (lhq_moe_expert_mlp_w4a16_bf16, include/longhorn_hip.h).
// Synchronous on host memory; a HIP failure aborts with the library's message.
#ifndef LONGHORN_MI355X_KERNELS_MOE_HPP
#define LONGHORN_MI355X_KERNELS_MOE_HPP

#include <cstdint>

namespace lh {

struct MoEConfig {
    int n_tokens = 0;
    int hidden_dim = 0;
    int intermediate_dim = 0;
    int n_experts = 0;
    int top_k = 1;
    // renormalise the chosen top-k gates to sum to 1 (used by the router,
    // which this backend does not provide)
    bool renorm_gates = true;
};

void moe_dispatch(const float* hidden, const int32_t* expert_ids,
                  int32_t* expert_offsets, int32_t* token_idx,
                  int32_t* slot_idx, float* expert_inputs,
                  const MoEConfig& cfg);

void moe_combine(const float* expert_outputs, const int32_t* expert_offsets,
                 const int32_t* token_idx, const int32_t* slot_idx,
                 const float* gate_weights, float* output,
                 const MoEConfig& cfg);

}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_MOE_HPP
