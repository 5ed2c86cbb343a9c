// moe.cpp -- lh::moe_dispatch / lh::moe_combine (reference moe.cpp:102-140,
// 198-221) on the MI355X backend: host arrays are staged in device memory,
// the C ABI kernels run, and the results are copied back.
#include "kernels/moe.hpp"

#include "kernels/device.hpp"
#include "longhorn_hip.h"

namespace lh {

namespace {

using dev::Buffer;

size_t nonneg(int64_t v) { return v > 0 ? static_cast<size_t>(v) : 0; }

}  // namespace

void moe_dispatch(const float* hidden, const int32_t* expert_ids, int32_t* expert_offsets, int32_t* token_idx,
                  int32_t* slot_idx, float* expert_inputs, const MoEConfig& cfg) {
    const int T = cfg.n_tokens, H = cfg.hidden_dim, E = cfg.n_experts, K = cfg.top_k;
    const size_t S = nonneg(int64_t{T} * K);
    Buffer dh(nonneg(int64_t{T} * H) * sizeof(float)), dids(S * sizeof(int32_t));
    Buffer doff(nonneg(int64_t{E} + 1) * sizeof(int32_t)), dtok(S * sizeof(int32_t)), dslot(S * sizeof(int32_t));
    Buffer dpos(S * sizeof(int32_t)), dout(S * nonneg(H) * sizeof(float));
    dh.upload(hidden, dh.bytes());
    dids.upload(expert_ids, dids.bytes());
    dev::check(lhq_moe_dispatch_f32(dh.as<float>(), dids.as<int32_t>(), doff.as<int32_t>(), dtok.as<int32_t>(),
                                    dslot.as<int32_t>(), dpos.as<int32_t>(), dout.as<float>(), T, H, E, K,
                                    dev::stream()),
               "moe_dispatch");
    doff.download(expert_offsets, doff.bytes());
    dtok.download(token_idx, dtok.bytes());
    dslot.download(slot_idx, dslot.bytes());
    dout.download(expert_inputs, dout.bytes());
}

void moe_combine(const float* expert_outputs, const int32_t* /*expert_offsets*/, const int32_t* token_idx,
                 const int32_t* slot_idx, const float* gate_weights, float* output, const MoEConfig& cfg) {
    // the offsets are not needed: (token_idx, slot_idx) name every slot, as
    // in the reference (moe.cpp:198-221 ignores them too)
    const int T = cfg.n_tokens, H = cfg.hidden_dim, K = cfg.top_k;
    const size_t S = nonneg(int64_t{T} * K);
    Buffer dy(S * nonneg(H) * sizeof(float)), dtok(S * sizeof(int32_t)), dslot(S * sizeof(int32_t));
    Buffer dpos(S * sizeof(int32_t)), dg(S * sizeof(float)), dout(nonneg(int64_t{T} * H) * sizeof(float));
    dy.upload(expert_outputs, dy.bytes());
    dtok.upload(token_idx, dtok.bytes());
    dslot.upload(slot_idx, dslot.bytes());
    dg.upload(gate_weights, dg.bytes());
    dev::check(lhq_moe_slot_positions(dtok.as<int32_t>(), dslot.as<int32_t>(), dpos.as<int32_t>(), T, K,
                                      dev::stream()),
               "moe_combine (slot positions)");
    dev::check(lhq_moe_combine_f32(dy.as<float>(), dpos.as<int32_t>(), dg.as<float>(), dout.as<float>(), T, H, K,
                                   dev::stream()),
               "moe_combine");
    dout.download(output, dout.bytes());
}

}  // namespace lh
