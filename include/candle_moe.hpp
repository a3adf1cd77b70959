// C++ host API of candle-moe for MI355X: the reference's Rust surface
// (/root/reference/src/lib.rs) restated over tensor descriptors.
//
//   apply_topk_softmax_inplace(g, w, i, ei)            lib.rs:124-155
//   enum Activation { Silu, Gelu, Relu }               lib.rs:157-172
//   FusedMoE::new(num_experts, top_k, activation)      lib.rs:250-256
//   FusedMoE::forward(x, gate, up, down?, w, idx, moe_type, out)   lib.rs:273-335
//
// Errors come back as a Status carrying the reference's message text where
// the reference has one (candle::bail! sites in lib.rs); the C entry points
// behind it are declared in candle_moe.h.
#pragma once

#include <string>

#include "candle_moe.h"

namespace candle_moe {

using Tensor = cm_tensor_t;

struct Status {
    int code = CANDLE_MOE_OK;
    std::string message;
    bool ok() const { return code == CANDLE_MOE_OK; }
};

inline Status status_from(int code) {
    Status s;
    s.code = code;
    if (code != CANDLE_MOE_OK) s.message = candle_moe_last_error();
    return s;
}

enum class Activation : int { Silu = 0, Gelu = 1, Relu = 2 };

inline Status apply_topk_softmax_inplace(const Tensor& gating_output, const Tensor& topk_weight,
                                         const Tensor& topk_indices, const Tensor& token_expert_indices,
                                         void* stream = nullptr) {
    return status_from(candle_moe_apply_topk_softmax_inplace(&gating_output, &topk_weight, &topk_indices,
                                                             &token_expert_indices, stream));
}

class FusedMoE {
public:
    FusedMoE(size_t num_experts, size_t num_selected_experts, Activation activation)
        : num_experts(num_experts), num_selected_experts(num_selected_experts), activation(activation) {}

    // `output` is the zero-initialised [num_tokens, hidden_dim] result tensor
    // (forward zeroes it before accumulating, like Tensor::zeros in lib.rs:296).
    Status forward(const Tensor& input, const Tensor& gate_weights, const Tensor& up_weights,
                   const Tensor* down_weights, const Tensor& routing_weights, const Tensor& expert_indices,
                   uint32_t moe_type, const Tensor& output, void* stream = nullptr) const {
        cm_fused_moe_t self = {(int64_t)num_experts, (int64_t)num_selected_experts, (int32_t)activation};
        return status_from(candle_moe_fused_moe_forward(&self, &input, &gate_weights, &up_weights, down_weights,
                                                        &routing_weights, &expert_indices, moe_type, &output,
                                                        stream));
    }

    size_t num_experts;
    size_t num_selected_experts;
    Activation activation;
};

}  // namespace candle_moe
