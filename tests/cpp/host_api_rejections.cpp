// The C++ host API (include/candle_moe.hpp) rejects what the reference's
// Rust layer rejects, with its message text (/root/reference/src/lib.rs:47-94,
// 184-242), before any HIP call: every call here is invalid, so nothing is
// launched and no GPU is needed. Prints "ok" and exits 0 when every rejection
// carries the expected text.
#include <cstdio>
#include <initializer_list>
#include <string>

#include "candle_moe.hpp"

using candle_moe::Activation;
using candle_moe::FusedMoE;
using candle_moe::Status;
using candle_moe::Tensor;

static Tensor make(std::initializer_list<int64_t> shape, int32_t dtype, int32_t device = 0) {
    Tensor t{};
    t.data = nullptr;
    t.dtype = dtype;
    t.rank = (int32_t)shape.size();
    int i = 0;
    for (int64_t d : shape) t.dims[i++] = d;
    int64_t acc = 1;
    for (int j = t.rank - 1; j >= 0; --j) {
        t.strides[j] = acc;
        acc *= t.dims[j];
    }
    t.device = device;
    return t;
}

static int failures = 0;

static void expect(const Status& s, const char* want, const char* what) {
    if (s.ok() || s.message.find(want) == std::string::npos) {
        std::printf("FAIL %s: code %d, message \"%s\", expected \"%s\"\n", what, s.code, s.message.c_str(), want);
        ++failures;
    }
}

int main() {
    // apply_topk_softmax_inplace (lib.rs:47-94)
    const Tensor g = make({8, 4}, CM_DT_F32), w = make({8, 2}, CM_DT_F32);
    const Tensor i = make({8, 2}, CM_DT_U32), ei = make({8, 2}, CM_DT_U32);
    expect(candle_moe::apply_topk_softmax_inplace(make({8, 6}, CM_DT_F32), w, i, ei),
           "num_experts should be power of 2 and smaller than 256", "topk E=6");
    expect(candle_moe::apply_topk_softmax_inplace(make({8, 4, 1}, CM_DT_F32), w, i, ei),
           "expects input tensors of rank 2", "topk rank");
    expect(candle_moe::apply_topk_softmax_inplace(g, w, make({8, 3}, CM_DT_U32), ei), "shape mismatch topk_indices",
           "topk indices shape");
    expect(candle_moe::apply_topk_softmax_inplace(make({8, 4}, CM_DT_F32, -1), w, i, ei),
           "gating_output must be a cuda tensor", "topk host tensor");
    expect(candle_moe::apply_topk_softmax_inplace(g, make({8, 2}, CM_DT_I64), i, ei),
           "is only supported for f32, f16 and bf16", "topk weight dtype");

    // FusedMoE::forward (lib.rs:184-242)
    const FusedMoE moe(8, 2, Activation::Silu);
    const Tensor x = make({16, 64}, CM_DT_BF16), gate = make({8, 64, 256}, CM_DT_BF16);
    const Tensor up = make({8, 64, 256}, CM_DT_BF16), down = make({8, 256, 64}, CM_DT_BF16);
    const Tensor rw = make({16, 2}, CM_DT_F32), ri = make({16, 2}, CM_DT_U32), out = make({16, 64}, CM_DT_BF16);
    expect(FusedMoE(4, 2, Activation::Silu).forward(x, gate, up, &down, rw, ri, 0, out),
           "Number of experts mismatch", "moe experts");
    expect(moe.forward(x, make({8, 32, 256}, CM_DT_BF16), up, &down, rw, ri, 0, out),
           "Hidden dimension mismatch for gate/up weights", "moe hidden");
    expect(moe.forward(x, gate, make({8, 64, 128}, CM_DT_BF16), &down, rw, ri, 0, out),
           "Intermediate dimension mismatch (gate: 256, up: 128, down: 256)", "moe intermediate");
    expect(moe.forward(x, gate, up, &down, make({15, 2}, CM_DT_F32), ri, 0, out), "Number of tokens mismatch",
           "moe tokens");
    expect(moe.forward(x, gate, up, &down, rw, ri, 2, out), "moe_type must be one of 0 or 1", "moe type");
    expect(moe.forward(x, gate, up, &down, rw, make({16, 2}, CM_DT_I64), 0, out),
           "unexpected dtype for expert_indices, expected: U32", "moe index dtype");
    expect(moe.forward(make({16, 64}, CM_DT_BF16, -1), gate, up, &down, rw, ri, 0, out),
           "input must be a cuda tensor", "moe host tensor");

    std::printf(failures ? "FAILED %d\n" : "ok\n", failures);
    return failures ? 1 : 0;
}
