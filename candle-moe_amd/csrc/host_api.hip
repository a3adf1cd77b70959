// Host API: the validation and dispatch of the reference's Rust layer
// (/root/reference/src/lib.rs) over cm_tensor_t descriptors. Error texts
// follow the reference's candle::bail! messages; checks the reference lacks
// (contiguity, top-k <= E, router rows, Qwen3 without down weights,
// /root/reference/src/lib.rs:59-68,393-446) are added with their own text.
#include <stdio.h>

#include <string>

#include "../../include/candle_moe.h"
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

static const char* dt_name(int dt) {
    switch (dt) {
        case CM_DT_F16: return "F16";
        case CM_DT_BF16: return "BF16";
        case CM_DT_F32: return "F32";
        case CM_DT_U32: return "U32";
        case CM_DT_I64: return "I64";
        case CM_DT_F64: return "F64";
        case CM_DT_U8: return "U8";
        default: return "Unknown";
    }
}

static std::string shape_str(const cm_tensor_t* t) {
    std::string s = "[";
    for (int i = 0; i < t->rank; ++i) {
        if (i) s += ", ";
        s += std::to_string((long long)t->dims[i]);
    }
    return s + "]";
}

static bool contiguous(const cm_tensor_t* t) {
    long long expect = 1;
    for (int i = t->rank - 1; i >= 0; --i) {
        if (t->dims[i] != 1 && t->strides[i] != expect) return false;
        expect *= t->dims[i];
    }
    return true;
}

static int need(const cm_tensor_t* t, const char* name) {
    if (!t) return set_error(CANDLE_MOE_ERR_INVALID, "%s is missing", name);
    if (t->rank < 0 || t->rank > CM_MAX_RANK) return set_error(CANDLE_MOE_ERR_INVALID, "%s has an invalid rank", name);
    return CANDLE_MOE_OK;
}

static int on_gpu(const cm_tensor_t* t, const char* name) {
    if (t->device < 0) return set_error(CANDLE_MOE_ERR_INVALID, "%s must be a cuda tensor", name);
    return CANDLE_MOE_OK;
}

static int is_dtype(const cm_tensor_t* t, int dt, const char* name) {
    if (t->dtype != dt)
        return set_error(CANDLE_MOE_ERR_INVALID, "unexpected dtype for %s, expected: %s, got: %s", name, dt_name(dt),
                         dt_name(t->dtype));
    return CANDLE_MOE_OK;
}

static int is_contig(const cm_tensor_t* t, const char* name) {
    if (!contiguous(t)) return set_error(CANDLE_MOE_ERR_INVALID, "%s must be contiguous (shape %s)", name, shape_str(t).c_str());
    return CANDLE_MOE_OK;
}

static int rank_is(const cm_tensor_t* t, int r, const char* name) {
    if (t->rank != r)
        return set_error(CANDLE_MOE_ERR_INVALID, "unexpected rank, expected: %d, got: %d (%s %s)", r, t->rank, name,
                         shape_str(t).c_str());
    return CANDLE_MOE_OK;
}

#define CM_TRY(x) do { const int rc_ = (x); if (rc_) return rc_; } while (0)

// /root/reference/src/lib.rs:10-155
static int validate_topk(const cm_tensor_t* g, const cm_tensor_t* w, const cm_tensor_t* i, const cm_tensor_t* ei) {
    clear_error();
    CM_TRY(need(g, "gating_output"));
    CM_TRY(need(w, "topk_weight"));
    CM_TRY(need(i, "topk_indices"));
    CM_TRY(need(ei, "token_expert_indices"));
    // dtype dispatch on topk_weight (lib.rs:130-153)
    if (w->dtype != CM_DT_F16 && w->dtype != CM_DT_BF16 && w->dtype != CM_DT_F32)
        return set_error(CANDLE_MOE_ERR_INVALID,
                         "apply_topk_softmax_inplace is only supported for f32, f16 and bf16 (%s)", dt_name(w->dtype));
    CM_TRY(on_gpu(g, "gating_output"));
    CM_TRY(on_gpu(w, "topk_weight"));
    CM_TRY(on_gpu(i, "topk_indices"));
    CM_TRY(on_gpu(ei, "token_expert_indices"));
    if (g->rank != 2 || w->rank != 2 || i->rank != 2 || ei->rank != 2)
        return set_error(CANDLE_MOE_ERR_INVALID,
                         "apply_topk_softmax_inplace expects input tensors of rank 2 (w: %s, i: %s, ei: %s, g: %s)",
                         shape_str(w).c_str(), shape_str(i).c_str(), shape_str(ei).c_str(), shape_str(g).c_str());
    // as_cuda_slice::<T>() with T from topk_weight, ::<u32>() for the indices (lib.rs:59-62)
    CM_TRY(is_dtype(g, w->dtype, "gating_output"));
    CM_TRY(is_dtype(i, CM_DT_U32, "topk_indices"));
    CM_TRY(is_dtype(ei, CM_DT_U32, "token_expert_indices"));
    const long long T = w->dims[0], k = w->dims[1], E = g->dims[1];
    const bool pow2 = E != 0 && (E & (E - 1)) == 0;
    if (!pow2 || E > 256)
        return set_error(CANDLE_MOE_ERR_INVALID,
                         "num_experts should be power of 2 and smaller than 256 (num_experts: %lld)", E);
    if (i->dims[0] != T || i->dims[1] != k)
        return set_error(CANDLE_MOE_ERR_INVALID, "shape mismatch topk_indices %s, expected (%lld, %lld)",
                         shape_str(i).c_str(), T, k);
    if (ei->dims[0] != T || ei->dims[1] != k)
        return set_error(CANDLE_MOE_ERR_INVALID, "shape mismatch token_expert_indices %s, expected (%lld, %lld)",
                         shape_str(ei).c_str(), T, k);
    if (g->dims[0] != T)
        return set_error(CANDLE_MOE_ERR_INVALID, "shape mismatch gating_output %s, expected (%lld, %lld)",
                         shape_str(g).c_str(), T, E);
    if (k < 1 || k > E)
        return set_error(CANDLE_MOE_ERR_INVALID, "top_k must be in [1, num_experts] (top_k: %lld, num_experts: %lld)",
                         k, E);
    if (T > 0x7fffffffLL) return set_error(CANDLE_MOE_ERR_INVALID, "num_tokens exceeds 2^31-1");
    CM_TRY(is_contig(g, "gating_output"));
    CM_TRY(is_contig(w, "topk_weight"));
    CM_TRY(is_contig(i, "topk_indices"));
    CM_TRY(is_contig(ei, "token_expert_indices"));
    return CANDLE_MOE_OK;
}

// /root/reference/src/lib.rs:184-242 plus the dtype / device checks of cuda_fwd (lib.rs:338-446)
static int validate_moe(const cm_fused_moe_t* m, const cm_tensor_t* x, const cm_tensor_t* gate, const cm_tensor_t* up,
                        const cm_tensor_t* down, const cm_tensor_t* rw, const cm_tensor_t* idx, uint32_t moe_type,
                        const cm_tensor_t* out) {
    clear_error();
    if (!m) return set_error(CANDLE_MOE_ERR_INVALID, "FusedMoE is missing");
    CM_TRY(need(x, "input"));
    CM_TRY(need(gate, "gate_weights"));
    CM_TRY(need(up, "up_weights"));
    if (down) CM_TRY(need(down, "down_weights"));
    CM_TRY(need(rw, "routing_weights"));
    CM_TRY(need(idx, "expert_indices"));
    CM_TRY(rank_is(x, 2, "input"));
    CM_TRY(rank_is(gate, 3, "gate_weights"));
    CM_TRY(rank_is(up, 3, "up_weights"));
    if (down) CM_TRY(rank_is(down, 3, "down_weights"));
    CM_TRY(rank_is(rw, 2, "routing_weights"));
    CM_TRY(rank_is(idx, 2, "expert_indices"));
    const long long T = x->dims[0], H = x->dims[1];
    const long long ne_g = gate->dims[0], hd_g = gate->dims[1], id_g = gate->dims[2];
    const long long ne_u = up->dims[0], hd_u = up->dims[1], id_u = up->dims[2];
    long long ne_d = m->num_experts, id_d = id_u, hd_d = hd_u;
    if (down) { ne_d = down->dims[0]; id_d = down->dims[1]; hd_d = down->dims[2]; }
    const long long nt = rw->dims[0], nse = rw->dims[1], nt2 = idx->dims[0], nse2 = idx->dims[1];
    if (ne_g != m->num_experts || ne_u != m->num_experts || ne_d != m->num_experts)
        return set_error(CANDLE_MOE_ERR_INVALID, "Number of experts mismatch");
    if (hd_g != H || hd_u != H) return set_error(CANDLE_MOE_ERR_INVALID, "Hidden dimension mismatch for gate/up weights");
    if (hd_d != H)
        return set_error(CANDLE_MOE_ERR_INVALID, "Hidden dimension mismatch for down weights (expected %lld, got %lld)",
                         H, hd_d);
    if (id_g != id_u || id_u != id_d)
        return set_error(CANDLE_MOE_ERR_INVALID, "Intermediate dimension mismatch (gate: %lld, up: %lld, down: %lld)",
                         id_g, id_u, id_d);
    if (nt != T || nt2 != T) return set_error(CANDLE_MOE_ERR_INVALID, "Number of tokens mismatch");
    if (nse != m->num_selected_experts || nse2 != m->num_selected_experts)
        return set_error(CANDLE_MOE_ERR_INVALID, "Number of selected experts mismatch");
    if (moe_type > 1) return set_error(CANDLE_MOE_ERR_INVALID, "moe_type must be one of 0 or 1");
    if (x->dtype != CM_DT_F16 && x->dtype != CM_DT_BF16 && x->dtype != CM_DT_F32)
        return set_error(CANDLE_MOE_ERR_INVALID, "FusedMoE is only supported for f16, bf16 and f32 (%s)", dt_name(x->dtype));
    if (moe_type == 0 && !down)
        return set_error(CANDLE_MOE_ERR_INVALID, "down_weights is required for moe_type 0 (Qwen3)");
    if (m->activation < 0 || m->activation > 2)
        return set_error(CANDLE_MOE_ERR_INVALID, "activation must be Silu, Gelu or Relu (got %d)", m->activation);
    CM_TRY(on_gpu(x, "input"));
    CM_TRY(on_gpu(gate, "gate_weights"));
    CM_TRY(on_gpu(up, "up_weights"));
    if (down) CM_TRY(on_gpu(down, "down_weights"));
    CM_TRY(on_gpu(rw, "routing_weights"));
    CM_TRY(on_gpu(idx, "expert_indices"));
    CM_TRY(is_dtype(gate, x->dtype, "gate_weights"));
    CM_TRY(is_dtype(up, x->dtype, "up_weights"));
    if (down) CM_TRY(is_dtype(down, x->dtype, "down_weights"));
    CM_TRY(is_dtype(rw, CM_DT_F32, "routing_weights"));
    CM_TRY(is_dtype(idx, CM_DT_U32, "expert_indices"));
    CM_TRY(is_contig(x, "input"));
    CM_TRY(is_contig(gate, "gate_weights"));
    CM_TRY(is_contig(up, "up_weights"));
    if (down) CM_TRY(is_contig(down, "down_weights"));
    CM_TRY(is_contig(rw, "routing_weights"));
    CM_TRY(is_contig(idx, "expert_indices"));
    if (out) {
        CM_TRY(need(out, "output"));
        CM_TRY(on_gpu(out, "output"));
        CM_TRY(rank_is(out, 2, "output"));
        CM_TRY(is_dtype(out, x->dtype, "output"));
        if (out->dims[0] != T || out->dims[1] != H)
            return set_error(CANDLE_MOE_ERR_INVALID, "shape mismatch output %s, expected (%lld, %lld)",
                             shape_str(out).c_str(), T, H);
        CM_TRY(is_contig(out, "output"));
    }
    if (T > 0x7fffffffLL || H > 0x7fffffffLL || id_g > 0x7fffffffLL || m->num_experts > 0x7fffffffLL ||
        m->num_selected_experts > 0x7fffffffLL)
        return set_error(CANDLE_MOE_ERR_INVALID, "dimension exceeds the C ABI's int range");
    return CANDLE_MOE_OK;
}

}  // namespace cm

extern "C" {

int candle_moe_validate_topk_softmax(const cm_tensor_t* g, const cm_tensor_t* w, const cm_tensor_t* i,
                                     const cm_tensor_t* ei) {
    return cm::validate_topk(g, w, i, ei);
}

int candle_moe_apply_topk_softmax_inplace(const cm_tensor_t* g, const cm_tensor_t* w, const cm_tensor_t* i,
                                          const cm_tensor_t* ei, void* stream) {
    const int rc = cm::validate_topk(g, w, i, ei);
    if (rc) return rc;
    return cm::topk_softmax_impl(g->data, g->dtype, w->data, w->dtype, i->data, ei->data, (int)g->dims[1],
                                 (int)w->dims[0], (int)w->dims[1], stream);
}

int candle_moe_validate_fused_moe(const cm_fused_moe_t* m, const cm_tensor_t* x, const cm_tensor_t* gate,
                                  const cm_tensor_t* up, const cm_tensor_t* down, const cm_tensor_t* rw,
                                  const cm_tensor_t* idx, uint32_t moe_type, const cm_tensor_t* out) {
    if (!out) return cm::set_error(CANDLE_MOE_ERR_INVALID, "output is missing");
    return cm::validate_moe(m, x, gate, up, down, rw, idx, moe_type, out);
}

int candle_moe_fused_moe_forward(const cm_fused_moe_t* m, const cm_tensor_t* x, const cm_tensor_t* gate,
                                 const cm_tensor_t* up, const cm_tensor_t* down, const cm_tensor_t* rw,
                                 const cm_tensor_t* idx, uint32_t moe_type, const cm_tensor_t* out, void* stream) {
    if (!out) return cm::set_error(CANDLE_MOE_ERR_INVALID, "output is missing");
    int rc = cm::validate_moe(m, x, gate, up, down, rw, idx, moe_type, out);
    if (rc) return rc;
    // The reference zeroes a fresh output and accumulates into it
    // (lib.rs:296); here the last kernel writes every element of out instead
    // (overwrite), which gives the same tensor without the clear.
    return cm::fused_moe_impl(x->data, gate->data, up->data, down ? down->data : nullptr, rw->data, idx->data,
                              out->data, (int)x->dims[0], (int)x->dims[1], (int)gate->dims[2], (int)m->num_experts,
                              (int)m->num_selected_experts, m->activation, moe_type, (uint32_t)x->dtype, nullptr, 0,
                              true, true, stream);
}

}  // extern "C"
