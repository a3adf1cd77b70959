/*
 * candle-moe for MI355X (gfx950): C ABI of libcandle_moe_hip.so.
 *
 * The first two symbols are the drop-in boundary: the same names, argument
 * order, meaning and codes as the reference's FFI, so a Rust (or any C)
 * caller that binds them needs no change other than linking this library.
 * Everything is stream-ordered and asynchronous on `stream` (NULL = the
 * default stream); all tensors are caller-owned, row-major, contiguous
 * device memory.
 *
 * Codes:  activation 0 = SiLU, 1 = GELU (tanh approximation), 2 = ReLU
 *         moe_type   0 = Qwen3 (gate, up -> down), 1 = Nomic (fc1 -> fc2)
 *         dtype      0 = f16, 1 = bf16, 2 = f32
 * Routing weights are always f32, expert indices always u32.
 */
#ifndef CANDLE_MOE_H
#define CANDLE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the *_status / host-API entry points. */
enum {
    CANDLE_MOE_OK = 0,
    CANDLE_MOE_ERR_INVALID = 1,     /* argument / shape / dtype rejected before any launch */
    CANDLE_MOE_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
    CANDLE_MOE_ERR_HIP = 3,         /* a HIP runtime call or launch failed */
    CANDLE_MOE_ERR_WORKSPACE = 4    /* caller workspace too small / allocation failed */
};

/* ---------------------------------------------------------------------
 * Drop-in symbols
 * ------------------------------------------------------------------- */

/*
 * Router: softmax over num_experts logits per token, then the top-k.
 * Replaces the reference symbol declared at /root/reference/src/ffi.rs:15-24
 * (defined at /root/reference/kernels/topk_softmax.cu:331-353).
 *   gating_output        [num_tokens, num_experts] f32
 *   topk_weight          [num_tokens, topk] f32   (descending probability)
 *   topk_indices         [num_tokens, topk] u32   (ties -> lower expert index)
 *   token_expert_indices [num_tokens, topk] u32   (= j * num_tokens + t)
 * Indices are those of the exact softmax (f64 exponential rounded to f32,
 * f64 row sum, correctly rounded quotient), ties included. So are the
 * weights, except for f32 weights with num_experts 64, 128 or 256 and
 * topk < num_experts / 8: there they come from an f32 softmax within 6e-7
 * relative of the exact one.
 * num_tokens is a C int, as the reference caller passes it (the reference
 * definition's int64_t parameter did not match its caller). On invalid
 * sizes nothing is launched and candle_moe_last_error() says why.
 */
void topk_softmax(const void* gating_output, void* topk_weight, void* topk_indices,
                  void* token_expert_indices, int num_experts, int num_tokens, int topk,
                  void* stream);

/*
 * Fused MoE forward: output[t] += sum_j w[t,j] * expert_{idx[t,j]}(input[t]).
 * Replaces the reference symbol declared at /root/reference/src/ffi.rs:45-62
 * (defined at /root/reference/kernels/moe.cu:453-771).
 *   input          [num_tokens, hidden_dim]                       dtype
 *   gate_weights   [num_experts, hidden_dim, intermediate_dim]    dtype
 *   up_weights     [num_experts, hidden_dim, intermediate_dim]    dtype
 *   down_weights   [num_experts, intermediate_dim, hidden_dim]    dtype (Qwen3; NULL for Nomic)
 *   routing_weights[num_tokens, num_selected_experts]             f32
 *   expert_indices [num_tokens, num_selected_experts]             u32
 *   output         [num_tokens, hidden_dim]                       dtype, zero-initialised by
 *                                                                 the caller (results are added)
 * Qwen3: y = (act(x G) * (x U)) D.   Nomic: y = act(x G) U^T.
 * The workspace is library-owned: one buffer per (device, stream), allocated
 * stream-ordered (hipMallocAsync on `stream`) on first use, grown when a call
 * needs more and kept for the next call on that stream;
 * candle_moe_trim_workspaces releases them. No host synchronisation. A stream
 * being captured into a graph gets no new or larger workspace (the graph
 * would own that memory): such a call fails with CANDLE_MOE_ERR_WORKSPACE
 * before enqueuing anything, so make one call of the largest size on the
 * stream before capturing it.
 */
void fused_moe(const void* input, const void* gate_weights, const void* up_weights,
               const void* down_weights, const void* routing_weights, const void* expert_indices,
               void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
               int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
               void* stream);

/* ---------------------------------------------------------------------
 * Status-returning variants of the two symbols (the reference returns
 * nothing and checks nothing). Same arguments; return a CANDLE_MOE_* code.
 * ------------------------------------------------------------------- */
int candle_moe_topk_softmax_status(const void* gating_output, void* topk_weight, void* topk_indices,
                                   void* token_expert_indices, int num_experts, int num_tokens,
                                   int topk, void* stream);

/* Router with 16-bit logits / weights (dtype codes above for each tensor).
 * The reference accepts f16/bf16 topk_weight at /root/reference/src/lib.rs:130-148
 * but its kernel reads them as f32; this entry point implements them. */
int candle_moe_topk_softmax_ex(const void* gating_output, int gating_dtype, void* topk_weight,
                               int weight_dtype, void* topk_indices, void* token_expert_indices,
                               int num_experts, int num_tokens, int topk, void* stream);

int candle_moe_fused_moe_status(const void* input, const void* gate_weights, const void* up_weights,
                                const void* down_weights, const void* routing_weights,
                                const void* expert_indices, void* output, int num_tokens,
                                int hidden_dim, int intermediate_dim, int num_experts,
                                int num_selected_experts, int activation_type, uint32_t moe_type,
                                uint32_t dtype, void* stream);

/* Caller-provided workspace: bytes needed by candle_moe_fused_moe_ws for
 * these sizes, for either moe_type and any operand alignment (0 when the
 * arguments are invalid). */
size_t candle_moe_fused_moe_workspace_size(int num_tokens, int hidden_dim, int intermediate_dim,
                                           int num_experts, int num_selected_experts,
                                           uint32_t dtype);

/* fused_moe with a caller-owned device workspace of >= workspace_size bytes
 * (256-byte aligned); allocates nothing. */
int candle_moe_fused_moe_ws(const void* input, const void* gate_weights, const void* up_weights,
                            const void* down_weights, const void* routing_weights,
                            const void* expert_indices, void* output, int num_tokens,
                            int hidden_dim, int intermediate_dim, int num_experts,
                            int num_selected_experts, int activation_type, uint32_t moe_type,
                            uint32_t dtype, void* workspace, size_t workspace_bytes, void* stream);

/* fused_moe that allocates nothing, for callers that cannot allocate (code
 * under HIP graph capture, serving loops that must not call hipMalloc,
 * harnesses that forbid it). It has no counterpart in the reference.
 * Same arguments and result as candle_moe_fused_moe_status (output is added
 * into); the workspace is a fixed device array inside the library, one per
 * GPU, of candle_moe_fused_moe_noalloc_scratch_bytes() bytes (32 MiB: decode
 * and small prefill batches, e.g. Qwen3 H4096 I1536 E8 k2 up to ~1400 tokens),
 * held until the process ends. A call that needs more is rejected with
 * CANDLE_MOE_ERR_WORKSPACE before anything is launched. All calls on one GPU
 * share that array: calls that may overlap on one GPU (other streams, other
 * host threads without ordering) race and must be serialised by the caller.
 * Each call clears, with its own kernels, every piece of the array that must
 * start at zero (split-K arrival counters, accumulators); no call depends on
 * what an earlier call left in the array, so a race between overlapping calls
 * corrupts only their own outputs. */
int candle_moe_fused_moe_noalloc(const void* input, const void* gate_weights, const void* up_weights,
                                 const void* down_weights, const void* routing_weights,
                                 const void* expert_indices, void* output, int num_tokens,
                                 int hidden_dim, int intermediate_dim, int num_experts,
                                 int num_selected_experts, int activation_type, uint32_t moe_type,
                                 uint32_t dtype, void* stream);
size_t candle_moe_fused_moe_noalloc_scratch_bytes(void);

/* Per-kernel timing for benchmarks: between begin and end, every internal
 * launch is bracketed by HIP events on the caller's stream. end() waits for
 * those events and returns, per slot, the summed milliseconds and the number
 * of launches; begin() returns the number of slots. */
int candle_moe_profile_begin(void);
/* As profile_begin, bracketing only the slots whose bit is set in slot_mask
 * (fewer event records in a timed region). */
int candle_moe_profile_begin_slots(uint32_t slot_mask);
int candle_moe_profile_end(double* total_ms, int* counts, int nslots);
const char* candle_moe_profile_slot_name(int slot);

/* Combine strategy of fused_moe (process-wide): 0 = choose per call (default),
 * 1 = always the pair path (the down GEMM over expert-sorted pairs; each
 *     pair's weighted row stored and a token's k rows summed, or, on the
 *     32-row decode and f32 kernels, f32 atomics into an accumulator),
 * 2 = the expert-set path whenever the shape allows it (MFMA dtypes,
 *     intermediate_dim % 64 == 0, (E+1)^k <= 1024, k <= 8). */
int candle_moe_set_combine_policy(int policy);
/* GEMM kernel of fused_moe (process-wide): 0 = choose per call (default);
 * 1 = register-staged MFMA kernel, 128x128 block tile (taken by default only
 *     when an operand exceeds the 2 GiB range of the LDS-DMA kernels);
 * LDS-DMA MFMA kernels: 5 = 128x128, 7 = 256x256 (8 waves),
 * 12 = 32x256 with K splits (for <= 32 rows per expert on average where 18
 *     does not apply, and for <= 128 where intermediate_dim >= 1024 and the
 *     128x128 tile would give the down GEMM fewer tiles than CUs, as with
 *     Nomic's hidden_dim 768),
 * 14 = 128x256 (BK 32, two workgroups per CU);
 * 18 = the decode kernels (f16 / bf16 / fp8, at most 1024 pairs and 4096
 *     experts): no grouping launch (each workgroup groups the pairs in LDS),
 *     weights loaded straight into registers (transposed there for the API
 *     layout), K split across the waves of a workgroup and, for large
 *     gate/up streams, across workgroups; default for <= 32 rows per expert
 *     on average and at most 256 pairs (fp8: 128). By default 5 is taken for
 * <= 128 rows per expert where the 256x256 tile would give few workgroups,
 * 14 for < 1024 rows per expert with hidden_dim <= 2048 when the down GEMM
 * has at least two 128x256 tiles per CU, else 7.
 * f32 (vector FMA): 15 = 32x128 tile, 16 = 128x128 tile, both with K splits
 * when the tiles are few; by default 15 for <= 32 rows per expert, else 16
 * (the scalar 64x64 kernel 0 when hidden_dim or intermediate_dim is not a
 * multiple of 4 or an operand is not 16-byte aligned).
 * 17 concerns fp8 weights only (candle_moe_fused_moe_fp8; fused_moe
 * treats it as 0): the register-operand decode kernel, the default for at
 * most 16 pairs only where 18 does not apply (more than 4096 experts, or
 * operands beyond its 32-bit offsets); for fp8 weights 18, 12 and 7 force the decode
 * kernels, the 32-row and the 256x256 kernel, other codes leave the fp8
 * choice automatic.
 * Other codes are rejected with CANDLE_MOE_ERR_INVALID. */
int candle_moe_set_tile_policy(int policy);

/* Grouping of fused_moe above 2048 items (process-wide; no counterpart in the
 * reference, whose preprocessing is /root/reference/kernels/preprocessing.cuh:5-313):
 * 0 = one launch (per-block histograms, a bounded wait for every block's
 *     counts, stable scatter) on library-owned workspaces up to 32 blocks of
 *     1024 pairs; two launches beyond, on caller workspaces and on the
 *     no-allocation scratch (default),
 * 1 = always two launches (histogram; scan + scatter),
 * 2 = one launch in which every workgroup recounts all items itself instead
 *     of waiting (the fallback of a wait that runs out; for tests).
 * Other codes are rejected with CANDLE_MOE_ERR_INVALID. */
int candle_moe_set_grouping_mode(int mode);
/* Which path fused_moe takes for these sizes under the current policies:
 * bits 0-1: 2 = expert-set MFMA path, 1 = pair MFMA path, 0 = SIMT path;
 * bits 2 and up: the GEMM kernel (policy code above); -1 = invalid sizes. */
int candle_moe_fused_moe_path(int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                              int num_selected_experts, uint32_t dtype);
/* The same for a given moe_type (candle_moe_fused_moe_path answers for
 * moe_type 0, Qwen3; the Nomic fc1 tile can differ), with bit 8 set when the
 * pair path stores pair rows and sums them per token (clear: f32 atomics
 * into an accumulator and a finalize pass). */
int candle_moe_fused_moe_path_ex(int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                 int num_selected_experts, uint32_t dtype, uint32_t moe_type);

/* Router GEMM fused with topk-softmax (no counterpart symbol in the
 * reference; its callers compute the logits with a separate candle matmul,
 * /root/reference/README.md:61-71, then call topk_softmax on them):
 *   logits[t,e] = dtype(sum_h hidden[t,h] * router_weight[e,h])   (f32 accumulation,
 *                 one rounding to dtype, as candle's Linear in that dtype stores them)
 *   then topk_softmax of f32(logits): topk_weight f32 [T,k], topk_indices u32 [T,k],
 *   token_expert_indices u32 [T,k] = j*T + t.
 *   hidden [T,H], router_weight [E,H] (candle Linear layout), both `dtype`,
 *   16-byte aligned; H a multiple of 8 (4 for f32), at most 2^22; 1 <= E <= 128.
 * Reads hidden once (HBM-bound); the logits never reach memory. Small 16-bit
 * batches over more than 32 experts (at most 8 tiles of 32 tokens) split the
 * weight stream over workgroups, with f32 partial logits in the library's
 * per-stream workspace (the one fused_moe keeps; allocated on first use,
 * never while the stream is being captured: see fused_moe). */
int candle_moe_router_topk(const void* hidden, const void* router_weight, void* topk_weight,
                           void* topk_indices, void* token_expert_indices, int num_tokens,
                           int hidden_dim, int num_experts, int topk, uint32_t dtype, void* stream);

/* Pre-packed 16-bit expert weights (opt-in; no counterpart in the reference,
 * whose weights are used in the API layout only, src/lib.rs:273-335): every
 * weight matrix stored K-contiguous, [E][N][K], so that the GEMMs read it
 * without transposing (ds_read_b128 fragments instead of transposed LDS
 * reads; whole MFMA operands straight from memory at decode sizes).
 *   pack_weights: weights [num_experts][k_dim][n_dim] (f16 / bf16, dtype 0 /
 *     1) -> packed [num_experts][n_dim][k_dim], out of place, on the stream.
 *   fused_moe_packed: fused_moe over packed weights, same arguments, result
 *     and accumulate-into-output contract:
 *     Qwen3 (moe_type 0): gate_packed / up_packed [E][I][H] (pack of the API's
 *       [E][H][I]), down_packed [E][H][I] (pack of [E][I][H]);
 *     Nomic (moe_type 1): gate_packed = fc1 [E][I][H] (pack of [E][H][I]),
 *       up_packed = fc2 [E][H][I] exactly as fused_moe takes it (already
 *       K-contiguous), down_packed NULL.
 *   f16 / bf16 only, hidden_dim and intermediate_dim multiples of 8, 16-byte
 *   aligned tensors; otherwise CANDLE_MOE_ERR_UNSUPPORTED. */
int candle_moe_pack_weights(const void* weights, uint32_t dtype, int num_experts, int k_dim, int n_dim,
                            void* packed, void* stream);
int candle_moe_fused_moe_packed(const void* input, const void* gate_packed, const void* up_packed,
                                const void* down_packed, const void* routing_weights, const void* expert_indices,
                                void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
                                void* stream);

/* Test support, no counterpart in the reference: evaluates the router's f32
 * exponential (the f32 softmax used for f32 weights over 64-256 experts) and
 * its f64 one on the count f32 values whose bit patterns are first_bits,
 * first_bits + 1, ..., and folds into stats (2 device u32, zeroed by the
 * caller): stats[0] = max(stats[0], largest distance in ulp), stats[1] +=
 * number of inputs where the two differ. */
int candle_moe_test_router_exp(uint32_t first_bits, uint32_t count, uint32_t* stats, void* stream);

/* Token->expert grouping as fused_moe runs it internally (the reference's
 * launch_preprocessing, /root/reference/kernels/preprocessing.cuh:5-313, which
 * has no exported symbol; exposed for callers that route themselves and for
 * tests). Pairs p of expert_indices [num_pairs] u32 (p = t*k + j) are grouped
 * by expert, stable (ascending p inside an expert); ids >= num_experts are
 * dropped.
 *   offsets [num_experts + 2] i32: exclusive scan of the per-expert counts,
 *     offsets[E] = valid pairs, offsets[E+1] = largest count;
 *   sorted_pairs [num_pairs] i32: the first offsets[E] entries are the valid
 *     pair ids in that order (the reference stores the token ids p / k and the
 *     weights w[p] instead; both follow from the pair id).
 * workspace: candle_moe_grouping_workspace_size(num_pairs, num_experts) bytes,
 * 256-byte aligned; nothing is allocated. Asynchronous on `stream`. */
size_t candle_moe_grouping_workspace_size(int num_pairs, int num_experts);
int candle_moe_group_pairs(const void* expert_indices, int num_pairs, int num_experts, void* offsets,
                           void* sorted_pairs, void* workspace, size_t workspace_bytes, void* stream);

/* Opt-in FP8 expert weights (no counterpart in the reference, whose fused_moe
 * takes the weights in the activation dtype, /root/reference/src/lib.rs:273-335;
 * for decode, where the weight stream is the whole cost). Format: OCP FP8
 * e4m3 (E4M3FN: bias 7, largest finite 448, no infinities, 0x7F/0xFF NaN),
 * one f32 scale per output channel, codes K-contiguous:
 *   codes [E][N][K] u8, scales [E][N] f32, w[e][k][n] ~ decode(codes[e][n][k]) * scales[e][n]
 *   scale = max_k |w[e][k][n]| / 448 (1 for an all-zero channel),
 *   code = e4m3(w / scale), round to nearest even, |x| >= 448 -> +-448.
 * quantize_fp8: weights [E][K][N] (input_kn = 1: gate/up [E][H][I] and
 * down [E][I][H] of Qwen3, fc1 [E][H][I] of Nomic, the reference's layouts)
 * or [E][N][K] (input_kn = 0: fc2 of Nomic, [E][H][I]) in dtype 0/1/2. */
int candle_moe_quantize_fp8(const void* weights, uint32_t dtype, int num_experts, int k_dim, int n_dim,
                            int input_kn, void* codes, float* scales, void* stream);
/* out [E][N][K] of dtype = dtype(decode(codes) * scales): the weights the fp8
 * MoE multiplies by. */
int candle_moe_dequantize_fp8(const void* codes, const float* scales, int num_experts, int n_dim, int k_dim,
                              void* out, uint32_t dtype, void* stream);
/* fused_moe with fp8 expert weights: output += the MoE of input over the
 * dequantized weights, f32 accumulation (as candle_moe_fused_moe_status,
 * accumulating). Qwen3 (moe_type 0): gate_q/up_q codes [E][I][H] with scales
 * [E][I] (quantize_fp8 of gate/up [E][H][I]), down_q [E][H][I] with scales
 * [E][H] (of down [E][I][H]). Nomic (moe_type 1), as fused_moe takes fc1 /
 * fc2 in gate / up: gate_q = fc1 codes [E][I][H] with gate_scale [E][I],
 * up_q = fc2 codes [E][H][I] with up_scale [E][H]; down_q and down_scale
 * unused. Activations f16 or bf16;
 * hidden_dim and intermediate_dim multiples of 16; every tensor 16-byte
 * aligned. Runs the decode kernels up to 128 pairs (at most 1024 pairs and
 * 4096 experts), the 32-row GEMM kernel beyond that up to 32 pairs per
 * touched expert, or up to 256 while it streams at most 384 MiB of weights
 * (the touched experts' codes once per 32 rows), and the 8-wave 256x256
 * kernel past it, with the combine path chosen as for fused_moe (expert
 * sets, on the 256x256 kernel only, or pairs). */
int candle_moe_fused_moe_fp8(const void* input, const void* gate_q, const void* up_q, const void* down_q,
                             const float* gate_scale, const float* up_scale, const float* down_scale,
                             const void* routing_weights, const void* expert_indices, void* output, int num_tokens,
                             int hidden_dim, int intermediate_dim, int num_experts, int num_selected_experts,
                             int activation_type, uint32_t moe_type, uint32_t dtype, void* stream);

/* Releases the library-owned workspaces of fused_moe / candle_moe_fused_moe_status,
 * the FusedMoE forward and candle_moe_router_topk (hipFree: waits for the
 * device, so the streams they were used on may already be destroyed; not
 * while a stream is being captured); the next call allocates again. No counterpart in the reference, whose fused_moe
 * allocates and frees per call (/root/reference/kernels/moe.cu:570,770). */
int candle_moe_trim_workspaces(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* candle_moe_last_error(void);
const char* candle_moe_version(void);

/* ---------------------------------------------------------------------
 * Host API: the reference's Rust surface (/root/reference/src/lib.rs) over
 * tensor descriptors, with the same validation and error text.
 * ------------------------------------------------------------------- */
enum {
    CM_DT_F16 = 0,
    CM_DT_BF16 = 1,
    CM_DT_F32 = 2,
    CM_DT_U32 = 3,
    CM_DT_I64 = 4,
    CM_DT_F64 = 5,
    CM_DT_U8 = 6
};

#define CM_MAX_RANK 4
typedef struct {
    void* data;                 /* address of element 0 (start offset applied) */
    int32_t dtype;              /* CM_DT_* */
    int32_t rank;
    int64_t dims[CM_MAX_RANK];
    int64_t strides[CM_MAX_RANK]; /* in elements */
    int32_t device;             /* GPU ordinal, or -1 for host memory */
} cm_tensor_t;

typedef struct {
    int64_t num_experts;
    int64_t num_selected_experts;
    int32_t activation;         /* 0 SiLU, 1 GELU, 2 ReLU */
} cm_fused_moe_t;

/* apply_topk_softmax_inplace (/root/reference/src/lib.rs:124-155). */
int candle_moe_apply_topk_softmax_inplace(const cm_tensor_t* gating_output, const cm_tensor_t* topk_weight,
                                          const cm_tensor_t* topk_indices,
                                          const cm_tensor_t* token_expert_indices, void* stream);

/* FusedMoE::forward (/root/reference/src/lib.rs:273-335). `output` is the
 * [num_tokens, hidden_dim] tensor of the input dtype that forward returns in
 * the reference (Tensor::zeros at lib.rs:296 plus the accumulation): every
 * element is written, so it needs no clearing. down_weights may be NULL
 * (Rust None). */
int candle_moe_fused_moe_forward(const cm_fused_moe_t* moe, const cm_tensor_t* input,
                                 const cm_tensor_t* gate_weights, const cm_tensor_t* up_weights,
                                 const cm_tensor_t* down_weights, const cm_tensor_t* routing_weights,
                                 const cm_tensor_t* expert_indices, uint32_t moe_type,
                                 const cm_tensor_t* output, void* stream);

/* The validation half of the two calls above, without launching anything
 * (runs without a GPU). Returns CANDLE_MOE_OK or CANDLE_MOE_ERR_INVALID. */
int candle_moe_validate_topk_softmax(const cm_tensor_t* gating_output, const cm_tensor_t* topk_weight,
                                     const cm_tensor_t* topk_indices,
                                     const cm_tensor_t* token_expert_indices);
int candle_moe_validate_fused_moe(const cm_fused_moe_t* moe, const cm_tensor_t* input,
                                  const cm_tensor_t* gate_weights, const cm_tensor_t* up_weights,
                                  const cm_tensor_t* down_weights, const cm_tensor_t* routing_weights,
                                  const cm_tensor_t* expert_indices, uint32_t moe_type,
                                  const cm_tensor_t* output);

#ifdef __cplusplus
}
#endif
#endif /* CANDLE_MOE_H */
