/*
 * CPU oracle for the candle-moe fused-MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the
 * smoke() entry point and bench.py's cpu_baseline leg may load it; the
 * product (libcandle_moe_hip.so and the candle_moe package) never does.
 *
 * It restates, in plain C, the reference's *candle-native* semantics
 * (the path the reference's own tests compare against):
 *   router  : candle_nn::ops::softmax_last_dim + TopKLastDimOp
 *             /root/reference/tests/topk_softmax_tests.rs:29-34, output layout
 *             /root/reference/kernels/topk_softmax.cu:246-254
 *   grouping: /root/reference/kernels/preprocessing.cuh:5-59 (histogram, exclusive
 *             scan, scatter), with a stable order inside each expert
 *   MoE     : naive_forward / naive_qwen3_mlp / naive_nomic_mlp
 *             /root/reference/tests/moe_tests.rs:124-189
 *   act     : /root/reference/kernels/common.cuh:116-138 (SiLU, tanh-GELU, ReLU)
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   om_philox4x32_10   Random123 known-answer vectors (Salmon et al. 2011)
 *   om_topk_softmax    float64 softmax + stable argsort (numpy), closed-form
 *                      special cases (E=1, equal logits, k=E), planted ties
 *   om_preprocess      brute-force counting sort + invariants
 *   om_e4m3_decode     all 256 codes against the OCP e4m3 formula evaluated
 *                      independently and against torch.float8_e4m3fn
 *   om_e4m3_encode     torch.float8_e4m3fn rounding on every finite value, every
 *                      midpoint and its f32 neighbours, subnormals; saturation
 *   om_quantize_fp8    the channel maximum encodes to +-448, layout symmetry
 *                      (kn vs the transposed nk input), zero channels
 *   om_fused_moe       float64 dense matmul (numpy) per expert, one-hot routing
 *                      == dense MLP, k=1/w=1 exact expert MLP, linearity in w
 * Per-op dtype rounding of candle's f16/bf16 path (activation op sequence,
 * matmul accumulation order) is not pinned by any reference vector (the
 * reference ships none); the tolerances of the parity tests absorb it.
 */
#ifndef CANDLE_MOE_ORACLE_H
#define CANDLE_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes follow /root/reference/src/lib.rs:174-182 */
enum { OM_F16 = 0, OM_BF16 = 1, OM_F32 = 2 };
/* activation codes follow /root/reference/src/lib.rs:164-171 */
enum { OM_SILU = 0, OM_GELU = 1, OM_RELU = 2 };
/* moe_type codes follow /root/reference/src/ffi.rs:42 */
enum { OM_QWEN3 = 0, OM_NOMIC = 1 };
/* om_fused_moe modes */
enum { OM_MODE_CANDLE = 0, OM_MODE_EXACT = 1, OM_MODE_F32ACC = 2 };

/* Philox4x32-10 block function. */
void om_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* n normal draws mean + std * N(0,1) (Philox4x32-10 + Box-Muller), f32. */
void om_fill_normal(float* out, size_t n, uint64_t seed, uint64_t stream, float mean, float std_);

/* f32 <-> f16/bf16 (round to nearest even) helpers on raw 16-bit storage. */
void om_f32_to_dtype(const float* in, void* out, size_t n, int dtype);
void om_dtype_to_f32(const void* in, float* out, size_t n, int dtype);

/*
 * Router: softmax over E then top-k, ties to the lower expert index.
 * exp is the f32-rounded f64 exponential and the row sum is the f32-rounded
 * f64 sum (both <= 0.5 ulp); p = e / S is an IEEE f32 division.
 * Writes w[T*k], idx[T*k], tei[T*k] with tei[t*k+j] = j*T + t.
 * Returns 0, or -1 on invalid sizes (k < 1 or k > E).
 */
int om_topk_softmax(const float* logits, int T, int E, int k,
                    float* w, uint32_t* idx, uint32_t* tei);

/* Literal f32 variant: expf and a left-to-right f32 sum (candle's CPU
 * softmax_last_dim as written). Used only to show that the choice above
 * agrees with it. */
int om_topk_softmax_f32lit(const float* logits, int T, int E, int k,
                           float* w, uint32_t* idx, uint32_t* tei);

/*
 * Grouping of (token, slot) pairs by expert (counting sort, stable).
 * offsets[E+2]: exclusive scan of counts, offsets[E] = number of valid
 * pairs, offsets[E+1] = max count. Pairs with idx >= E are dropped.
 * sorted_tok[pos] = p / k, sorted_w[pos] = w[p], sorted_pair[pos] = p.
 */
void om_preprocess(const uint32_t* idx, const float* w, int T, int k, int E,
                   int32_t* offsets, int32_t* sorted_tok, float* sorted_w,
                   int32_t* sorted_pair);

/*
 * Fused MoE forward (candle-native per-expert loop).
 * x [T,H]; gate [E,H,I]; up [E,H,I]; down [E,I,H] (moe_type 0) or NULL;
 * w [T,k] f32; idx [T,k] u32; storage dtype `dtype` for x/gate/up/down.
 * out_init [T,H] f64 (NULL = zeros). out [T,H] f64.
 * mode OM_MODE_CANDLE: every op rounds to dtype, matmuls accumulate in f32.
 * mode OM_MODE_EXACT : everything in f64 from the dtype-valued inputs.
 * mode OM_MODE_F32ACC: the reference kernels' numerics ("f32 accumulation"):
 *                      f32 matmuls and activation, the intermediate h rounded
 *                      once to dtype (the reference keeps it in the dtype,
 *                      /root/reference/kernels/moe.cu:557-583), f32 combine,
 *                      one final rounding of the output to dtype.
 * rows: optional token subset (n_rows tokens, ascending); out is then
 *       [n_rows, H] and only those tokens are computed (NULL = all).
 * nthreads: OpenMP threads (0 = runtime default).
 * Returns 0, or a negative code on invalid arguments.
 */
int om_fused_moe(const void* x, const void* gate, const void* up, const void* down,
                 const float* w, const uint32_t* idx, const double* out_init,
                 double* out, int T, int H, int I, int E, int k, int act,
                 int moe_type, int dtype, int mode, const int32_t* rows,
                 int n_rows, int nthreads);

/*
 * FP8 expert weights (the product's opt-in format, no counterpart in the
 * reference). OCP OFP8 e4m3 (E4M3FN): bias 7, no infinities, 0x7F/0xFF NaN.
 * decode: exact value of a code. encode: nearest value, ties to the even
 * code, |x| >= 448 -> +-448, NaN -> 0x7F.
 * quantize: w [E][K][N] (kn = 1) or [E][N][K] (kn = 0) of dtype ->
 *   scales[e][n] = max_k |w| / 448 (f32 division; 1 for a zero channel),
 *   q[e][n][k] = encode(w / scales[e][n]) (f32 division).
 * dequantize: out[r][k] = decode(q[r][k]) * scales[r] (one f32 product).
 */
float om_e4m3_decode(uint8_t c);
uint8_t om_e4m3_encode(float x);
void om_quantize_fp8(const void* w, int dtype, int E, int K, int N, int kn, uint8_t* q, float* scales);
void om_dequantize_fp8(const uint8_t* q, const float* scales, size_t rows, int K, float* out);

#ifdef __cplusplus
}
#endif
#endif
