// Router: softmax over the experts of each token, then top-k selection.
//
// Semantics follow the reference kernel and the candle-native path it is
// tested against (/root/reference/kernels/topk_softmax.cu:136-266,
// /root/reference/tests/topk_softmax_tests.rs:29-34):
//   p_e = exp(x_e - max) / sum_e' exp(x_e' - max)
//   the k largest p in descending order, ties to the lower expert index,
//   topk_weight[t,j] = p, topk_indices[t,j] = e, token_expert_indices[t,j] = j*T + t.
// Numerics (shared with the CPU oracle so indices agree bit-exactly):
//   exp is evaluated in f64 and rounded once to f32, the row sum is an f64
//   sum rounded once to f32, and p = e / S is an IEEE f32 division.
//
// Layout: one group of LPR lanes per token row; lane g of the group owns
// the VPT consecutive experts [g*VPT, g*VPT+VPT), loaded with 16-byte
// vector loads, so a wave reads 64/LPR whole rows as one contiguous span.
// Max, sum and argmax are butterflies over the group (DPP quad_perm,
// ds_swizzle), so no LDS and no barriers are used.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

template <int LPR, typename V>
__device__ __forceinline__ V group_max(V v) {
    if constexpr (LPR >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (LPR >= 16) v = fmaxf(v, xor_lane<8>(v));
    if constexpr (LPR >= 8) v = fmaxf(v, xor_lane<4>(v));
    if constexpr (LPR >= 4) v = fmaxf(v, xor_lane<2>(v));
    if constexpr (LPR >= 2) v = fmaxf(v, xor_lane<1>(v));
    return v;
}

template <int LPR>
__device__ __forceinline__ double group_sum(double v) {
    if constexpr (LPR >= 32) v += xor_lane<16>(v);
    if constexpr (LPR >= 16) v += xor_lane<8>(v);
    if constexpr (LPR >= 8) v += xor_lane<4>(v);
    if constexpr (LPR >= 4) v += xor_lane<2>(v);
    if constexpr (LPR >= 2) v += xor_lane<1>(v);
    return v;
}

template <int M>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
    const float ov = xor_lane<M>(v);
    const int oi = xor_lane_i32<M>(i);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

template <int LPR>
__device__ __forceinline__ void group_argmax(float& v, int& i) {
    if constexpr (LPR >= 32) argmax_step<16>(v, i);
    if constexpr (LPR >= 16) argmax_step<8>(v, i);
    if constexpr (LPR >= 8) argmax_step<4>(v, i);
    if constexpr (LPR >= 4) argmax_step<2>(v, i);
    if constexpr (LPR >= 2) argmax_step<1>(v, i);
}

template <int VPT, int INDT>
__device__ __forceinline__ void load_row_values(const void* __restrict__ logits, long long row, int E,
                                                int e0, bool full, float (&x)[VPT]) {
    typedef typename Elem<INDT>::storage S;
    const S* src = reinterpret_cast<const S*>(logits) + row * (long long)E + e0;
    constexpr int BYTES = VPT * (int)sizeof(S);
    if (full && (BYTES % 16 == 0)) {
        constexpr int NV = BYTES / 16;
        const u32x4* vp = reinterpret_cast<const u32x4*>(src);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const u32x4 q = __builtin_nontemporal_load(vp + v);
            if constexpr (INDT == kF32) {
#pragma unroll
                for (int j = 0; j < 4; ++j) x[v * 4 + j] = __uint_as_float(q[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[v * 8 + 2 * j] = Elem<INDT>::to_f32((uint16_t)(q[j] & 0xffffu));
                    x[v * 8 + 2 * j + 1] = Elem<INDT>::to_f32((uint16_t)(q[j] >> 16));
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            x[j] = (e0 + j < E) ? Elem<INDT>::to_f32(src[j]) : -__builtin_inff();
    }
}

template <int VPT, int LPR, int INDT, int OUTDT>
__global__ __launch_bounds__(128) void topk_softmax_kernel(const void* __restrict__ logits,
                                                          void* __restrict__ wout,
                                                          uint32_t* __restrict__ iout,
                                                          uint32_t* __restrict__ eiout, int T, int E,
                                                          int k, int aligned) {
    const long long gtid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long row = gtid / LPR;
    const int g = (int)(gtid % LPR);
    // Lanes past the last row still take part in the group butterflies
    // (their group is entirely past the end, so it only reads row T-1).
    const bool valid = row < T;
    const long long r = valid ? row : (long long)T - 1;
    const int e0 = g * VPT;
    const bool full = aligned && (E == LPR * VPT);

    float x[VPT];
    load_row_values<VPT, INDT>(logits, r, E, e0, full, x);

    float m = x[0];
#pragma unroll
    for (int j = 1; j < VPT; ++j) m = fmaxf(m, x[j]);
    m = group_max<LPR>(m);

    float p[VPT];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const float d = x[j] - m;
        p[j] = (e0 + j < E) ? (float)exp((double)d) : 0.0f;
        s += (double)p[j];
    }
    s = group_sum<LPR>(s);
    const float S = (float)s;
#pragma unroll
    for (int j = 0; j < VPT; ++j) p[j] = (e0 + j < E) ? p[j] / S : -1.0f;

    typedef typename Elem<OUTDT>::storage WS;
    WS* wo = reinterpret_cast<WS*>(wout);
    for (int j = 0; j < k; ++j) {
        float bv = p[0];
        int bi = e0;
#pragma unroll
        for (int q = 1; q < VPT; ++q)
            if (p[q] > bv) { bv = p[q]; bi = e0 + q; }
        group_argmax<LPR>(bv, bi);
        if (valid && g == (j % LPR)) {
            const long long o = row * (long long)k + j;
            wo[o] = Elem<OUTDT>::from_f32(bv);
            iout[o] = (uint32_t)bi;
            eiout[o] = (uint32_t)j * (uint32_t)T + (uint32_t)row;
        }
#pragma unroll
        for (int q = 0; q < VPT; ++q)
            if (e0 + q == bi) p[q] = -2.0f;
    }
}

template <int VPT, int LPR, int INDT, int OUTDT>
static hipError_t launch_cfg(const void* logits, void* w, uint32_t* idx, uint32_t* ei, int T, int E,
                             int k, hipStream_t stream) {
    constexpr int BLOCK = 128;
    const long long threads = (long long)T * LPR;
    const unsigned grid = (unsigned)cdivll(threads, BLOCK);
    const int aligned = ((uintptr_t)logits % 16) == 0;
    hipLaunchKernelGGL((topk_softmax_kernel<VPT, LPR, INDT, OUTDT>), dim3(grid), dim3(BLOCK), 0, stream,
                       logits, w, idx, ei, T, E, k, aligned);
    return hipGetLastError();
}

template <int INDT, int OUTDT>
static hipError_t launch_dt(const void* logits, void* w, uint32_t* idx, uint32_t* ei, int T, int E, int k,
                            hipStream_t stream) {
    if (E <= 1) return launch_cfg<1, 1, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 2) return launch_cfg<2, 1, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 4) return launch_cfg<4, 1, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 8) return launch_cfg<8, 1, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 16) return launch_cfg<8, 2, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 32) return launch_cfg<8, 4, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 64) return launch_cfg<8, 8, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 128) return launch_cfg<8, 16, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 256) return launch_cfg<8, 32, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    if (E <= 512) return launch_cfg<16, 32, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
    return launch_cfg<32, 32, INDT, OUTDT>(logits, w, idx, ei, T, E, k, stream);
}

hipError_t launch_topk_softmax(const void* logits, int in_dtype, void* w, int w_dtype, uint32_t* idx,
                               uint32_t* ei, int T, int E, int k, hipStream_t stream) {
    if (T == 0) return hipSuccess;
    if (in_dtype == kF32 && w_dtype == kF32) return launch_dt<kF32, kF32>(logits, w, idx, ei, T, E, k, stream);
    if (in_dtype == kBF16 && w_dtype == kBF16) return launch_dt<kBF16, kBF16>(logits, w, idx, ei, T, E, k, stream);
    if (in_dtype == kF16 && w_dtype == kF16) return launch_dt<kF16, kF16>(logits, w, idx, ei, T, E, k, stream);
    if (in_dtype == kBF16 && w_dtype == kF32) return launch_dt<kBF16, kF32>(logits, w, idx, ei, T, E, k, stream);
    if (in_dtype == kF16 && w_dtype == kF32) return launch_dt<kF16, kF32>(logits, w, idx, ei, T, E, k, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
