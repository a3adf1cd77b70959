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
    if constexpr (LPR >= 64) v = fmaxf(v, xor_lane<32>(v));
    if constexpr (LPR >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (LPR >= 16) v = fmaxf(v, xor_lane<8>(v));
    if constexpr (LPR >= 8) v = fmaxf(v, xor_lane<4>(v));
    if constexpr (LPR >= 4) v = fmaxf(v, xor_lane<2>(v));
    if constexpr (LPR >= 2) v = fmaxf(v, xor_lane<1>(v));
    return v;
}

template <int LPR>
__device__ __forceinline__ double group_sum(double v) {
    if constexpr (LPR >= 64) v += xor_lane<32>(v);
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
    if constexpr (LPR >= 64) argmax_step<32>(v, i);
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

// Softmax over one token's E logits held by a group of LPR lanes (lane g of
// the group: experts e0 .. e0+VPT-1, -inf past E), then the top k in
// descending order, ties to the lower index; lane j % LPR writes output j.
template <int VPT, int LPR, int OUTDT>
__device__ __forceinline__ void softmax_topk_group(const float (&x)[VPT], int e0, int g, int E, int k, int T,
                                                   long long row, bool valid, void* __restrict__ wout,
                                                   uint32_t* __restrict__ iout, uint32_t* __restrict__ eiout) {
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

    softmax_topk_group<VPT, LPR, OUTDT>(x, e0, g, E, k, T, row, valid, wout, iout, eiout);
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

// ------------------------------------------------------------------------
// Router GEMM fused with topk-softmax: logits[t,e] = dtype(sum_h x[t,h] *
// w[e,h]) with f32 accumulation and one rounding to the input dtype (the
// output of candle's matmul / Linear in that dtype), then the softmax and
// top-k above on f32(logits). w is [E,H], candle's Linear weight layout.
// One wave per TPW tokens: lane l multiplies the 8 (f32: 4) consecutive h at
// each step's 16-byte chunk l (16-byte loads of x and of the E weight rows,
// which stay in L2), keeping TPW x EMAX partial sums (f32 FMAs on the
// converted values); the partials go through
// LDS ([value][lane], padded) and lane l sums the 64 partials of the logits
// it owns for the softmax: LPR = 64 / TPW lanes per token, VPT experts each.
// Bound: HBM reading x (T*H*sizeof(dtype)).
template <int DT, int EMAX, int TPW>
__global__ __launch_bounds__(64) void router_topk_kernel(const void* __restrict__ xin, const void* __restrict__ win,
                                                         float* __restrict__ wout, uint32_t* __restrict__ iout,
                                                         uint32_t* __restrict__ eiout, int T, int H, int E, int k) {
    typedef typename Elem<DT>::storage S;
    constexpr int LPR = 64 / TPW;
    constexpr int VPT = EMAX / LPR;
    constexpr int NV = TPW * EMAX;  // partial sums per lane
    constexpr int EPV = 16 / (int)sizeof(S);  // elements per 16-byte load
    constexpr int EC = 8;                      // weight rows per batch of loads
    static_assert(VPT * LPR == EMAX && EMAX % EC == 0, "router tile");
    __shared__ float s_part[NV][65];
    const int lane = threadIdx.x;
    const long long t0 = (long long)blockIdx.x * TPW;
    const S* X = reinterpret_cast<const S*>(xin);
    const S* W = reinterpret_cast<const S*>(win);
    // acc += x . w over one 16-byte chunk of each
    auto dot16 = [](const u32x4& xq, const u32x4& wq, float acc) {
        if constexpr (DT == kBF16) {
            // (v_dot2_f32_bf16 / _f16 were tried: they do not return the exact
            // sum even where every product and partial sum is representable
            // in f32, so FMAs on converted values)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = fmaf(__uint_as_float(xq[j] << 16), __uint_as_float(wq[j] << 16), acc);
                acc = fmaf(__uint_as_float(xq[j] & 0xffff0000u), __uint_as_float(wq[j] & 0xffff0000u), acc);
            }
        } else if constexpr (DT == kF16) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = fmaf(Elem<kF16>::to_f32((uint16_t)(xq[j] & 0xffffu)), Elem<kF16>::to_f32((uint16_t)(wq[j] & 0xffffu)),
                           acc);
                acc = fmaf(Elem<kF16>::to_f32((uint16_t)(xq[j] >> 16)), Elem<kF16>::to_f32((uint16_t)(wq[j] >> 16)), acc);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = fmaf(__uint_as_float(xq[j]), __uint_as_float(wq[j]), acc);
        }
        return acc;
    };
    float acc[TPW][EMAX];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int e = 0; e < EMAX; ++e) acc[t][e] = 0.f;
    for (int h0 = 0; h0 < H; h0 += 64 * EPV) {
        const int h = h0 + EPV * lane;
        const bool hv = h < H;
        u32x4 xq[TPW];
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            xq[t] = u32x4{0u, 0u, 0u, 0u};
            if (hv && t0 + t < T) xq[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(X + (t0 + t) * H + h));
        }
#pragma unroll
        for (int e0 = 0; e0 < EMAX; e0 += EC) {
            if (e0 >= E) break;
            u32x4 wq[EC];
#pragma unroll
            for (int j = 0; j < EC; ++j) {
                wq[j] = u32x4{0u, 0u, 0u, 0u};
                if (hv && e0 + j < E) wq[j] = *reinterpret_cast<const u32x4*>(W + (long long)(e0 + j) * H + h);
            }
#pragma unroll
            for (int j = 0; j < EC; ++j)
#pragma unroll
                for (int t = 0; t < TPW; ++t) acc[t][e0 + j] = dot16(xq[t], wq[j], acc[t][e0 + j]);
        }
    }
    // transpose-reduce through LDS: value v = t*EMAX + e of every lane
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int e = 0; e < EMAX; ++e) s_part[t * EMAX + e][lane] = acc[t][e];
    __syncthreads();
    const int tl = lane / LPR, g = lane % LPR, e0 = g * VPT;
    float x[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int e = e0 + j;
        float sum = 0.f;
        for (int i = 0; i < 64; ++i) sum += s_part[tl * EMAX + e][i];
        // the logit as the matmul would store it in the input dtype
        x[j] = e < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(sum)) : -__builtin_inff();
    }
    const long long row = t0 + tl;
    const bool valid = row < T;
    softmax_topk_group<VPT, LPR, kF32>(x, e0, g, E, k, T, valid ? row : 0, valid, wout, iout, eiout);
}

template <int DT, int EMAX, int TPW>
static hipError_t launch_router_cfg(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                    int H, int E, int k, hipStream_t stream) {
    const long long grid = (T + TPW - 1) / TPW;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((router_topk_kernel<DT, EMAX, TPW>), dim3((unsigned)grid), dim3(64), 0, stream, x, w, wo, io,
                       eo, T, H, E, k);
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_router_dt(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                   int H, int E, int k, hipStream_t stream) {
    if (E <= 8) return launch_router_cfg<DT, 8, 8>(x, w, wo, io, eo, T, H, E, k, stream);
    if (E <= 16) return launch_router_cfg<DT, 16, 4>(x, w, wo, io, eo, T, H, E, k, stream);
    if (E <= 32) return launch_router_cfg<DT, 32, 2>(x, w, wo, io, eo, T, H, E, k, stream);
    if (E <= 64) return launch_router_cfg<DT, 64, 1>(x, w, wo, io, eo, T, H, E, k, stream);
    if (E <= 128) return launch_router_cfg<DT, 128, 1>(x, w, wo, io, eo, T, H, E, k, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_router_topk(const void* x, const void* w, int dtype, float* wo, uint32_t* io, uint32_t* eo, int T,
                              int H, int E, int k, hipStream_t stream) {
    if (T == 0) return hipSuccess;
    if (dtype == kBF16) return launch_router_dt<kBF16>(x, w, wo, io, eo, T, H, E, k, stream);
    if (dtype == kF16) return launch_router_dt<kF16>(x, w, wo, io, eo, T, H, E, k, stream);
    if (dtype == kF32) return launch_router_dt<kF32>(x, w, wo, io, eo, T, H, E, k, stream);
    return hipErrorInvalidValue;
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
