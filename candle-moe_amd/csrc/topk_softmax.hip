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
// the group: experts e0 + q*ESTR, q < VPT, -inf past E), then the top k in
// descending order, ties to the lower index; lane j % LPR writes output j.
template <int VPT, int LPR, int OUTDT, int ESTR = 1>
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
        p[j] = (e0 + j * ESTR < E) ? (float)exp((double)d) : 0.0f;
        s += (double)p[j];
    }
    s = group_sum<LPR>(s);
    const float S = (float)s;
#pragma unroll
    for (int j = 0; j < VPT; ++j) p[j] = (e0 + j * ESTR < E) ? p[j] / S : -1.0f;

    typedef typename Elem<OUTDT>::storage WS;
    WS* wo = reinterpret_cast<WS*>(wout);
    for (int j = 0; j < k; ++j) {
        float bv = p[0];
        int bi = e0;
#pragma unroll
        for (int q = 1; q < VPT; ++q)
            if (p[q] > bv) { bv = p[q]; bi = e0 + q * ESTR; }
        group_argmax<LPR>(bv, bi);
        if (valid && g == (j % LPR)) {
            const long long o = row * (long long)k + j;
            wo[o] = Elem<OUTDT>::from_f32(bv);
            iout[o] = (uint32_t)bi;
            eiout[o] = (uint32_t)j * (uint32_t)T + (uint32_t)row;
        }
#pragma unroll
        for (int q = 0; q < VPT; ++q)
            if (e0 + q * ESTR == bi) p[q] = -2.0f;
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
// Reduce-scatter of 64 values over the 64 lanes of a wave: afterwards lane l
// holds the wave-wide sum of value l. At the step for lane bit b the lanes
// with that bit set keep the upper half of the remaining values, the others
// the lower half, and each adds its partner's copy of the half it keeps.
template <int HALF>
__device__ __forceinline__ void reduce_scatter_step(float* v, int lane) {
    const bool hi = (lane & HALF) != 0;
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
        const float a = v[i], b = v[i + HALF];
        const float send = hi ? a : b;
        v[i] = (hi ? b : a) + xor_lane<HALF>(send);
    }
}
__device__ __forceinline__ float reduce_scatter64(float (&v)[64], int lane) {
    reduce_scatter_step<32>(v, lane);
    reduce_scatter_step<16>(v, lane);
    reduce_scatter_step<8>(v, lane);
    reduce_scatter_step<4>(v, lane);
    reduce_scatter_step<2>(v, lane);
    reduce_scatter_step<1>(v, lane);
    return v[0];
}

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
    constexpr bool RS = (NV == 64);  // reduce-scatter in registers, else through LDS
    __shared__ float s_part[RS ? 1 : NV][65];
    const int lane = threadIdx.x;
    const S* X = reinterpret_cast<const S*>(xin);
    const S* W = reinterpret_cast<const S*>(win);
    const long long t0 = (long long)blockIdx.x * TPW;
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
            if (e0 >= E) continue;
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
    const int tl = lane / LPR, g = lane % LPR, e0 = g * VPT;
    float x[VPT];
    if constexpr (RS) {
        // lane l = t*EMAX + e receives logit (t, e): LPR = EMAX, VPT = 1
        const float sum = reduce_scatter64(reinterpret_cast<float(&)[64]>(acc), lane);
        x[0] = e0 < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(sum)) : -__builtin_inff();
    } else {
        // transpose-reduce through LDS: value v = t*EMAX + e of every lane
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int e = 0; e < EMAX; ++e) s_part[t * EMAX + e][lane] = acc[t][e];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int e = e0 + j;
            float sum = 0.f;
            for (int i = 0; i < 64; ++i) sum += s_part[tl * EMAX + e][i];
            // the logit as the matmul would store it in the input dtype
            x[j] = e < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(sum)) : -__builtin_inff();
        }
    }
    const long long row = t0 + tl;
    const bool valid = row < T;
    softmax_topk_group<VPT, LPR, kF32>(x, e0, g, E, k, T, valid ? row : 0, valid, wout, iout, eiout);
}

// 16-bit router on the matrix cores: one workgroup per 32 tokens, KW waves
// splitting K (wave w takes the 32-wide chunks w, w+KW, ...), the E experts
// padded to NB blocks of 32 columns, v_mfma_f32_32x32x16 with both operands
// straight from global memory: the K order inside each 32-wide chunk is
// permuted identically for x and the weight rows (lane half hh takes the 16
// consecutive h at 16*hh, as two MFMA k16 steps), so that every lane loads 32
// contiguous bytes of its row. The result layout puts expert 32c + l%32 of
// token 8(i/4) + 4(l/32) + i%4 in register i of block c of lane l. The KW
// partial sums meet in LDS (summed in wave order: deterministic); wave w then
// takes registers i of [16w/KW, 16(w+1)/KW), each one token per 32-lane half,
// for the softmax over 32-lane groups (VPT = NB experts per lane, stride 32).
// Every workgroup reads the whole weight (E*H*2 bytes) once from L2, so the
// K split (rather than fewer tokens per workgroup) is what spreads a small
// batch over more waves.
template <int DT, int NB, int KW, int D>
__global__ __launch_bounds__(64 * KW) void router_mfma_kernel(const void* __restrict__ xin,
                                                              const void* __restrict__ win,
                                                              float* __restrict__ wout, uint32_t* __restrict__ iout,
                                                              uint32_t* __restrict__ eiout, int T, int H, int E,
                                                              int k) {
    static_assert(KW == 4 || KW == 8, "waves");
    typedef typename Elem<DT>::storage S;
    __shared__ float red[KW][NB][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long long t0 = (long long)blockIdx.x * 32;  // < T (grid = ceil(T/32))
    const int r = lane & 31, hh = lane >> 5;
    const long long xrow = t0 + r < T ? t0 + r : (long long)T - 1;  // rows past T compute garbage, unused
    const S* xr = reinterpret_cast<const S*>(xin) + xrow * H + 16 * hh;
    const S* wr[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c)
        wr[c] = reinterpret_cast<const S*>(win) + (long long)(r + 32 * c < E ? r + 32 * c : 0) * H + 16 * hh;
    f32x16 acc[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
    const u32x4 z = {0u, 0u, 0u, 0u};
    // D of this wave's chunks in flight: the loads of its chunk j + D are
    // issued as chunk j is consumed (slot = j % D, unrolled so slots are
    // registers)
    u32x4 xa[D][2], wb[D][NB][2];
    auto load = [&](int sl, int j) {
        const int k0 = (wave + KW * j) * 32;
        const bool in0 = k0 + 16 * hh < H, in1 = k0 + 16 * hh + 8 < H;
        xa[sl][0] = in0 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + k0)) : z;
        xa[sl][1] = in1 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + k0 + 8)) : z;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const bool ev = r + 32 * c < E;
            wb[sl][c][0] = (ev && in0) ? *reinterpret_cast<const u32x4*>(wr[c] + k0) : z;
            wb[sl][c][1] = (ev && in1) ? *reinterpret_cast<const u32x4*>(wr[c] + k0 + 8) : z;
        }
    };
    const int nch = (H + 31) / 32;
    const int mine = nch > wave ? (nch - wave + KW - 1) / KW : 0;  // this wave's chunks
#pragma unroll
    for (int sl = 0; sl < D; ++sl)
        if (sl < mine) load(sl, sl);
    for (int j0 = 0; j0 < mine; j0 += D) {
#pragma unroll
        for (int sl = 0; sl < D; ++sl) {
            if (j0 + sl < mine) {
#pragma unroll
                for (int c = 0; c < NB; ++c) {
                    acc[c] = mfma32<DT>(xa[sl][0], wb[sl][c][0], acc[c]);
                    acc[c] = mfma32<DT>(xa[sl][1], wb[sl][c][1], acc[c]);
                }
                if (j0 + sl + D < mine) load(sl, j0 + sl + D);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[wave][c][i][lane] = acc[c][i];
    __syncthreads();
    constexpr int RPW = 16 / KW;  // result registers per wave
#pragma unroll
    for (int ii = 0; ii < RPW; ++ii) {
        const int i = RPW * wave + ii;
        const long long row = t0 + 8 * (i / 4) + 4 * hh + (i % 4);
        const bool valid = row < T;
        float x[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            float sum = red[0][c][i][lane];
#pragma unroll
            for (int w = 1; w < KW; ++w) sum += red[w][c][i][lane];
            // the logit as the matmul would store it in the input dtype
            x[c] = r + 32 * c < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(sum)) : -__builtin_inff();
        }
        softmax_topk_group<NB, 32, kF32, 32>(x, r, r, E, k, T, valid ? row : 0, valid, wout, iout, eiout);
    }
}

template <int DT, int NB>
static hipError_t launch_router_mfma(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                     int H, int E, int k, hipStream_t stream) {
    const long long grid = ((long long)T + 31) / 32;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    // fewer workgroups than CUs: 8 waves per workgroup, otherwise 4
    constexpr int D = NB == 2 ? 4 : 3;
    if (grid < 256)
        hipLaunchKernelGGL((router_mfma_kernel<DT, NB, 8, D>), dim3((unsigned)grid), dim3(512), 0, stream, x, w, wo,
                           io, eo, T, H, E, k);
    else
        hipLaunchKernelGGL((router_mfma_kernel<DT, NB, 4, D>), dim3((unsigned)grid), dim3(256), 0, stream, x, w, wo,
                           io, eo, T, H, E, k);
    return hipGetLastError();
}

template <int DT, int EMAX, int TPW>
static hipError_t launch_router_cfg(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                    int H, int E, int k, hipStream_t stream) {
    const long long groups = (T + TPW - 1) / TPW;
    if (groups > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((router_topk_kernel<DT, EMAX, TPW>), dim3((unsigned)groups), dim3(64), 0, stream, x, w, wo, io,
                       eo, T, H, E, k);
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_router_dt(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                   int H, int E, int k, hipStream_t stream) {
    // 16-bit with more than 32 experts: the matrix-core kernel (2.5x faster
    // than the FMA kernel at E=128); up to 32 experts the FMA kernel, whose
    // coalesced row loads beat the MFMA kernel's strided fragments 2x
    if constexpr (DT != kF32) {
        if (E > 32 && E <= 64) return launch_router_mfma<DT, 2>(x, w, wo, io, eo, T, H, E, k, stream);
        if (E > 64) return launch_router_mfma<DT, 4>(x, w, wo, io, eo, T, H, E, k, stream);
    }
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
