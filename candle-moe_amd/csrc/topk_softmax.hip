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
//   f32 weights over 64..256 experts take an f32 softmax first (exp within
//   1 ulp, weights within 5.4e-7 of the above) and keep it for every row
//   whose top k + 1 are far enough apart that the exact p order is the same;
//   the other rows redo the exact softmax.
//
// Layout: one group of LPR lanes per token row; lane g of the group owns
// the VPT consecutive experts [g*VPT, g*VPT+VPT), loaded with 16-byte
// vector loads, so a wave reads 64/LPR whole rows as one contiguous span.
// Max, sum and the selection are butterflies over the group (DPP and
// v_permlane16/32_swap lane exchanges, all VALU); LDS holds only the row of
// probabilities the fast selection reads its weights back from.
#include "cm_common.hpp"
#include "cm_internal.hpp"
#include "cm_lds.hpp"

namespace cm {

// Lane-group exchange step M (1, 2, 4, 8, 16, 32): a and b are the values of
// a lane pair that straddles the two halves of an aligned group of 2M lanes
// (quad xor 1 / 2 by DPP quad_perm, mirror inside 8 / 16 lanes by DPP
// row_half_mirror / row_mirror, the row swaps of v_permlane16 / 32_swap);
// both lanes of a pair get the same (a, b). All VALU, no LDS round trip.
// A symmetric combine of (a, b) over the steps M < LPR leaves every lane of
// an LPR-lane group with the reduction of the whole group.
template <int M>
__device__ __forceinline__ void lane_pair(uint32_t v, uint32_t& a, uint32_t& b) {
    if constexpr (M == 16 || M == 32) {
        const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                               : __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = r[0];
        b = r[1];
    } else {
        constexpr int ctrl = M == 1 ? 0xB1 : (M == 2 ? 0x4E : (M == 4 ? 0x141 : 0x140));
        a = v;
        b = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, false);
    }
}

template <int M>
__device__ __forceinline__ float max_step(float v) {
    uint32_t a, b;
    lane_pair<M>(__float_as_uint(v), a, b);
    return fmaxf(__uint_as_float(a), __uint_as_float(b));
}
template <int M>
__device__ __forceinline__ double sum_step(double v) {
    const uint64_t u = __double_as_longlong(v);
    uint32_t al, bl, ah, bh;
    lane_pair<M>((uint32_t)u, al, bl);
    lane_pair<M>((uint32_t)(u >> 32), ah, bh);
    // a + b in the same order on both lanes of the pair: identical sums
    return __longlong_as_double(((uint64_t)ah << 32) | al) + __longlong_as_double(((uint64_t)bh << 32) | bl);
}

template <int LPR>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (LPR >= 2) v = max_step<1>(v);
    if constexpr (LPR >= 4) v = max_step<2>(v);
    if constexpr (LPR >= 8) v = max_step<4>(v);
    if constexpr (LPR >= 16) v = max_step<8>(v);
    if constexpr (LPR >= 32) v = max_step<16>(v);
    if constexpr (LPR >= 64) v = max_step<32>(v);
    return v;
}

template <int LPR>
__device__ __forceinline__ double group_sum(double v) {
    if constexpr (LPR >= 2) v = sum_step<1>(v);
    if constexpr (LPR >= 4) v = sum_step<2>(v);
    if constexpr (LPR >= 8) v = sum_step<4>(v);
    if constexpr (LPR >= 16) v = sum_step<8>(v);
    if constexpr (LPR >= 32) v = sum_step<16>(v);
    if constexpr (LPR >= 64) v = sum_step<32>(v);
    return v;
}

// (value, expert) pairs ordered by value, then the lower expert: a total
// order, so the pairwise pick is symmetric and the group agrees on the top.
template <int M>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
    uint32_t va, vb, ia, ib;
    lane_pair<M>(__float_as_uint(v), va, vb);
    lane_pair<M>((uint32_t)i, ia, ib);
    const float fa = __uint_as_float(va), fb = __uint_as_float(vb);
    const bool take_b = (fb > fa) | ((fb == fa) & ((int)ib < (int)ia));
    v = take_b ? fb : fa;
    i = take_b ? (int)ib : (int)ia;
}

template <int LPR>
__device__ __forceinline__ void group_argmax(float& v, int& i) {
    if constexpr (LPR >= 2) argmax_step<1>(v, i);
    if constexpr (LPR >= 4) argmax_step<2>(v, i);
    if constexpr (LPR >= 8) argmax_step<4>(v, i);
    if constexpr (LPR >= 16) argmax_step<8>(v, i);
    if constexpr (LPR >= 32) argmax_step<16>(v, i);
    if constexpr (LPR >= 64) argmax_step<32>(v, i);
}

// f32(e^d) for an f32 d <= 0: the f64 exponential rounded once to f32, as the
// CPU restatement computes it ((float)exp((double)d)). Reduction by ln 2
// (n = rint(d / ln 2), r = d - n ln 2 with ln 2 split in a 40-bit head and a
// tail, both steps exact but the last rounding), e^r = 1 + r (1 + r/2 + ... +
// r^11/12!) by Horner in fused multiply-adds, times 2^n. This exact sequence
// of IEEE f64 operations (every step an explicit fma, no contraction left to
// the compiler) gives the same f32 as glibc's exp for every one of the
// 1,120,927,745 f32 values in [-104, 0] (checked exhaustively); below -104 the
// result rounds to +0. NaN stays NaN.
// The coefficients sit in a mutable __constant__ array so that the compiler
// loads them into scalar registers once instead of rebuilding each 64-bit
// literal in vector registers at every use.
__constant__ double kExpCoef[15] = {
    0x1.71547652b82fep+0,
    0x1.62e42fefa4000p-1,
    -0x1.8432a1b0e2634p-43,
    0x1.1eed8eff8d898p-29,
    0x1.ae64567f544e4p-26,
    0x1.27e4fb7789f5cp-22,
    0x1.71de3a556c734p-19,
    0x1.a01a01a01a01ap-16,
    0x1.a01a01a01a01ap-13,
    0x1.6c16c16c16c17p-10,
    0x1.1111111111111p-7,
    0x1.5555555555555p-5,
    0x1.5555555555555p-3,
    0x1.0000000000000p-1,
    0x1.0000000000000p+0};  // 1/ln2, ln2 head, ln2 tail, 1/12! .. 1/1!
__device__ __forceinline__ float exp_f32_f64(float d) {
#pragma clang fp contract(off)
    const double x = (double)d;
    const double n = __builtin_rint(x * kExpCoef[0]);
    double r = __builtin_fma(-n, kExpCoef[1], x);
    r = __builtin_fma(-n, kExpCoef[2], r);
    double s = kExpCoef[3];
#pragma unroll
    for (int i = 4; i < 15; ++i) s = __builtin_fma(r, s, kExpCoef[i]);
    const double y = __builtin_ldexp(__builtin_fma(s, r, 1.0), (int)n);
    return d < -104.0f ? 0.0f : (float)y;
}

// e^d in f32 arithmetic for an f32 d <= 0, within 1 ulp of the correctly
// rounded value wherever that is a normal number (d >= -87.33; checked on the
// GPU against exp_f32_f64 for every f32 d in that range: 96.7 % equal, the
// rest 1 ulp apart). t = d log2(e) is carried as th + tl: th = f32(d L) with
// L = f32(log2 e), tl = the product's rounding error (an exact fma) plus
// d (log2 e - L); then 2^t = 2^th (1 + tl ln 2) to first order, |tl| being
// below 2^-16. 2^th is the hardware v_exp_f32. Below the normal range the
// result is approximate (possibly 0); below -104 it is +0, as above.
__device__ __forceinline__ float exp_f32_fast(float d) {
#pragma clang fp contract(off)
    constexpr float L = 1.44269504088896341f;        // log2(e) rounded to f32
    constexpr float Llo = 1.9259629911783648e-08f;   // log2(e) - L
    constexpr float LN2 = 0.693147180559945309f;
    const float th = d * L;
    const float tl = __builtin_fmaf(d, Llo, __builtin_fmaf(d, L, -th));
    const float y = __builtin_amdgcn_exp2f(th);
    return d < -104.0f ? 0.0f : __builtin_fmaf(y, tl * LN2, y);
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

// Selection keys: (p, expert) in the order p descending, then the lower
// expert, as one unsigned 64-bit value: high word the bits of p (p >= +0, so
// its bits order like its value), low word ~expert. Slots past E get p = +0
// and an expert >= E, so they order after every real expert (also those
// with p = 0), and k <= E never selects them.
__device__ __forceinline__ uint64_t sel_key(float p, int e) {
    return ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(~(uint32_t)e);
}
// a, b -> (max, min)
__device__ __forceinline__ void key_cx(uint64_t& a, uint64_t& b) {
    const bool s = b > a;
    const uint64_t hi = s ? b : a, lo = s ? a : b;
    a = hi;
    b = lo;
}
// Sorting networks (descending), checked exhaustively over 0/1 inputs in the
// tests: 1 comparator for 2 keys, 5 for 4, 19 for 8.
template <int N>
__device__ __forceinline__ void sort_keys(uint64_t (&k)[N]) {
    if constexpr (N == 2) {
        key_cx(k[0], k[1]);
    } else if constexpr (N == 4) {
        key_cx(k[0], k[1]); key_cx(k[2], k[3]);
        key_cx(k[0], k[2]); key_cx(k[1], k[3]);
        key_cx(k[1], k[2]);
    } else if constexpr (N == 8) {
        key_cx(k[0], k[2]); key_cx(k[1], k[3]); key_cx(k[4], k[6]); key_cx(k[5], k[7]);
        key_cx(k[0], k[4]); key_cx(k[1], k[5]); key_cx(k[2], k[6]); key_cx(k[3], k[7]);
        key_cx(k[0], k[1]); key_cx(k[2], k[3]); key_cx(k[4], k[5]); key_cx(k[6], k[7]);
        key_cx(k[2], k[4]); key_cx(k[3], k[5]);
        key_cx(k[1], k[4]); key_cx(k[3], k[6]);
        key_cx(k[1], k[2]); key_cx(k[3], k[4]); key_cx(k[5], k[6]);
    } else {
        static_assert(N == 1, "sort_keys: 1, 2, 4 or 8 keys");
    }
}
// The lanes of `mask` (a wave-wide lane mask) take b, the others keep a: one
// v_cndmask_b32 per 32-bit word. (Written as a plain select inside the
// head-drop shift below, the compiler turns `pop ? key[q+1] : key[q]` into
// an indexed read key[q + pop] and expands that into a compare chain per
// slot.)
__device__ __forceinline__ uint64_t key_take(uint64_t a, uint64_t b, uint64_t mask) {
    uint32_t lo, hi;
    asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(lo) : "v"((uint32_t)a), "v"((uint32_t)b), "s"(mask));
    asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(hi) : "v"((uint32_t)(a >> 32)), "v"((uint32_t)(b >> 32)), "s"(mask));
    return ((uint64_t)hi << 32) | lo;
}
// 32-bit keys: compare-exchange by max / min, the same networks.
__device__ __forceinline__ void key32_cx(uint32_t& a, uint32_t& b) {
    const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
    a = hi;
    b = lo;
}
template <int N>
__device__ __forceinline__ void sort_keys32(uint32_t (&k)[N]) {
    if constexpr (N == 2) {
        key32_cx(k[0], k[1]);
    } else if constexpr (N == 4) {
        key32_cx(k[0], k[1]); key32_cx(k[2], k[3]);
        key32_cx(k[0], k[2]); key32_cx(k[1], k[3]);
        key32_cx(k[1], k[2]);
    } else if constexpr (N == 8) {
        key32_cx(k[0], k[2]); key32_cx(k[1], k[3]); key32_cx(k[4], k[6]); key32_cx(k[5], k[7]);
        key32_cx(k[0], k[4]); key32_cx(k[1], k[5]); key32_cx(k[2], k[6]); key32_cx(k[3], k[7]);
        key32_cx(k[0], k[1]); key32_cx(k[2], k[3]); key32_cx(k[4], k[5]); key32_cx(k[6], k[7]);
        key32_cx(k[2], k[4]); key32_cx(k[3], k[5]);
        key32_cx(k[1], k[4]); key32_cx(k[3], k[6]);
        key32_cx(k[1], k[2]); key32_cx(k[3], k[4]); key32_cx(k[5], k[6]);
    } else {
        static_assert(N == 1, "sort_keys32: 1, 2, 4 or 8 keys");
    }
}
__device__ __forceinline__ uint32_t key_take32(uint32_t a, uint32_t b, uint64_t mask) {
    uint32_t r;
    asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
    return r;
}
// max(v, v of the partner lane) in one DPP-modified v_max_u32 for the
// steps inside a row of 16 lanes (the s_nop covers the wait states between a
// VALU write of v and its DPP read, which the compiler does not track across
// inline asm).
template <int M>
__device__ __forceinline__ uint32_t key32_max_step(uint32_t v) {
    if constexpr (M == 1 || M == 2 || M == 4 || M == 8) {
        uint32_t r;
        if constexpr (M == 1)
            asm volatile("s_nop 1\n\tv_max_u32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
                         : "=v"(r) : "v"(v));
        else if constexpr (M == 2)
            asm volatile("s_nop 1\n\tv_max_u32_dpp %0, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
                         : "=v"(r) : "v"(v));
        else if constexpr (M == 4)
            asm volatile("s_nop 1\n\tv_max_u32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf"
                         : "=v"(r) : "v"(v));
        else
            asm volatile("s_nop 1\n\tv_max_u32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xf"
                         : "=v"(r) : "v"(v));
        return r;
    } else {
        uint32_t a, b;
        lane_pair<M>(v, a, b);
        return a > b ? a : b;
    }
}
template <int LPR>
__device__ __forceinline__ uint32_t group_key32_max(uint32_t v) {
    if constexpr (LPR >= 2) v = key32_max_step<1>(v);
    if constexpr (LPR >= 4) v = key32_max_step<2>(v);
    if constexpr (LPR >= 8) v = key32_max_step<4>(v);
    if constexpr (LPR >= 16) v = key32_max_step<8>(v);
    if constexpr (LPR >= 32) v = key32_max_step<16>(v);
    if constexpr (LPR >= 64) v = key32_max_step<32>(v);
    return v;
}
// Largest key of an LPR-lane group (every lane of the group gets it).
template <int M>
__device__ __forceinline__ uint64_t key_max_step(uint64_t v) {
    uint32_t al, bl, ah, bh;
    lane_pair<M>((uint32_t)v, al, bl);
    lane_pair<M>((uint32_t)(v >> 32), ah, bh);
    const uint64_t a = ((uint64_t)ah << 32) | al, b = ((uint64_t)bh << 32) | bl;
    return b > a ? b : a;
}
template <int LPR>
__device__ __forceinline__ uint64_t group_key_max(uint64_t v) {
    if constexpr (LPR >= 2) v = key_max_step<1>(v);
    if constexpr (LPR >= 4) v = key_max_step<2>(v);
    if constexpr (LPR >= 8) v = key_max_step<4>(v);
    if constexpr (LPR >= 16) v = key_max_step<8>(v);
    if constexpr (LPR >= 32) v = key_max_step<16>(v);
    if constexpr (LPR >= 64) v = key_max_step<32>(v);
    return v;
}

// Softmax over one token's E logits held by a group of LPR lanes (lane g of
// the group: experts e0 + q*ESTR, q < VPT, -inf past E), then the top k in
// descending order, ties to the lower index; output j of a row is written by
// lane j of its group (k <= LPR, one coalesced store per output tensor after
// the k passes) or lane j % LPR right away (k > LPR).
// R independent tokens per lane group at once (row r's logits in x[r]): their
// cross-lane exchanges interleave, which hides the exchange latencies when a
// SIMD holds a single wave.
// Selection (VPT <= 8): each lane sorts its VPT keys once; pass j takes the
// group's largest head key and the lane that owned it drops its head.
template <int VPT, int LPR, int OUTDT, int ESTR, int R, bool TIES = false>
__device__ __forceinline__ void softmax_topk_rows(const float (&x)[R][VPT], int e0, int g, int E, int k, int T,
                                                  const long long (&row)[R], const bool (&valid)[R],
                                                  void* __restrict__ wout, uint32_t* __restrict__ iout,
                                                  uint32_t* __restrict__ eiout, float* s_row = nullptr) {
    float m[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = x[r][0];
#pragma unroll
        for (int j = 1; j < VPT; ++j) m[r] = fmaxf(m[r], x[r][j]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) m[r] = group_max<LPR>(m[r]);

    typedef typename Elem<OUTDT>::storage WS;
    WS* wo = reinterpret_cast<WS*>(wout);
    auto put = [&](long long rw, int j, float v, int e) {
        const long long o = rw * (long long)k + j;
        wo[o] = Elem<OUTDT>::from_f32(v);
        iout[o] = (uint32_t)e;
        eiout[o] = (uint32_t)j * (uint32_t)T + (uint32_t)rw;
    };

    // f32 weights over 64 to 256 experts (8 per lane, whole rows): the
    // softmax in f32 arithmetic first. e = exp_f32_fast(x - max) (within 1 ulp
    // of the correctly rounded e), S = the f64 sum of those e, p = e * rcp(S).
    // Against the exact p (f32(exp_f64), f64 sum rounded to f32, correctly
    // rounded quotient) each p is within 6e-7 relative (e 1 ulp; S 2.4e-7
    // after both roundings; the reciprocal 1 ulp; the product's and the exact
    // p's roundings 0.6e-7 each), inside the 1e-6 weight tolerance.
    // Selection: k + 1 passes over the lanes' sorted 32-bit keys (as in the
    // exact path below) give the candidates, positions 0 .. c - 1 (c = k + 1)
    // of the key order, lane j of the group keeping position j; the group's
    // next key (position c) is the first expert left out. The top k in the
    // exact order are the candidates' top k when
    //  * position c's key lies at least two units of the key's upper bits
    //    (2^IB ulps each) below position c - 1's: every expert left out then
    //    has p smaller by more than 7.6e-6 relative than every candidate (up
    //    to two more passes move the boundary down when it is not, while
    //    lanes are left to hold the extra candidates);
    //  * no two neighbouring candidates have p within 2e-6 relative (nor in
    //    the wrong order, which the keys allow inside one unit): the exact p
    //    are then ordered as these, being within 6e-7 of them;
    // and the candidates' p are >= 2^-100 (normal e, where the 1-ulp bound
    // holds) and the row is finite. Candidates closer than 2e-6 are ranked
    // by their exact e instead (exp_f32_f64, one per lane), e descending,
    // then the lower expert: p = f32(e / S) with one S for the row is equal
    // for equal e and ordered like e where the e differ by two ulps or more;
    // where they differ by one ulp and the larger e has the higher expert
    // index, equal p (and the lower index first) depends on the exact S.
    // That case, a boundary still too close after the extra passes, tiny p
    // and non-finite rows send the wave to the exact softmax below.
    if constexpr (R == 1 && VPT == 8 && LPR >= 8 && LPR * VPT <= 256 && OUTDT == kF32) {
        if (s_row != nullptr && k < LPR && E == LPR * VPT) {
            constexpr int IB = 32 - __builtin_clz(LPR * VPT - 1);
            constexpr uint32_t MASK = (1u << IB) - 1u;
            constexpr uint32_t TWO_UNITS = 2u << IB;
            constexpr float PMIN = 7.88860905e-31f;  // 2^-100
            constexpr float DELTA = 2e-6f;
            const int lane = (int)(threadIdx.x & 63u);
            const float mf = m[0];
            float pf[VPT];
            double sf = 0.0;
#pragma unroll
            for (int q = 0; q < VPT; ++q) {
                pf[q] = exp_f32_fast(x[0][q] - mf);
                sf += (double)pf[q];
            }
            sf = group_sum<LPR>(sf);
            const float sff = (float)sf;
            const float inv = __builtin_amdgcn_rcpf(sff);
#pragma unroll
            for (int q = 0; q < VPT; ++q) {
                pf[q] *= inv;
                s_row[e0 + q * ESTR] = pf[q];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            uint32_t key[VPT];
#pragma unroll
            for (int q = 0; q < VPT; ++q)
                key[q] = ((__float_as_uint(pf[q]) | MASK) - (uint32_t)(e0 + q * ESTR)) + 1u;
            sort_keys32<VPT>(key);
            uint32_t mine = 0u;  // lane j of the group: the key at position j
            // the group's largest remaining key (every lane of the group gets it)
            auto top = [&]() { return group_key32_max<LPR>(key[0]); };
            // its owner drops it
            auto drop = [&](uint32_t best) {
                const uint64_t pop = __builtin_amdgcn_ballot_w64(key[0] == best);
#pragma unroll
                for (int q = 0; q + 1 < VPT; ++q) key[q] = key_take32(key[q], key[q + 1], pop);
                key[VPT - 1] = key_take32(key[VPT - 1], 0u, pop);
            };
            // key b two units of the upper bits below key a (both >= 1)
            auto far_below = [&](uint32_t a, uint32_t b) {
                const uint32_t ua = (a - 1u) | MASK, ub = (b - 1u) | MASK;
                return ua >= TWO_UNITS && ub <= ua - TWO_UNITS;
            };
            int c = k + 1;
            uint32_t last = 0u;
            for (int j = 0; j < c; ++j) {
                const uint32_t best = top();
                drop(best);
                mine = g == j ? best : mine;
                last = best;
            }
            // the boundary: position c's key (not stored) against position
            // c - 1's; while too close, position c joins the candidates
            uint32_t next = top();
            uint64_t open = __builtin_amdgcn_ballot_w64(!far_below(last, next));
            for (int ext = 0; ext < 2 && open != 0ull && c < LPR; ++ext) {
                drop(next);
                mine = g == c ? next : mine;
                ++c;
                last = next;
                next = top();
                open = __builtin_amdgcn_ballot_w64(!far_below(last, next));
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int ej = (int)(MASK - ((mine - 1u) & MASK));  // lane j < c: candidate j's expert
            const float pj = s_row[ej];
            // p of candidate g - 1 (lane g - 1 of the group; lane 0: its own)
            const int prev_addr = (lane - (g > 0 ? 1 : 0)) << 2;
            const float pprev = __int_as_float(__builtin_amdgcn_ds_bpermute(prev_addr, __float_as_int(pj)));
            const bool near = g >= 1 && g < c && !(pprev - pj >= DELTA * pprev);
            const bool bad = (g < c && !(pj >= PMIN)) || !(sff <= 3.0e38f);
            const uint64_t any_near = __builtin_amdgcn_ballot_w64(near);
            const uint64_t any_bad = __builtin_amdgcn_ballot_w64(bad);
            if (open == 0ull && any_bad == 0ull) {
                if (any_near == 0ull) {
                    if (valid[0] && g < k) put(row[0], g, pj, ej);
                    return;
                }
                // rank the candidates by exact e: the row's logits into the
                // row buffer (its p are read), each candidate's exact e, then
                // (e, expert) pairs at the buffer's start
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int q = 0; q < VPT; ++q) s_row[e0 + q * ESTR] = x[0][q];
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
                const float xj = s_row[ej];
                if constexpr (TIES) {
                    // equal logits (frequent among 16-bit logits) have equal
                    // e, equal p and keys ordered by expert index, the exact
                    // order: where every close pair is such a tie the keys
                    // stand
                    const float xprev = __int_as_float(__builtin_amdgcn_ds_bpermute(prev_addr, __float_as_int(xj)));
                    if (__builtin_amdgcn_ballot_w64(near && !(xprev == xj)) == 0ull) {
                        if (valid[0] && g < k) put(row[0], g, pj, ej);
                        return;
                    }
                }
                const float ee = exp_f32_f64(xj - mf);
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (g < c) {
                    s_row[2 * g] = ee;
                    s_row[2 * g + 1] = __int_as_float(ej);
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
                int rank = 0;
                bool amb = false;
                for (int i = 0; i < c; ++i) {
                    const float ei = s_row[2 * i];
                    const int xi = __float_as_int(s_row[2 * i + 1]);
                    rank += (ei > ee || (ei == ee && xi < ej)) ? 1 : 0;
                    amb = amb || (__float_as_uint(ei) == __float_as_uint(ee) + 1u && xi > ej);
                }
                if (__builtin_amdgcn_ballot_w64(g < c && amb) == 0ull) {
                    if (valid[0] && g < c && rank < k) put(row[0], rank, pj, ej);
                    return;
                }
            }
        }
    }

    float p[R][VPT];
    double s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        s[r] = 0.0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const float d = x[r][j] - m[r];
            const float ex = exp_f32_f64(d);  // every slot: straight-line code
            p[r][j] = (e0 + j * ESTR < E) ? ex : 0.0f;
            s[r] += (double)p[r][j];
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) s[r] = group_sum<LPR>(s[r]);
    // p = e / S in f32: e * (1 / S) with both steps in f64 and one rounding to
    // f32 is the correctly rounded quotient (its error, < 2^-52 relative,
    // stays below the distance of any f32 quotient from a rounding midpoint)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const double inv = 1.0 / (double)(float)s[r];
#pragma unroll
        for (int j = 0; j < VPT; ++j) p[r][j] = (float)((double)p[r][j] * inv);
    }

    // Fast selection on 32-bit keys (R == 1 with an LDS row buffer, k <= LPR): the key
    // of expert e is p's bits with the low IB bits replaced by MASK - e, plus
    // one (so that 0 stays below every expert). Keys order as (upper bits of
    // p, lower expert), and where the upper bits of two keys differ that is
    // the order of (p, lower expert) itself. k + 1 passes over the lanes'
    // sorted keys give the first k + 1 keys; if their upper bits strictly
    // decrease, the first k are the exact top k in order (every other expert
    // has smaller upper bits than the k-th). Otherwise (near-equal p, e.g.
    // planted ties) the wave redoes the row with the exact 64-bit keys below.
    // The weights are the exact p, read back from the row buffer in LDS.
    bool exact_done = false;
    if constexpr (R == 1 && VPT <= 8 && LPR * VPT <= 256) {
        if (s_row != nullptr && k <= LPR) {  // lane j of the group writes output j
            constexpr int IB = (LPR * VPT <= 2) ? 1 : 32 - __builtin_clz(LPR * VPT - 1);
            constexpr uint32_t MASK = (1u << IB) - 1u;
#pragma unroll
            for (int q = 0; q < VPT; ++q) s_row[e0 + q * ESTR] = p[0][q];
            // (read back by other lanes of this wave after the passes: LDS
            // runs one wave's instructions in order; keep the compiler from
            // moving the reads above the writes)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            uint32_t key[VPT];
#pragma unroll
            for (int q = 0; q < VPT; ++q)
                key[q] = ((__float_as_uint(p[0][q]) | MASK) - (uint32_t)(e0 + q * ESTR)) + 1u;
            sort_keys32<VPT>(key);
            uint32_t mine = 0u, prev = 0xffffffffu;
            bool ordered = true;
            for (int j = 0; j <= k; ++j) {
                const uint32_t best = group_key32_max<LPR>(key[0]);
                // (once only zero keys are left every lane pops a zero: harmless)
                const uint64_t pop = __builtin_amdgcn_ballot_w64(key[0] == best);
#pragma unroll
                for (int q = 0; q + 1 < VPT; ++q) key[q] = key_take32(key[q], key[q + 1], pop);
                key[VPT - 1] = key_take32(key[VPT - 1], 0u, pop);
                const uint32_t up = (best - 1u) | MASK;  // upper bits of p (0 keys: none left)
                if (j < k || k < E) ordered = ordered && (best == 0u ? j == k : up < prev);
                prev = up;
                mine = g == j ? best : mine;
            }
            // one wave-wide decision: a row that needs the exact path sends
            // its whole wave there
            if (__builtin_amdgcn_ballot_w64(!ordered) == 0ull) {
                exact_done = true;
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (valid[0] && g < k) {
                    const int e = (int)(MASK - ((mine - 1u) & MASK));
                    put(row[0], g, s_row[e], e);
                }
            }
        }
    }
    if (exact_done) return;
    if constexpr (VPT <= 8) {
        uint64_t key[R][VPT];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int q = 0; q < VPT; ++q) key[r][q] = sel_key(p[r][q], e0 + q * ESTR);
            sort_keys<VPT>(key[r]);
        }
        const bool gather = k <= LPR;  // lane j keeps output j
        float ov[R];
        int oi[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ov[r] = 0.0f;
            oi[r] = 0;
        }
        for (int j = 0; j < k; ++j) {
            uint64_t best[R];
#pragma unroll
            for (int r = 0; r < R; ++r) best[r] = group_key_max<LPR>(key[r][0]);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // the owner of the best key drops its head
                const uint64_t pop = __builtin_amdgcn_ballot_w64(key[r][0] == best[r]);
#pragma unroll
                for (int q = 0; q + 1 < VPT; ++q) key[r][q] = key_take(key[r][q], key[r][q + 1], pop);
                key[r][VPT - 1] = key_take(key[r][VPT - 1], 0ull, pop);
                const float bv = __uint_as_float((uint32_t)(best[r] >> 32));
                const int bi = (int)~(uint32_t)best[r];
                if (gather) {
                    ov[r] = g == j ? bv : ov[r];
                    oi[r] = g == j ? bi : oi[r];
                } else if (valid[r] && g == (j % LPR)) {
                    put(row[r], j, bv, bi);
                }
            }
        }
        if (gather) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (valid[r] && g < k) put(row[r], g, ov[r], oi[r]);
        }
    } else {
        // many experts per lane: k argmax passes over the lane's values
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < VPT; ++j) p[r][j] = (e0 + j * ESTR < E) ? p[r][j] : -1.0f;
        for (int j = 0; j < k; ++j) {
            float bv[R];
            int bi[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                bv[r] = p[r][0];
                bi[r] = e0;
#pragma unroll
                for (int q = 1; q < VPT; ++q) {
                    const bool take = p[r][q] > bv[r];
                    bv[r] = take ? p[r][q] : bv[r];
                    bi[r] = take ? e0 + q * ESTR : bi[r];
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) group_argmax<LPR>(bv[r], bi[r]);
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int q = 0; q < VPT; ++q) p[r][q] = (e0 + q * ESTR == bi[r]) ? -2.0f : p[r][q];
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (valid[r] && g == (j % LPR)) put(row[r], j, bv[r], bi[r]);
        }
    }
}

template <int VPT, int LPR, int OUTDT, int ESTR = 1, bool TIES = false>
__device__ __forceinline__ void softmax_topk_group(const float (&x)[VPT], int e0, int g, int E, int k, int T,
                                                   long long row, bool valid, void* __restrict__ wout,
                                                   uint32_t* __restrict__ iout, uint32_t* __restrict__ eiout,
                                                   float* s_row = nullptr) {
    const float(&xr)[1][VPT] = reinterpret_cast<const float(&)[1][VPT]>(x);
    const long long rr[1] = {row};
    const bool vr[1] = {valid};
    softmax_topk_rows<VPT, LPR, OUTDT, ESTR, 1, TIES>(xr, e0, g, E, k, T, rr, vr, wout, iout, eiout, s_row);
}

template <int VPT, int LPR, int INDT, int OUTDT>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const void* __restrict__ logits,
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

    // one LDS row of p per lane group (the fast selection reads the weights
    // of the chosen experts back from it; written and read by one wave)
    constexpr bool FAST = VPT <= 8 && LPR * VPT <= 256 && LPR > 1;
    __shared__ float s_p[FAST ? 256 / LPR : 1][FAST ? LPR * VPT : 1];
    // (16-bit logits: the shortcut for exactly tied candidates)
    softmax_topk_group<VPT, LPR, OUTDT, 1, INDT != kF32>(x, e0, g, E, k, T, row, valid, wout, iout, eiout,
                                                         FAST ? s_p[threadIdx.x / LPR] : nullptr);
}

template <int VPT, int LPR, int INDT, int OUTDT>
static hipError_t launch_cfg(const void* logits, void* w, uint32_t* idx, uint32_t* ei, int T, int E,
                             int k, hipStream_t stream) {
    constexpr int BLOCK = 256;
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

constexpr int kRouterMaxSlots = 8;  // K splits of the small-batch router at most
// The softmax / top-k of logits given as ns f32 partial sums: logit[t][e] =
// dtype(part[0][t][e] + part[1][t][e] + ... ) summed in slot order (the
// K-split router), rounded once to the router's dtype as the matmul stores it.
template <int VPT, int LPR, int DT>
__global__ __launch_bounds__(256) void topk_partials_kernel(const float* __restrict__ part, int ns,
                                                           void* __restrict__ wout, uint32_t* __restrict__ iout,
                                                           uint32_t* __restrict__ eiout, int T, int E, int k,
                                                           int aligned) {
    const long long gtid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long row = gtid / LPR;
    const int g = (int)(gtid % LPR);
    const bool valid = row < T;
    const long long r = valid ? row : (long long)T - 1;
    const int e0 = g * VPT;
    const bool full = aligned && (E == LPR * VPT);
    // every slot's loads in flight together (ns <= kRouterMaxSlots), then
    // the sums in slot order
    float y[kRouterMaxSlots][VPT];
#pragma unroll
    for (int sl = 0; sl < kRouterMaxSlots; ++sl)
        if (sl < ns) load_row_values<VPT, kF32>(part + (long long)sl * T * E, r, E, e0, full, y[sl]);
    float x[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) x[j] = y[0][j];
#pragma unroll
    for (int sl = 1; sl < kRouterMaxSlots; ++sl)
        if (sl < ns) {
#pragma unroll
            for (int j = 0; j < VPT; ++j) x[j] += y[sl][j];
        }
#pragma unroll
    for (int j = 0; j < VPT; ++j)
        x[j] = e0 + j < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(x[j])) : -__builtin_inff();
    constexpr bool FAST = VPT <= 8 && LPR * VPT <= 256 && LPR > 1;
    __shared__ float s_p[FAST ? 256 / LPR : 1][FAST ? LPR * VPT : 1];
    softmax_topk_group<VPT, LPR, kF32, 1, true>(x, e0, g, E, k, T, row, valid, wout, iout, eiout,
                                                FAST ? s_p[threadIdx.x / LPR] : nullptr);
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

// 16-bit router on the matrix cores (E > 32): one workgroup per 32*MT tokens
// and NB*KH waves, wave (c, h) computing the logits of experts 32c .. 32c+31
// with v_mfma_f32_32x32x16 (A = token rows, B = weight rows, both
// K-contiguous) over the k16 steps h*4/KH .. (h+1)*4/KH-1 of every K tile;
// the waves with h = 0 issue the DMA.
// K tiles of 64 reach LDS by buffer_load ... lds in an NST-stage ring, each
// instruction covering 8 rows x 128 contiguous bytes (row loads straight
// into the MFMA fragment registers touch 32 rows per instruction, which the
// address unit serialises); rows past T or E and the K tail read as zeros.
// Rows of a stage hold 8 16-byte chunks, chunk c of row r at a_swz(r, c)
// (conflict-free fragment reads). The result layout puts expert 32c + l%32
// of token 32m + 8(i/4) + 4(l/32) + i%4 in register i of block m of lane l;
// the waves swap blocks through LDS (summing the KH partial products in
// order) so that each holds whole tokens for the softmax over 32-lane groups
// (VPT = NB experts per lane, stride 32); KH = 2 halves the rows each wave
// ranks, whose top-k passes dominate small batches.
// PART (small batches): the grid is token tiles x ks K splits; split s of a
// tile runs K tiles [s*per, (s+1)*per) and stores each wave's f32 partial
// logits (no rounding, no softmax) to part[s*KH + kh][t][e], for
// topk_partials_kernel to sum in split order.
template <int DT, int NB, int MT, int NST, int KH, bool PART = false>
__global__ __launch_bounds__(64 * NB * KH) void router_mfma_kernel(const void* __restrict__ xin,
                                                              const void* __restrict__ win,
                                                              float* __restrict__ wout, uint32_t* __restrict__ iout,
                                                              uint32_t* __restrict__ eiout, int T, int H, int E,
                                                              int k, float* __restrict__ part = nullptr,
                                                              int ks = 1) {
    using namespace lds;
    typedef typename Elem<DT>::storage S;
    constexpr int TM = 32 * MT;                   // tokens per workgroup
    constexpr int EW = 32 * NB;                   // weight rows (experts, padded)
    constexpr int STAGE = (TM + EW) * 128;        // one K tile of 64: 128 bytes per row
    constexpr int INS = STAGE / 1024;             // DMA instructions per stage (8 rows each)
    constexpr int LOADS = INS / NB;               // per wave
    static_assert(LOADS * NB == INS && LOADS * (NST - 2) < 64, "router stage split");
    static_assert(KH * MT * NB * 16 * 64 * 4 <= NST * STAGE, "softmax exchange fits the ring");
    static_assert(KH == 1 || KH == 2, "K halves");
    __shared__ __attribute__((aligned(1024))) char smem[NST * STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cb = wave % NB, kh = wave / NB;  // expert block, K part
    const int split = PART ? (int)(blockIdx.x % ks) : 0;
    const long long t0 = (long long)(PART ? blockIdx.x / ks : blockIdx.x) * TM;  // < T (grid = ceil(T/TM) x ks)
    const int rows = T - t0 < TM ? (int)(T - t0) : TM;
    const i32x4 rx = make_rsrc(reinterpret_cast<const S*>(xin) + t0 * H, (long long)rows * H * 2);
    const i32x4 rw = make_rsrc(win, (long long)E * H * 2);
    const uint32_t sbase = __builtin_amdgcn_readfirstlane(lds_addr(smem));

    // per-lane source offsets of this wave's LOADS instructions (instruction
    // q = NB*i + wave of the stage: rows 8q .. 8q+7, token rows first), the K
    // position of a full tile in the SGPR offset
    uint32_t off[LOADS];
    int chunk_k[LOADS];
    bool is_x[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int q = NB * i + cb;
        const int row = 8 * q + lane / 8;  // row of the stage
        const int c = a_swz<8>(row, lane % 8);
        chunk_k[i] = 8 * c;
        is_x[i] = 8 * q < TM;  // whole instructions: TM is a multiple of 8 (wave-uniform)
        off[i] = is_x[i] ? ((uint32_t)row * (uint32_t)H + 8u * c) * 2u
                         : ((uint32_t)(row - TM) * (uint32_t)H + 8u * c) * 2u;  // rows >= rows / E: past the resource
    }
    const int nk_all = (H + 63) / 64;
    const int per = (nk_all + ks - 1) / ks;
    const int kt_lo = PART ? min(nk_all, split * per) : 0;
    const int nk = PART ? min(nk_all, kt_lo + per) - kt_lo : nk_all;  // this split's K tiles (may be 0)
    auto issue = [&](int stage, int k0) {
        const uint32_t sl = sbase + stage * STAGE;
        const bool full = k0 + 64 <= H;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t v = (full || k0 + chunk_k[i] < H) ? off[i] : kOob;
            dma16s(is_x[i] ? rx : rw, sl + (NB * i + cb) * 1024, v, (uint32_t)k0 * 2u);
        }
    };

    f32x16 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] = 0.f;
    const int lr = lane & 31, lh = lane >> 5;
    const bool dma = kh == 0;
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (dma && s < nk) issue(s, (kt_lo + s) * 64);
    for (int kt = 0; kt < nk; ++kt) {
        // this wave's DMA of tile kt (NST-2 newer tiles may stay in flight),
        // then the barrier makes every wave's part visible and frees slot kt-1
        const int newer = min(NST - 2, nk - 1 - kt);
        if (newer >= 4) wait_vm<4 * LOADS>();
        else if (newer == 3) wait_vm<3 * LOADS>();
        else if (newer == 2) wait_vm<2 * LOADS>();
        else if (newer == 1) wait_vm<LOADS>();
        else wait_vm<0>();
        wait_lgkm0();
        block_barrier();
        if (dma && kt + NST - 1 < nk) issue((kt + NST - 1) % NST, (kt_lo + kt + NST - 1) * 64);
        const char* sx = smem + (kt % NST) * STAGE;
        const char* sw = sx + TM * 128;
#pragma unroll
        for (int s4 = 0; s4 < 4 / KH; ++s4) {
            const int st = kh * (4 / KH) + s4;
            const int c = 2 * st + lh;
            const int wr = 32 * cb + lr;  // weight row; stage row TM + wr (the swizzle's row)
            const u32x4 b = *reinterpret_cast<const u32x4*>(sw + wr * 128 + a_swz<8>(TM + wr, c) * 16);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int xr = 32 * m + lr;
                const u32x4 a = *reinterpret_cast<const u32x4*>(sx + xr * 128 + a_swz<8>(xr, c) * 16);
                acc[m] = mfma32<DT>(a, b, acc[m]);
            }
        }
    }
    if constexpr (PART) {
        // register i of block m: token 32m + 8(i/4) + 4(l/32) + i%4, expert
        // 32cb + l%32 (32 consecutive experts per store instruction)
        float* dst = part + (long long)(split * KH + kh) * T * E;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const long long t = t0 + 32 * m + 8 * (i / 4) + 4 * lh + (i % 4);
                const int e = 32 * cb + lr;
                if (t < T && e < E) dst[t * E + e] = acc[m][i];
            }
        return;
    }
    // exchange through LDS (the ring is free after the barrier):
    // red[kh][m][c][i][lane]
    wait_lgkm0();
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[(((kh * MT + m) * NB + cb) * 16 + i) * 64 + lane] = acc[m][i];
    __syncthreads();
    // wave w takes result registers g = NW*ii + w ((m, i) = (g / 16, g % 16)):
    // the first tokens spread over all waves when the batch is small
    constexpr int NW = NB * KH;
    constexpr int RPW = MT * 16 / NW;  // result registers per wave
    static_assert(RPW * NW == MT * 16 && RPW % 2 == 0, "register split");
    float x[RPW][NB];
    long long row[RPW];
    bool valid[RPW];
#pragma unroll
    for (int ii = 0; ii < RPW; ++ii) {
        const int g = NW * ii + wave;
        const int m = g / 16, i = g % 16;
        const long long rw_ = t0 + 32 * m + 8 * (i / 4) + 4 * lh + (i % 4);
        valid[ii] = rw_ < T;
        row[ii] = valid[ii] ? rw_ : 0;
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            float v = red[((m * NB + c) * 16 + i) * 64 + lane];
            if constexpr (KH == 2) v += red[(((MT + m) * NB + c) * 16 + i) * 64 + lane];
            // the logit as the matmul would store it in the input dtype
            x[ii][c] = lr + 32 * c < E ? Elem<DT>::to_f32(Elem<DT>::from_f32(v)) : -__builtin_inff();
        }
    }
    // all rows valid: one interleaved pass over the RPW rows; otherwise (the
    // last, partly filled block: small batches) pairs of rows, skipping pairs
    // past T (a top-k pass costs ~1 us per 4 rows with one wave per SIMD)
    bool all = true;
#pragma unroll
    for (int ii = 0; ii < RPW; ++ii) all = all && valid[ii];
    if (__all(all)) {
        softmax_topk_rows<NB, 32, kF32, 32, RPW>(x, lr, lr, E, k, T, row, valid, wout, iout, eiout);
    } else {
#pragma unroll
        for (int h = 0; h < RPW; h += 2) {
            if (!__any(valid[h] || valid[h + 1])) continue;  // wave-uniform
            const float(&xh)[2][NB] = reinterpret_cast<const float(&)[2][NB]>(x[h]);
            const long long rh[2] = {row[h], row[h + 1]};
            const bool vh[2] = {valid[h], valid[h + 1]};
            softmax_topk_rows<NB, 32, kF32, 32, 2>(xh, lr, lr, E, k, T, rh, vh, wout, iout, eiout);
        }
    }
}

// Small batches (at most kRouterSplitTiles tiles of 32 tokens): K split over
// ks workgroups per tile (aiming at ~64 workgroups, at least 2 K tiles each,
// at most kRouterMaxSlots splits), one f32 partial per split in the caller's
// workspace (the split's waves each cover all of its K tiles), then the
// softmax / top-k summing them (two launches instead of one workgroup per
// tile streaming the whole router weight).
constexpr int kRouterSplitTiles = 8;
int router_splits(int T, int H, int E, int dtype) {
    if (dtype == kF32 || E <= 32 || E > 128) return 1;
    const long long tiles = ((long long)T + 31) / 32;
    if (tiles > kRouterSplitTiles) return 1;
    const int nk = (H + 63) / 64;
    int ks = (int)(64 / tiles);
    ks = std::min(ks, std::min(kRouterMaxSlots, nk / 2));
    return ks >= 2 ? ks : 1;
}
size_t router_ws_bytes(int T, int H, int E, int dtype) {
    const int ks = router_splits(T, H, E, dtype);
    return ks > 1 ? (size_t)ks * T * E * sizeof(float) : 0;
}

template <int DT, int NB>
static hipError_t launch_router_split(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                      int H, int E, int k, int ks, float* part, hipStream_t stream) {
    const long long grid = ((long long)T + 31) / 32 * ks;
    hipLaunchKernelGGL((router_mfma_kernel<DT, NB, 1, 6, 1, true>), dim3((unsigned)grid), dim3(64 * NB), 0, stream,
                       x, w, wo, io, eo, T, H, E, k, part, ks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int aligned = ((uintptr_t)part % 16) == 0;
    const unsigned g2 = (unsigned)cdivll((long long)T * 16, 256);
    if (E <= 64)
        hipLaunchKernelGGL((topk_partials_kernel<8, 8, DT>), dim3((unsigned)cdivll((long long)T * 8, 256)), dim3(256),
                           0, stream, part, ks, wo, io, eo, T, E, k, aligned);
    else
        hipLaunchKernelGGL((topk_partials_kernel<8, 16, DT>), dim3(g2), dim3(256), 0, stream, part, ks, wo, io, eo,
                           T, E, k, aligned);
    return hipGetLastError();
}

template <int DT, int NB>
static hipError_t launch_router_mfma(const void* x, const void* w, float* wo, uint32_t* io, uint32_t* eo, int T,
                                     int H, int E, int k, hipStream_t stream) {
    // 64 tokens per workgroup (each weight tile serves twice the rows) once
    // that still gives >= 256 workgroups, 3 stages (72 KB: two workgroups per
    // CU, 85 -> 63 us at T=32768, E=128 against 5 stages); else 32 tokens and
    // 6 stages (the one workgroup of a CU keeps more of the weight in flight)
    if ((long long)T >= 256LL * 64) {
        const long long grid = ((long long)T + 63) / 64;
        if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
        hipLaunchKernelGGL((router_mfma_kernel<DT, NB, 2, 3, 2>), dim3((unsigned)grid), dim3(128 * NB), 0, stream, x, w,
                           wo, io, eo, T, H, E, k);
    } else {
        const long long grid = ((long long)T + 31) / 32;
        hipLaunchKernelGGL((router_mfma_kernel<DT, NB, 1, 6, 2>), dim3((unsigned)grid), dim3(128 * NB), 0, stream, x, w,
                           wo, io, eo, T, H, E, k);
    }
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
    // 16-bit with more than 32 experts: the matrix-core kernel (several times
    // faster than the FMA kernel at E=128); up to 32 experts the FMA kernel
    // (at E=8 56 us against 72 us for the matrix-core kernel, whose weight
    // block is then three quarters padding)
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
                              int H, int E, int k, hipStream_t stream, float* part, size_t part_bytes) {
    if (T == 0) return hipSuccess;
    const int ks = router_splits(T, H, E, dtype);
    if (ks > 1 && part && part_bytes >= router_ws_bytes(T, H, E, dtype)) {
        if (dtype == kBF16)
            return E <= 64 ? launch_router_split<kBF16, 2>(x, w, wo, io, eo, T, H, E, k, ks, part, stream)
                           : launch_router_split<kBF16, 4>(x, w, wo, io, eo, T, H, E, k, ks, part, stream);
        return E <= 64 ? launch_router_split<kF16, 2>(x, w, wo, io, eo, T, H, E, k, ks, part, stream)
                       : launch_router_split<kF16, 4>(x, w, wo, io, eo, T, H, E, k, ks, part, stream);
    }
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

namespace cm {

// Test support (candle_moe_test_router_exp): the f32 exponential of the
// router's f32 softmax against the f64 one, for the n f32 values whose bit
// patterns are first, first + 1, ... (any sign and exponent): stats[0] =
// the largest distance in units in the last place (bit patterns of the two
// results as integers), stats[1] = how many inputs differ at all. Grid-stride
// loop; every lane evaluates both functions and the wave folds its results
// before one lane updates stats with vector atomics.
__global__ __launch_bounds__(256) void router_exp_check_k(uint32_t first, uint32_t n, uint32_t* stats) {
    uint32_t worst = 0, differ = 0;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float d = __uint_as_float(first + i);
        const uint32_t a = __float_as_uint(exp_f32_fast(d));
        const uint32_t b = __float_as_uint(exp_f32_f64(d));
        const uint32_t dist = a > b ? a - b : b - a;
        worst = dist > worst ? dist : worst;
        differ += dist != 0;
        if (i > 0xffffffffu - stride) break;  // (i + stride would wrap)
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t w2 = __shfl_xor(worst, off);
        worst = w2 > worst ? w2 : worst;
        differ += __shfl_xor(differ, off);
    }
    if ((threadIdx.x & 63) == 0) {
        atomicMax(stats, worst);
        atomicAdd(stats + 1, differ);
    }
}

hipError_t launch_router_exp_check(uint32_t first, uint32_t n, uint32_t* stats, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(router_exp_check_k, dim3(2048), dim3(256), 0, stream, first, n, stats);
    return hipGetLastError();
}

}  // namespace cm
