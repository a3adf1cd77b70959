// Decode GEMMs over 16-bit expert weights (API layout or pre-packed) or fp8
// codes (gfx950), with no grouping launch and no LDS staging of the weights.
//
// At decode sizes the work is the weight stream and the fixed latency around
// it. The 32-row tile kernel needs the grouping's tile table (a launch and
// three dependent loads before the first weight DMA), stages the weights
// through LDS and meets in a split-K fixup. Here:
//  * every workgroup groups the (few) pairs itself: it loads the expert ids
//    into LDS, marks the touched experts in a bitmap, counts them (U) and
//    takes its item: the u-th touched expert, a block of 16 * CPL output
//    columns and one of ks K slices (ks from U, up to a host bound; 1 for
//    most GEMMs), then that expert's pairs, ascending; workgroups past the
//    items exit. Two workgroups share a CU (at most 256 registers a lane),
//    so the grid is one round of two per CU;
//  * its 4 waves split the slice (gate/up: two waves per tensor, two K
//    halves each; otherwise four K parts) over its column block; each lane
//    loads its weight chunks straight into registers, a ring of K steps in
//    flight (32 k wide; 64 on Nomic's fc2, 128 on fp8 codes), and meets the
//    other waves once, at the end, where the parts are summed through LDS in
//    a fixed order;
//  * v_mfma_f32_16x16x32: A = the expert's rows (x rows gathered by pair, or
//    intermediate rows by pair; 16 per row block), B = weight columns.
//    [K,N] weights (gate / up / fc1 / down): lane (g, i) (g = lane / 16,
//    i = lane % 16) loads k-rows k0 + 8g .. +7 of columns c_i .. c_i + CPL-1
//    (8 loads of 2*CPL bytes) and transposes that 8 x CPL block of 16-bit
//    values with v_perm into CPL MFMA operands: operand j holds the 8 k of
//    column c_i + j, so MFMA j computes columns {c_i + j}. [N,K] weights
//    (Nomic fc2, pre-packed, fp8): one 16-byte load is the operand of column
//    n, 8 k (fp8: 16 k, two operands); a lane loads one such chunk per
//    column and step (pre-packed gate/up, fc1, down: k0 + 8g .. +7, the k of
//    the API layout's MFMAs) or two adjacent ones (fc2, fp8: 128 contiguous
//    bytes of the column per lane group step). The A operand of lane (g, r)
//    holds row r at the same k.
// Workgroup outputs go through LDS: each wave stores its f32 part of the
// block, then every thread sums the parts of 8 consecutive columns of one
// row and stores them:
//  gate/up, fc1, ks == 1 : inter[p] = dtype(act(x_t . G) (* x_t . U))  (p = t*k + j)
//  gate/up, fc1, ks > 1  : f32 partial sums of slice s, by pair
//  down, fc2             : f32 partial sums by pair (unweighted)
// and a finishing launch (dec_finish_k) sums the partials in slice order:
// the activation for gate/up / fc1, out[t] = dtype(sum_j w_{t,j} * ...) over
// a token's k pairs in slot order for down / fc2. No workgroup reads what
// another writes: the kernel boundaries order the launches.
#include "cm_lds.hpp"

namespace cm {

using namespace lds;

namespace {

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
    if constexpr (DT == kBF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
}

constexpr int kDvWaves = 4;  // waves per workgroup
constexpr int kDvStep = 32;  // K per step (one MFMA deep)
// steps in flight per wave: 4, or 2 for 6 or 8 columns per lane, so that a
// wave stays within 256 registers and two workgroups share a CU; halved where
// each column takes WCH = 2 chunks of 16 bytes per step (the same bytes in
// flight)
template <int CPL, int WCH = 1>
constexpr int dec_ring() { return (CPL >= 6 ? 2 : 4) / WCH; }

// Operand j of a transposed 8 x CPL block: r[t] holds k-row t of CPL
// consecutive columns (pairs of 16-bit values, low half first); the result
// holds column j at k-rows 0..7 (pairs (2q, 2q+1), low half first).
template <int CPL>
__device__ __forceinline__ u32x4 column_operand(const uint32_t (&r)[8][CPL / 2], int j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __builtin_amdgcn_perm(r[2 * q + 1][j >> 1], r[2 * q][j >> 1], sel);
    return o;
}

// The touched-expert bitmap (LDS; the expert ids are kept in s_idx, -1:
// dropped) and this workgroup's item. With U touched experts and nblk column
// blocks, K is split into ks = min(cap / (U * nblk), ks_lim) slices (at least
// 1), so that the U * nblk * ks items fill one round of cap workgroups;
// workgroup w takes item w: the u-th touched expert (u = w / (nblk * ks)), a
// column block and a slice. [K,N] weights: the column blocks vary fastest,
// so that workgroups running side by side read neighbouring runs of the same
// k-rows; [N,K]: the slices, for neighbouring K runs of the same columns.
// s_misc[0..3] = expert (-1: no item), column block, slice, ks. Workgroup 0
// also stores ks to meta[slot] for the finishing launch.
template <int NT, bool TRANS>
__device__ __forceinline__ void dec_assign(const DecArgs& a, int slot, uint32_t* s_bm, int32_t* s_idx,
                                           int* s_misc) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwords = (a.E + 31) >> 5;
    for (int w = tid; w < nwords; w += NT) s_bm[w] = 0u;
    __syncthreads();
    for (int p = tid; p < a.P; p += NT) {
        const uint32_t e = a.idx[p];
        const bool ok = e < (uint32_t)a.E;
        s_idx[p] = ok ? (int)e : -1;
        if (ok) atomicOr(&s_bm[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    // wave 0: touched experts U, the slices, the item and its expert (the
    // u-th set bit; each lane two words: E <= 4096)
    if (wave == 0) {
        const uint32_t w0 = 2 * lane < nwords ? s_bm[2 * lane] : 0u;
        const uint32_t w1 = 2 * lane + 1 < nwords ? s_bm[2 * lane + 1] : 0u;
        const int c = __popc(w0) + __popc(w1);
        int incl = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off);
            if (lane >= off) incl += v;
        }
        const int excl = incl - c;
        const int U = __shfl(incl, 63);
        const long long un = (long long)U * a.nblk;
        const int ks = un > 0 ? (int)max(1LL, min((long long)a.cap / un, (long long)a.ks_lim)) : 1;
        const long long w = blockIdx.x;
        const int per_u = a.nblk * ks;
        const int u = (int)(w / per_u);
        const int r_u = (int)(w - (long long)u * per_u);
        const int sl = TRANS ? r_u / a.nblk : r_u % ks;
        const int cb = TRANS ? r_u - sl * a.nblk : r_u / ks;
        if (lane == 0) {
            s_misc[0] = -1;
            s_misc[1] = cb;
            s_misc[2] = sl;
            s_misc[3] = ks;
            if (blockIdx.x == 0) a.meta[slot] = ks;
        }
        __builtin_amdgcn_wave_barrier();
        if (u < U && u >= excl && u < incl) {
            int need = u - excl;  // set bits to skip in this lane's words
            uint32_t wd = w0;
            int base = 64 * lane;
            if (need >= __popc(w0)) {
                need -= __popc(w0);
                wd = w1;
                base += 32;
            }
            for (int q = 0; q < need; ++q) wd &= wd - 1u;  // drop the lowest set bits
            s_misc[0] = base + __builtin_ctz(wd);
        }
    }
    __syncthreads();
}

// Expert e's pairs, ascending (a stable compaction of s_idx over NT-pair
// chunks), into s_rows; returns their number.
template <int NT>
__device__ __forceinline__ int dec_rows(const DecArgs& a, int e, const int32_t* s_idx, int32_t* s_rows,
                                        int* s_misc) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int run = 0;
    for (int p0 = 0; p0 < a.P; p0 += NT) {
        const int p = p0 + tid;
        const bool hit = p < a.P && s_idx[p] == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) s_misc[8 + wave] = __popcll(m);
        __syncthreads();
        int before = run;
        for (int w = 0; w < wave; ++w) before += s_misc[8 + w];
        int total = run;
        for (int w = 0; w < NT / 64; ++w) total += s_misc[8 + w];
        if (hit) s_rows[before + __popcll(m & ((1ull << lane) - 1ull))] = p;
        run = total;
        __syncthreads();
    }
    return run;
}

// Finishing the K slices (fixed slice and slot order). Up to KSM slices and
// KM slots are unrolled with their loads all in flight, issued before the
// slice count is known (runtime-bounded loops, or addresses depending on it,
// waited for each load in turn): slices at or past ks_lim re-read the last
// one, and the slices past ks, the slots past k and the dropped pairs are
// selected away (their partials were never written).
template <int KSM>
__device__ __forceinline__ f32x4 slice_sum(const float* src, long long stride, int ks, int ks_lim) {
    f32x4 v[KSM];
#pragma unroll
    for (int sl = 0; sl < KSM; ++sl)
        v[sl] = *reinterpret_cast<const f32x4*>(src + (long long)min(sl, ks_lim - 1) * stride);
    f32x4 y = v[0];
#pragma unroll
    for (int sl = 1; sl < KSM; ++sl)
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = sl < ks ? y[j] + v[sl][j] : y[j];
    return y;
}

// gate/up, fc1: columns c .. c + 3 of pair row p (nothing for a dropped pair)
template <int DT, bool DUAL, bool W8, int KSM>
__device__ __forceinline__ void finish_pair4(const DecFinish& f, int ks, long long p, int c) {
    const long long NC = (long long)(DUAL ? 2 : 1) * f.N;
    const long long stride = (long long)f.P * NC;
    const uint32_t e = f.idx[p];
    const f32x4 g = slice_sum<KSM>(f.part + p * NC + c, stride, ks, f.ks_lim);
    f32x4 u = {0.f, 0.f, 0.f, 0.f};
    if constexpr (DUAL) u = slice_sum<KSM>(f.part + p * NC + f.N + c, stride, ks, f.ks_lim);
    if (e >= (uint32_t)f.E) return;  // dropped pair: no row
    float h[4];
    with_act(f.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float s0 = W8 ? f.scale0[(long long)e * f.N + c + j] : 1.0f;
            if constexpr (DUAL) {
                const float s1 = W8 ? f.scale1[(long long)e * f.N + c + j] : 1.0f;
                h[j] = act_t<ACT>(s0 * g[j]) * (s1 * u[j]);
            } else {
                h[j] = act_t<ACT>(s0 * g[j]);
            }
        }
    });
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(f.out) + p * f.N + c) =
        u32x2{pack2<DT>(h[0], h[1]), pack2<DT>(h[2], h[3])};
}

// down, fc2: columns c .. c + 3 of token row t
template <int DT, bool W8, int KSM, int KM>
__device__ __forceinline__ void finish_token4(const DecFinish& f, int ks, long long t, int c) {
    const long long stride = (long long)f.P * f.N;
    uint16_t* orow = reinterpret_cast<uint16_t*>(f.out) + t * f.N + c;
    const bool al8 = (reinterpret_cast<uintptr_t>(f.out) & 7u) == 0;  // else 2-byte accesses
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (!f.overwrite) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = Elem<DT>::to_f32(orow[j]);
    }
    // slots in groups of KM (k <= KM: one group)
    for (int j0 = 0; j0 < f.k_top; j0 += KM) {
        uint32_t ej[KM];
        float wj[KM];
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            const long long p = t * f.k_top + min(j0 + j, f.k_top - 1);
            ej[j] = f.idx[p];
            wj[j] = f.routing_w[p];
        }
        f32x4 yj[KM];
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            const long long p = t * f.k_top + min(j0 + j, f.k_top - 1);
            yj[j] = slice_sum<KSM>(f.part + p * f.N + c, stride, ks, f.ks_lim);
        }
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            const bool ok = j0 + j < f.k_top && ej[j] < (uint32_t)f.E;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float s0 = W8 ? f.scale0[(long long)(ok ? ej[j] : 0u) * f.N + c + q] : 1.0f;
                acc[q] = ok ? acc[q] + wj[j] * (s0 * yj[j][q]) : acc[q];
            }
        }
    }
    const u32x2 o = {pack2<DT>(acc[0], acc[1]), pack2<DT>(acc[2], acc[3])};
    if (al8) {
        *reinterpret_cast<u32x2*>(orow) = o;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) orow[j] = (uint16_t)((o[j >> 1] >> (16 * (j & 1))) & 0xffffu);
    }
}

template <int DT, int MODE, int RB, int CPL, bool PK, bool W8>
__global__ __launch_bounds__(64 * kDvWaves, 2) void moe_dec_gemv(DecArgs a) {
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    // [K,N] weights (the API layout but Nomic's fc2); [N,K]: fc2, every GEMM
    // on pre-packed weights (PK) and on fp8 codes (W8)
    constexpr bool TRANS = (MODE != kFc2Rows) && !PK && !W8;
    // W8: OCP fp8 e4m3 codes [E][N][K] (one byte per weight) with per-column
    // f32 scales. A step is 128 k: a lane's two 16-byte loads hold
    // k0 + 32g .. +31 of its column, the operands of four MFMAs (converted
    // exactly to DT), and the A operand holds the same k of its row in four
    // 16-byte loads.
    // fp8 codes and Nomic's fc2 ([N,K] weights): each lane reads WCH = 2
    // adjacent 16-byte chunks of its column per step, so that the 4 lane
    // groups cover 128 contiguous bytes of every column instead of 64
    // (Qwen3 T=16 fp8 gate/up 27.6 -> 25.7 us, down 18.0 -> 16.2 us; Nomic
    // T=16 bf16 fc2 15.4 -> 13.9 us). The other pre-packed GEMMs keep one
    // chunk: the same k per MFMA as on the API layout, hence the same sums
    // bit for bit.
    constexpr int WCH = (W8 || MODE == kFc2Rows) ? 2 : 1;
    constexpr int KSTEP = (W8 ? 64 : kDvStep) * WCH;
    constexpr int KG = (W8 ? 16 : 8) * WCH;  // k per lane group per step
    constexpr int KC = W8 ? 16 : 8;         // k per 16-byte weight chunk
    constexpr int WB = W8 ? 1 : 2;          // bytes per weight
    constexpr int AH = (W8 ? 2 : 1) * WCH;   // 16-byte A loads per row and step
    constexpr bool ROWS = (MODE == kDownRows || MODE == kFc2Rows);
    constexpr int NT = 64 * kDvWaves;
    constexpr int WGC = 16 * CPL;                // output columns per workgroup
    constexpr int NPART = kDvWaves;              // f32 parts in LDS (gate/up: 2 gate, 2 up)
    constexpr int KP = DUAL ? kDvWaves / 2 : kDvWaves;  // K parts per tensor
    constexpr int NB = TRANS ? CPL : WGC / 16;   // MFMA column blocks per step (operands)
    constexpr int NLD = TRANS ? 8 : NB * WCH;     // weight loads per lane per step
    // (3 and 6 only for [N,K] weights, whose operands are 16 independent
    // columns: blocks of 48 or 96 columns)
    static_assert(CPL == 2 || CPL == 4 || CPL == 8 || (!TRANS && (CPL == 3 || CPL == 6)), "columns per lane");
    static_assert(!TRANS || NB == CPL, "operands");

    __shared__ uint32_t s_bm[kDecMaxE / 32];
    __shared__ int32_t s_idx[kDecMaxPairs];
    __shared__ int32_t s_rows[kDecMaxPairs];
    __shared__ int s_misc[8 + kDvWaves];
    // (rows padded by 4 floats: the 4 row groups of a wave's store land in
    // different banks)
    constexpr int SPW = WGC + 4;
    __shared__ __attribute__((aligned(16))) float s_part[NPART][RB * 16][SPW];
    // fp8 down / fc2, unsliced: the block's column scales for the partials
    constexpr bool SCALED = W8 && ROWS;
    __shared__ float s_sc[SCALED ? WGC : 1];

    dec_assign<NT, TRANS>(a, ROWS ? 1 : 0, s_bm, s_idx, s_misc);
    const int e = s_misc[0];
    if (e < 0) return;
    const int cb = s_misc[1], sl = s_misc[2], ks = s_misc[3];
    // f32 partials (down / fc2 always; gate/up / fc1 with K slices), else
    // the finished rows in the dtype
    const bool part_out = ROWS || ks > 1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int tensor = DUAL ? wave / KP : 0;
    const int kpart = DUAL ? wave - tensor * KP : wave;
    const int K = a.K, N = a.N;
    const int col0 = cb * WGC;

    // weights of expert e (this wave's tensor): in-range loads only, zeros past
    const char* wbase = reinterpret_cast<const char*>(tensor ? a.B1 : a.B0) + (long long)e * a.strideB * WB;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wbase), 0, (int)(a.strideB * WB), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.A), 0, (int)a.a_bytes, 0x00020000);

    // this wave's steps: part kpart of slice sl, [s_lo, s_hi), run as a
    // whole number of ring rounds (the steps past s_hi load zeros), so that
    // the ring loop needs no guard. The parts depend on K, the slices and the
    // waves only (not on the ring or the column block).
    constexpr int RING = dec_ring<CPL, WCH>();
    const int nks = (K + KSTEP - 1) / KSTEP;
    const int nparts = KP * ks;
    const int per = (nks + nparts - 1) / nparts;
    const int s_lo = (sl * KP + kpart) * per;
    const int s_hi = min(s_lo + per, nks);
    const int trips = (per + RING - 1) / RING * RING;

    // per-lane column(s): [K,N]: columns col0 + CPL*li .. +CPL-1 of every
    // k-row; [N,K]: column col0 + 16*b + li of block b
    int ncol[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ncol[b] = TRANS ? col0 + CPL * li + b : col0 + 16 * b + li;

    // per-lane weight offsets, fixed: [K,N]: k-row 8g, columns ncol[0] ..;
    // [N,K]: column ncol[b], k KG*g. A lane whose columns lie past N starts at
    // kOob. (Every offset stays below 2^32: kOob plus less than the expert's
    // 2^31 bytes.)
    const uint32_t ldb2 = (uint32_t)a.ldb * (uint32_t)WB;  // bytes per weight row
    uint32_t wlane[TRANS ? 1 : NB];
#pragma unroll
    for (int b = 0; b < (TRANS ? 1 : NB); ++b)
        wlane[b] = ncol[b] < N ? (TRANS ? 8u * (uint32_t)g * ldb2 + 2u * (uint32_t)ncol[0]
                                        : (uint32_t)ncol[b] * ldb2 + (uint32_t)(KG * WB) * (uint32_t)g)
                               : kOob;

    // ring of steps: weight chunks (CPL 16-bit values each for [K,N], 8 for
    // [N,K]) and the A rows. Branch-free offsets (a branch, or a select on
    // the step alone, made the compiler wait for every load in flight): a
    // lane's k positions past K read zeros (kOob).
    constexpr int WDW = TRANS ? CPL / 2 : 4;  // dwords per weight load
    uint32_t wv[RING][NLD][WDW];
    u32x4 xv[RING][RB][AH];
    // this lane's k of step s, chunk c, inside the wave's part and K (K is a
    // multiple of KC: a chunk lies wholly inside or outside). Bitwise, not
    // short-circuit: a branch on the uniform s < s_hi made the compiler wait
    // for every load in flight at it.
    auto k_ok = [&](int s, int c) {
        return (s < s_hi) & (s * KSTEP + KG * g + KC * c < K);
    };
    auto load_w = [&](int i, int st) {
        const int s = s_lo + st;
#pragma unroll
        for (int t = 0; t < NLD; ++t) {
            const int c = TRANS ? 0 : t % WCH;
            const bool kok = k_ok(s, c);
            uint32_t o;
            if constexpr (TRANS) o = kok ? wlane[0] + (uint32_t)(s * KSTEP + t) * ldb2 : kOob;
            else o = kok ? wlane[t / WCH] + (uint32_t)(s * KSTEP * WB + 16 * c) : kOob;
            if constexpr (WDW == 4) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0);
#pragma unroll
                for (int d = 0; d < 4; ++d) wv[i][t][d] = v[d];
            } else if constexpr (WDW == 2) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, 0);
                wv[i][t][0] = v[0];
                wv[i][t][1] = v[1];
            } else {
                wv[i][t][0] = __builtin_amdgcn_raw_buffer_load_b32(rw, o, 0, 0);
            }
        }
    };
    // the first ring of weight steps goes out before the expert's rows are
    // gathered (it depends on the expert only)
#pragma unroll
    for (int i = 0; i < RING; ++i) load_w(i, i);
    // (read into a register now, stored to LDS after the K loop: a store
    // here would wait for the weight loads issued before it)
    float sc_reg = 0.0f;
    if constexpr (SCALED) {
        if (a.scale0 != nullptr && tid < WGC && col0 + tid < N) sc_reg = a.scale0[(long long)e * N + col0 + tid];
    }
    const int cnt = dec_rows<NT>(a, e, s_idx, s_rows, s_misc);


    for (int c0 = 0; c0 < cnt; c0 += RB * 16) {
        const int m_valid = min(RB * 16, cnt - c0);
        // A rows of this lane (row li of each row block), k 8g
        uint32_t abase[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int m = rb * 16 + li;
            const int p = s_rows[c0 + min(m, m_valid - 1)];
            const int src = GATHER ? p / a.k_top : p;
            abase[rb] = m < m_valid ? ((uint32_t)src * (uint32_t)K + (uint32_t)(KG * g)) * 2u : kOob;
        }
        f32x4 acc[RB][NB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[rb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto load_a = [&](int i, int st) {
            const int s = s_lo + st;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int h = 0; h < AH; ++h) {
                    // load h holds the k of weight chunk h / (AH / WCH)
                    const bool kok = k_ok(s, h / (AH / WCH));
                    xv[i][rb][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        rx, kok ? abase[rb] + (uint32_t)(s * KSTEP) * 2u + 16u * h : kOob, 0, 0);
                }
        };
        auto load = [&](int i, int st) {
            load_w(i, st);
            load_a(i, st);
        };
        auto compute = [&](int i) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if constexpr (W8) {
                    // chunk c: codes k0 + KG g + 16c .. +7 and .. +15 of
                    // column b, two operands; A loads 2c and 2c + 1 hold the
                    // same k of the row
#pragma unroll
                    for (int c = 0; c < WCH; ++c) {
                        const uint32_t(&w)[WDW] = wv[i][b * WCH + c];
                        const u32x4 wl = fp8x8_to<DT>(u32x2{w[0], w[1]});  // exact in DT
                        const u32x4 wh = fp8x8_to<DT>(u32x2{w[2], w[3]});
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) {
                            acc[rb][b] = mfma16<DT>(xv[i][rb][2 * c], wl, acc[rb][b]);
                            acc[rb][b] = mfma16<DT>(xv[i][rb][2 * c + 1], wh, acc[rb][b]);
                        }
                    }
                } else if constexpr (!TRANS) {
                    // chunk c: k0 + KG g + 8c .. +7 of column b, A load c
#pragma unroll
                    for (int c = 0; c < WCH; ++c) {
                        const uint32_t(&w)[WDW] = wv[i][b * WCH + c];
                        const u32x4 bop = u32x4{w[0], w[1], w[2], w[3]};
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) acc[rb][b] = mfma16<DT>(xv[i][rb][c], bop, acc[rb][b]);
                    }
                } else {
                    uint32_t r[8][CPL / 2];
#pragma unroll
                    for (int t = 0; t < 8; ++t)
#pragma unroll
                        for (int d = 0; d < CPL / 2; ++d) r[t][d] = wv[i][t][d];
                    const u32x4 bop = column_operand<CPL>(r, b);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) acc[rb][b] = mfma16<DT>(xv[i][rb][0], bop, acc[rb][b]);
                }
            }
        };
        // trips is a positive multiple of RING. The first ring round is
        // peeled: its loads went out in another order (the weights first,
        // before the rows were known), and inside the loop the compiler would
        // keep that round's shorter waits for every round. The last round
        // loads nothing; a further row chunk streams the weights again.
        if (c0 > 0) {
#pragma unroll
            for (int i = 0; i < RING; ++i) load_w(i, i);
        }
#pragma unroll
        for (int i = 0; i < RING; ++i) load_a(i, i);
        // (sched_barrier: the scheduler would otherwise hoist the MFMAs of
        // later slots above this slot's refill, waiting for data that should
        // still be in flight)
        if (trips > RING) {
#pragma unroll
            for (int i = 0; i < RING; ++i) {
                compute(i);
                __builtin_amdgcn_sched_barrier(0);
                load(i, i + RING);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int st = RING; st + RING < trips; st += RING) {
#pragma unroll
                for (int i = 0; i < RING; ++i) {
                    compute(i);
                    __builtin_amdgcn_sched_barrier(0);
                    load(i, st + i + RING);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RING; ++i) compute(i);

        // parts to LDS: lane (g, li) holds rows 4g .. 4g+3 of each row block
        // at local column CPL*li + b ([K,N]: CPL consecutive columns, stored
        // 4 at a time) or 16b + li ([N,K])
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float* row = &s_part[wave][rb * 16 + 4 * g + v][0];
                if constexpr (TRANS && CPL >= 4) {
#pragma unroll
                    for (int b = 0; b < CPL; b += 4)
                        *reinterpret_cast<f32x4*>(row + CPL * li + b) =
                            f32x4{acc[rb][b][v], acc[rb][b + 1][v], acc[rb][b + 2][v], acc[rb][b + 3][v]};
                } else {
#pragma unroll
                    for (int b = 0; b < NB; ++b) row[TRANS ? CPL * li + b : 16 * b + li] = acc[rb][b][v];
                }
            }
        if constexpr (SCALED) {
            if (tid < WGC) s_sc[tid] = sc_reg;
        }
        __syncthreads();

        // every thread: 8 consecutive output columns of one row; the parts
        // summed in a fixed order (gate/up: gate = parts 0 .. KP - 1, up =
        // parts KP .. 2 KP - 1)
        constexpr int CH = WGC / 8;
        // the K parts of tensor tn (0: gate / single, 1: up), columns c8 ..
        // c8 + 7 of row m, in wave order
        auto part_sums = [&](int m, int c8, int tn, float (&y)[8]) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                f32x4 v = *reinterpret_cast<const f32x4*>(&s_part[tn * KP][m][c8 + 4 * half]);
#pragma unroll
                for (int pt = 1; pt < KP; ++pt) {
                    const f32x4 w = *reinterpret_cast<const f32x4*>(&s_part[tn * KP + pt][m][c8 + 4 * half]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] += w[j];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) y[4 * half + j] = v[j];
            }
        };
        if (part_out) {
            // f32 partials of slice sl: part[(sl * P + p) * NC + col]
            constexpr int NT2 = DUAL ? 2 : 1;
            const long long NC = (long long)NT2 * N;
            for (int q = tid; q < m_valid * CH; q += NT) {
                const int m = q / CH, c8 = (q - m * CH) * 8;
                const int col = col0 + c8;
                if (col >= N) continue;
                const int p = s_rows[c0 + m];
#pragma unroll
                for (int tn = 0; tn < NT2; ++tn) {
                    float y[8];
                    part_sums(m, c8, tn, y);
                    // fp8 down / fc2 unsliced: the column scales here (the
                    // finishing launch's product s * y, the same f32 value),
                    // so that it reads no scales
                    if constexpr (SCALED) {
                        if (a.scale0 != nullptr) {
#pragma unroll
                            for (int j = 0; j < 8; ++j) y[j] *= s_sc[c8 + j];
                        }
                    }
                    float* dst = a.part + ((long long)sl * a.P + p) * NC + (long long)tn * N + col;
                    if (col + 8 <= N) {
                        *reinterpret_cast<f32x4*>(dst) = f32x4{y[0], y[1], y[2], y[3]};
                        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{y[4], y[5], y[6], y[7]};
                    } else {
                        for (int j = 0; j < 8 && col + j < N; ++j) dst[j] = y[j];
                    }
                }
            }
        } else {
            auto epilogue = [&](auto act_c) {
                constexpr int ACT = decltype(act_c)::value;
                for (int q = tid; q < m_valid * CH; q += NT) {
                    const int m = q / CH, c8 = (q - m * CH) * 8;
                    const int col = col0 + c8;
                    if (col >= N) continue;
                    const int p = s_rows[c0 + m];
                    float y0[8], y1[8], h[8];
                    part_sums(m, c8, 0, y0);
                    if constexpr (DUAL) part_sums(m, c8, 1, y1);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        // (fp8 weights: the column scales on the f32 sums first)
                        const int cc = col + j;
                        const float s0 = W8 ? (cc < N ? a.scale0[(long long)e * N + cc] : 0.0f) : 1.0f;
                        if constexpr (DUAL) {
                            const float s1 = W8 ? (cc < N ? a.scale1[(long long)e * N + cc] : 0.0f) : 1.0f;
                            h[j] = act_t<ACT>(s0 * y0[j]) * (s1 * y1[j]);
                        } else {
                            h[j] = act_t<ACT>(s0 * y0[j]);
                        }
                    }
                    u32x4 o;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[j] = pack2<DT>(h[2 * j], h[2 * j + 1]);
                    uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)p * N + col;
                    if (col + 8 <= N) {
                        *reinterpret_cast<u32x4*>(C) = o;
                    } else {
                        for (int j = 0; j < 8 && col + j < N; ++j)
                            C[j] = (uint16_t)((o[j >> 1] >> (16 * (j & 1))) & 0xffffu);
                    }
                }
            };
            with_act(a.act, epilogue);
        }
        __syncthreads();  // the parts are read before the next row chunk writes them
    }
}

// The finishing launch: one thread per 4 consecutive columns of a pair
// (gate/up, fc1) or token (down, fc2) row, in workgroups of 64 threads (a
// decode batch's rows spread over many CUs). KSM: slices unrolled (>= ks_lim).
template <int DT, int MODE, bool W8, int KSM, int KM>
__global__ __launch_bounds__(64) void dec_finish_k(DecFinish f) {
    constexpr bool ROWS = (MODE == kDownRows || MODE == kFc2Rows);
    const int n4 = f.N / 4;
    const long long i = (long long)blockIdx.x * 64 + threadIdx.x;
    if (i >= (ROWS ? f.T : f.P) * (long long)n4) return;
    const long long row = i / n4;
    const int c = (int)(i - row * n4) * 4;
    const int ks = min(f.meta[ROWS ? 1 : 0], f.ks_lim);
    if constexpr (ROWS) {
        finish_token4<DT, W8, KSM, KM>(f, ks, row, c);
    } else {
        if (ks <= 1) return;  // the GEMM wrote the rows
        finish_pair4<DT, MODE == kGateUp, W8, KSM>(f, ks, row, c);
    }
}

template <int DT, int MODE, int RB, int CPL>
hipError_t launch_cfg(const DecArgs& a, hipStream_t stream) {
    const long long nwg = std::max<long long>(a.cap, (long long)a.max_groups * a.nblk);
    if (nwg > 0x7fffffffLL) return hipErrorInvalidValue;
    if (a.max_groups <= 0) return hipSuccess;
    const dim3 grid((int)nwg), block(64 * kDvWaves);
    if (a.w8) {
        // fp8 codes are [N,K] for every GEMM (Nomic's fc2 runs the down mode)
        constexpr int M8 = MODE == kFc2Rows ? kDownRows : MODE;
        hipLaunchKernelGGL((moe_dec_gemv<DT, M8, RB, CPL, false, true>), grid, block, 0, stream, a);
        return hipGetLastError();
    }
    // (Nomic's fc2 is [N,K] either way: no packed instance)
    if constexpr (MODE != kFc2Rows) {
        if (a.packed) {
            hipLaunchKernelGGL((moe_dec_gemv<DT, MODE, RB, CPL, true, false>), grid, block, 0, stream, a);
            return hipGetLastError();
        }
    }
    if constexpr (MODE == kFc2Rows || (CPL != 3 && CPL != 6)) {
        hipLaunchKernelGGL((moe_dec_gemv<DT, MODE, RB, CPL, false, false>), grid, block, 0, stream, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;  // [K,N] weights: 2, 4 or 8 columns per lane
}

template <int DT, int MODE>
hipError_t launch_mode(const DecArgs& a, hipStream_t stream) {
    const bool rb2 = a.rows_max > 16;
    if (a.cpl == 2) return rb2 ? launch_cfg<DT, MODE, 2, 2>(a, stream) : launch_cfg<DT, MODE, 1, 2>(a, stream);
    if (a.cpl == 3) return rb2 ? launch_cfg<DT, MODE, 2, 3>(a, stream) : launch_cfg<DT, MODE, 1, 3>(a, stream);
    if (a.cpl == 6) return rb2 ? launch_cfg<DT, MODE, 2, 6>(a, stream) : launch_cfg<DT, MODE, 1, 6>(a, stream);
    if (a.cpl == 4) return rb2 ? launch_cfg<DT, MODE, 2, 4>(a, stream) : launch_cfg<DT, MODE, 1, 4>(a, stream);
    return rb2 ? launch_cfg<DT, MODE, 2, 8>(a, stream) : launch_cfg<DT, MODE, 1, 8>(a, stream);
}

template <int DT>
hipError_t launch_dt(int mode, const DecArgs& a, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return launch_mode<DT, kGateUp>(a, stream);
        case kFc1: return launch_mode<DT, kFc1>(a, stream);
        case kDownRows: return launch_mode<DT, kDownRows>(a, stream);
        case kFc2Rows: return launch_mode<DT, kFc2Rows>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_dec_gemv(int mode, int dtype, const DecArgs& a, hipStream_t stream) {
    if (a.cpl != 2 && a.cpl != 3 && a.cpl != 4 && a.cpl != 6 && a.cpl != 8) return hipErrorInvalidValue;
    if (a.P > kDecMaxPairs || a.E > kDecMaxE || a.ks_lim < 1 || a.ks_lim > kDecMaxSlices || a.cap < 1)
        return hipErrorInvalidValue;
    const bool rows = mode == kDownRows || mode == kFc2Rows;
    if (a.meta == nullptr || ((rows || a.ks_lim > 1) && a.part == nullptr) || (!rows && a.C == nullptr))
        return hipErrorInvalidValue;
    if (dtype == kBF16) return launch_dt<kBF16>(mode, a, stream);
    if (dtype == kF16) return launch_dt<kF16>(mode, a, stream);
    return hipErrorInvalidValue;
}

namespace {
template <int DT, int MODE, bool W8, int KSM>
hipError_t finish_ks(const DecFinish& f, const dim3& grid, hipStream_t stream) {
    if constexpr (MODE == kDownRows || MODE == kFc2Rows) {
        // slots per group: at most 32 / KSM (32 partial loads in flight)
        constexpr int K4 = KSM <= 8 ? 4 : 2, K8 = KSM <= 4 ? 8 : K4;
        if (f.k_top <= 2) hipLaunchKernelGGL((dec_finish_k<DT, MODE, W8, KSM, 2>), grid, dim3(64), 0, stream, f);
        else if (f.k_top <= 4) hipLaunchKernelGGL((dec_finish_k<DT, MODE, W8, KSM, K4>), grid, dim3(64), 0, stream, f);
        else hipLaunchKernelGGL((dec_finish_k<DT, MODE, W8, KSM, K8>), grid, dim3(64), 0, stream, f);
    } else {
        hipLaunchKernelGGL((dec_finish_k<DT, MODE, W8, KSM, 1>), grid, dim3(64), 0, stream, f);
    }
    return hipGetLastError();
}
template <int DT, int MODE, bool W8>
hipError_t finish_w8(const DecFinish& f, const dim3& grid, hipStream_t stream) {
    if (f.ks_lim <= 1) return finish_ks<DT, MODE, W8, 1>(f, grid, stream);
    if (f.ks_lim <= 2) return finish_ks<DT, MODE, W8, 2>(f, grid, stream);
    if (f.ks_lim <= 4) return finish_ks<DT, MODE, W8, 4>(f, grid, stream);
    if (f.ks_lim <= 8) return finish_ks<DT, MODE, W8, 8>(f, grid, stream);
    return finish_ks<DT, MODE, W8, 16>(f, grid, stream);
}
template <int DT, int MODE>
hipError_t finish_mode(const DecFinish& f, hipStream_t stream) {
    const long long rows = (MODE == kDownRows || MODE == kFc2Rows) ? f.T : f.P;
    const long long n = rows * (f.N / 4);
    if (n <= 0) return hipSuccess;
    if ((n + 63) / 64 > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + 63) / 64));
    return f.scale0 != nullptr ? finish_w8<DT, MODE, true>(f, grid, stream) : finish_w8<DT, MODE, false>(f, grid, stream);
}
template <int DT>
hipError_t finish_dt(int mode, const DecFinish& f, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return finish_mode<DT, kGateUp>(f, stream);
        case kFc1: return finish_mode<DT, kFc1>(f, stream);
        case kDownRows: return finish_mode<DT, kDownRows>(f, stream);
        case kFc2Rows: return finish_mode<DT, kFc2Rows>(f, stream);
        default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t launch_dec_finish(int mode, int dtype, const DecFinish& f, hipStream_t stream) {
    if (f.N % 8 != 0 || f.meta == nullptr || f.ks_lim < 1 || f.ks_lim > kDecMaxSlices ||
        (mode == kGateUp && f.scale0 != nullptr && f.scale1 == nullptr))
        return hipErrorInvalidValue;
    if (dtype == kBF16) return finish_dt<kBF16>(mode, f, stream);
    if (dtype == kF16) return finish_dt<kF16>(mode, f, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
