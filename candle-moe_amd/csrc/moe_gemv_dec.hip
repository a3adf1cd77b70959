// Decode GEMMs over 16-bit expert weights in the API layout (gfx950), with
// no grouping launch, no LDS staging of the weights and no K splits across
// workgroups.
//
// At decode sizes the work is the weight stream and the fixed latency around
// it. The 32-row tile kernel needs the grouping's tile table (a launch and
// three dependent loads before the first weight DMA), stages the weights
// through LDS and meets in a split-K fixup. Here:
//  * every workgroup groups the (few) pairs itself: it loads the expert ids
//    into LDS, marks the touched experts in a bitmap and takes the u-th
//    touched expert (u = its index / column blocks) and that expert's pairs,
//    ascending; workgroups past the touched experts exit;
//  * its 4 waves split K (gate/up: two waves per tensor, two K halves each;
//    otherwise four K quarters) over one block of 16 * CPL output columns;
//    each lane loads its weight chunks straight into registers, a ring of
//    kDvRing 32-wide K steps in flight, and meets the other waves once, at
//    the end, where the parts are summed through LDS in a fixed order;
//  * v_mfma_f32_16x16x32: A = the expert's rows (x rows gathered by pair, or
//    intermediate rows by pair; 16 per row block), B = weight columns.
//    [K,N] weights (gate / up / fc1 / down): lane (g, i) (g = lane / 16,
//    i = lane % 16) loads k-rows k0 + 8g .. +7 of columns c_i .. c_i + CPL-1
//    (8 loads of 2*CPL bytes) and transposes that 8 x CPL block of 16-bit
//    values with v_perm into CPL MFMA operands: operand j holds the 8 k of
//    column c_i + j, so MFMA j computes columns {c_i + j}. [N,K] weights
//    (Nomic fc2): one 16-byte load is the operand of column n, k0 + 8g .. +7.
//    The A operand of lane (g, r) holds row r at the same 8 k.
// Workgroup outputs go through LDS: each wave stores its f32 part of the
// block, then every thread sums the parts of 8 consecutive columns of one row
// (gate/up: act(gate) * up), converts and stores them with one 16-byte store:
//  gate/up, fc1 : inter[p] = dtype(act(x_t . G) (* x_t . U))        (p = t*k + j)
//  down, fc2    : rows[p]  = dtype(w_p * (inter[p] . D))             (summed per token afterwards)
// No workgroup reads what another writes: the kernel boundaries order the
// launches.
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
constexpr int kDvRing = 4;   // steps in flight per wave

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

// The touched-expert bitmap and this workgroup's expert (the u-th touched
// one), in LDS; the expert ids are kept in s_idx (-1: dropped). Returns the
// expert, or -1 when the workgroup has none.
template <int NT>
__device__ __forceinline__ int dec_expert(const DecArgs& a, int u, uint32_t* s_bm, int32_t* s_idx, int* s_misc) {
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
    // wave 0: the u-th set bit (each lane two words: E <= 4096)
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
        if (lane == 0) s_misc[0] = -1;
        __builtin_amdgcn_wave_barrier();
        if (u >= excl && u < incl) {
            int need = u - excl;  // set bits to skip in this lane's words
            uint32_t w = w0;
            int base = 64 * lane;
            if (need >= __popc(w0)) {
                need -= __popc(w0);
                w = w1;
                base += 32;
            }
            for (int b = 0; b < need; ++b) w &= w - 1u;  // drop the lowest set bits
            s_misc[0] = base + __builtin_ctz(w);
        }
    }
    __syncthreads();
    return s_misc[0];
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
        if (lane == 0) s_misc[4 + wave] = __popcll(m);
        __syncthreads();
        int before = run;
        for (int w = 0; w < wave; ++w) before += s_misc[4 + w];
        int total = run;
        for (int w = 0; w < NT / 64; ++w) total += s_misc[4 + w];
        if (hit) s_rows[before + __popcll(m & ((1ull << lane) - 1ull))] = p;
        run = total;
        __syncthreads();
    }
    return run;
}

template <int DT, int MODE, int RB, int CPL, bool PK, bool W8 = false>
__global__ __launch_bounds__(64 * kDvWaves, 1) void moe_dec_gemv(DecArgs a) {
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    // [K,N] weights (the API layout but Nomic's fc2); [N,K]: fc2, every GEMM
    // on pre-packed weights (PK) and on fp8 codes (W8)
    constexpr bool TRANS = (MODE != kFc2Rows) && !PK && !W8;
    // W8: OCP fp8 e4m3 codes [E][N][K] (one byte per weight) with per-column
    // f32 scales. A step is 64 k: a lane's 16-byte load holds k0 + 16g .. +15
    // of its column, the operands of two MFMAs (converted exactly to DT),
    // and the A operand holds the same k of its row in two 16-byte loads.
    constexpr int KSTEP = W8 ? 64 : kDvStep;
    constexpr int KG = W8 ? 16 : 8;   // k per lane group per step
    constexpr int WB = W8 ? 1 : 2;    // bytes per weight
    constexpr bool ROWS = (MODE == kDownRows || MODE == kFc2Rows);
    constexpr int NT = 64 * kDvWaves;
    constexpr int WGC = 16 * CPL;                // output columns per workgroup
    constexpr int NPART = kDvWaves;              // f32 parts in LDS (gate/up: 2 gate, 2 up)
    constexpr int KP = DUAL ? kDvWaves / 2 : kDvWaves;  // K parts per tensor
    constexpr int NB = TRANS ? CPL : WGC / 16;   // MFMA column blocks per step (operands)
    constexpr int NLD = TRANS ? 8 : NB;          // weight loads per lane per step
    static_assert(CPL == 2 || CPL == 4 || CPL == 8, "columns per lane");
    static_assert(!TRANS || NB == CPL, "operands");

    __shared__ uint32_t s_bm[kDecMaxE / 32];
    __shared__ int32_t s_idx[kDecMaxPairs];
    __shared__ int32_t s_rows[kDecMaxPairs];
    __shared__ int s_misc[4 + kDvWaves];
    __shared__ __attribute__((aligned(16))) float s_part[NPART][RB * 16][WGC];

    const int u = blockIdx.x / a.nblk, cb = blockIdx.x - u * a.nblk;
    const int e = dec_expert<NT>(a, u, s_bm, s_idx, s_misc);
    if (e < 0) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int tensor = DUAL ? (wave >> 1) : 0;
    const int kpart = DUAL ? (wave & 1) : wave;
    const int K = a.K, N = a.N;
    const int col0 = cb * WGC;

    // weights of expert e (this wave's tensor): in-range loads only, zeros past
    const char* wbase = reinterpret_cast<const char*>(tensor ? a.B1 : a.B0) + (long long)e * a.strideB * WB;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wbase), 0, (int)(a.strideB * WB), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.A), 0, (int)a.a_bytes, 0x00020000);

    // this wave's steps: a whole number of ring rounds (steps past K load
    // zeros), so that the ring loop needs no guard
    const int nks = (K + KSTEP - 1) / KSTEP;
    const int per = ((nks + KP - 1) / KP + kDvRing - 1) / kDvRing * kDvRing;
    const int s_lo = kpart * per;

    // per-lane column(s): [K,N]: columns col0 + CPL*li .. +CPL-1 of every
    // k-row; [N,K]: column col0 + 16*b + li of block b
    int ncol[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ncol[b] = TRANS ? col0 + CPL * li + b : col0 + 16 * b + li;

    // per-lane weight offsets, fixed: [K,N]: k-row 8g, columns ncol[0] ..;
    // [N,K]: column ncol[b], k 8g. A lane whose columns lie past N starts at
    // kOob. (Every offset stays below 2^32: kOob plus less than the expert's
    // 2^31 bytes.)
    const uint32_t ldb2 = (uint32_t)a.ldb * (uint32_t)WB;  // bytes per weight row
    uint32_t wlane[TRANS ? 1 : NB];
#pragma unroll
    for (int b = 0; b < (TRANS ? 1 : NB); ++b)
        wlane[b] = ncol[b] < N ? (TRANS ? 8u * (uint32_t)g * ldb2 + 2u * (uint32_t)ncol[0]
                                        : (uint32_t)ncol[b] * ldb2 + 16u * (uint32_t)g)
                               : kOob;

    // ring of steps: weight chunks (CPL 16-bit values each for [K,N], 8 for
    // [N,K]) and the A rows. Branch-free offsets (a select or branch on the
    // step made the compiler wait for every load in flight): K positions
    // past K read zeros (kOob); a [K,N] k-row past K lies past the expert's
    // matrix, which the buffer range turns into zeros as well.
    constexpr int WDW = TRANS ? CPL / 2 : 4;  // dwords per weight load
    uint32_t wv[kDvRing][NLD][WDW];
    u32x4 xv[kDvRing][RB][W8 ? 2 : 1];
    auto load_w = [&](int i, int st) {
        const int s = s_lo + st;
        const bool kok = s * KSTEP + KG * g < K;  // this lane's k of the step
#pragma unroll
        for (int t = 0; t < NLD; ++t) {
            uint32_t o;
            if constexpr (TRANS) o = wlane[0] + (uint32_t)(s * KSTEP + t) * ldb2;
            else o = kok ? wlane[t] + (uint32_t)(s * KSTEP * WB) : kOob;
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
    for (int i = 0; i < kDvRing; ++i) load_w(i, i);
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
            const bool kok = s * KSTEP + KG * g < K;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int h = 0; h < (W8 ? 2 : 1); ++h)
                    xv[i][rb][h] = __builtin_amdgcn_raw_buffer_load_b128(
                        rx, kok ? abase[rb] + (uint32_t)(s * KSTEP) * 2u + 16u * h : kOob, 0, 0);
        };
        auto load = [&](int i, int st) {
            load_w(i, st);
            load_a(i, st);
        };
        auto compute = [&](int i) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if constexpr (W8) {
                    // codes k0 + 16g .. +7 and .. +15 of column b: two operands
                    const u32x4 wl = fp8x8_to<DT>(u32x2{wv[i][b][0], wv[i][b][1]});  // exact in DT
                    const u32x4 wh = fp8x8_to<DT>(u32x2{wv[i][b][2], wv[i][b][3]});
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        acc[rb][b] = mfma16<DT>(xv[i][rb][0], wl, acc[rb][b]);
                        acc[rb][b] = mfma16<DT>(xv[i][rb][1], wh, acc[rb][b]);
                    }
                } else {
                    u32x4 bop;
                    if constexpr (TRANS) {
                        uint32_t r[8][CPL / 2];
#pragma unroll
                        for (int t = 0; t < 8; ++t)
#pragma unroll
                            for (int d = 0; d < CPL / 2; ++d) r[t][d] = wv[i][t][d];
                        bop = column_operand<CPL>(r, b);
                    } else {
                        bop = u32x4{wv[i][b][0], wv[i][b][1], wv[i][b][2], wv[i][b][3]};
                    }
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) acc[rb][b] = mfma16<DT>(xv[i][rb][0], bop, acc[rb][b]);
                }
            }
        };
        // per is a positive multiple of kDvRing. The first ring round is
        // peeled: its loads went out in another order (the weights first,
        // before the rows were known), and inside the loop the compiler would
        // keep that round's shorter waits for every round. The last round
        // loads nothing; a further row chunk streams the weights again.
        if (c0 > 0) {
#pragma unroll
            for (int i = 0; i < kDvRing; ++i) load_w(i, i);
        }
#pragma unroll
        for (int i = 0; i < kDvRing; ++i) load_a(i, i);
        // (sched_barrier: the scheduler would otherwise hoist the MFMAs of
        // later slots above this slot's refill, waiting for data that should
        // still be in flight)
        if (per > kDvRing) {
#pragma unroll
            for (int i = 0; i < kDvRing; ++i) {
                compute(i);
                __builtin_amdgcn_sched_barrier(0);
                load(i, i + kDvRing);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int st = kDvRing; st + kDvRing < per; st += kDvRing) {
#pragma unroll
                for (int i = 0; i < kDvRing; ++i) {
                    compute(i);
                    __builtin_amdgcn_sched_barrier(0);
                    load(i, st + i + kDvRing);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kDvRing; ++i) compute(i);

        // parts to LDS: lane (g, li) holds rows 4g .. 4g+3 of each row block
        // at local column CPL*li + b ([K,N]) or 16b + li ([N,K])
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    s_part[wave][rb * 16 + 4 * g + v][TRANS ? CPL * li + b : 16 * b + li] = acc[rb][b][v];
        __syncthreads();

        // every thread: 8 consecutive output columns of one row; the parts
        // summed in a fixed order (gate/up: gate = parts 0 + 1, up = 2 + 3)
        constexpr int CH = WGC / 8;
        auto epilogue = [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
            for (int q = tid; q < m_valid * CH; q += NT) {
                const int m = q / CH, c8 = (q - m * CH) * 8;
                const int col = col0 + c8;
                if (col >= N) continue;
                const int p = s_rows[c0 + m];
                const float w = ROWS ? a.routing_w[p] : 1.0f;
                float h[8];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    f32x4 v[NPART];
#pragma unroll
                    for (int pt = 0; pt < NPART; ++pt)
                        v[pt] = *reinterpret_cast<const f32x4*>(&s_part[pt][m][c8 + 4 * half]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        // (fp8 weights: the column scales on the f32 sums first)
                        const int cc = col + 4 * half + j;
                        const float s0 = W8 ? (cc < N ? a.scale0[(long long)e * N + cc] : 0.0f) : 1.0f;
                        float y;
                        if constexpr (DUAL) {
                            const float s1 = W8 ? (cc < N ? a.scale1[(long long)e * N + cc] : 0.0f) : 1.0f;
                            y = act_t<ACT>(s0 * (v[0][j] + v[1][j])) * (s1 * (v[2][j] + v[3][j]));
                        } else {
                            y = s0 * (((v[0][j] + v[1][j]) + v[2][j]) + v[3][j]);
                            if constexpr (GATHER) y = act_t<ACT>(y);
                        }
                        h[4 * half + j] = ROWS ? w * y : y;
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
        if constexpr (GATHER) with_act(a.act, epilogue);
        else epilogue(std::integral_constant<int, kSilu>{});
        __syncthreads();  // the parts are read before the next row chunk writes them
    }
}

template <int DT, int MODE, int RB, int CPL>
hipError_t launch_cfg(const DecArgs& a, hipStream_t stream) {
    const long long nwg = (long long)a.max_groups * a.nblk;
    if (nwg > 0x7fffffffLL) return hipErrorInvalidValue;
    if (nwg <= 0) return hipSuccess;
    if (a.w8) {
        // fp8 codes are [N,K] for every GEMM (Nomic's fc2 runs the down mode)
        constexpr int M8 = MODE == kFc2Rows ? kDownRows : MODE;
        hipLaunchKernelGGL((moe_dec_gemv<DT, M8, RB, CPL, false, true>), dim3((int)nwg), dim3(64 * kDvWaves), 0,
                           stream, a);
        return hipGetLastError();
    }
    // (Nomic's fc2 is [N,K] either way: no packed instance)
    if constexpr (MODE != kFc2Rows) {
        if (a.packed) {
            hipLaunchKernelGGL((moe_dec_gemv<DT, MODE, RB, CPL, true>), dim3((int)nwg), dim3(64 * kDvWaves), 0,
                               stream, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((moe_dec_gemv<DT, MODE, RB, CPL, false>), dim3((int)nwg), dim3(64 * kDvWaves), 0, stream, a);
    return hipGetLastError();
}

template <int DT, int MODE>
hipError_t launch_mode(const DecArgs& a, hipStream_t stream) {
    const bool rb2 = a.rows_max > 16;
    if (a.cpl == 2) return rb2 ? launch_cfg<DT, MODE, 2, 2>(a, stream) : launch_cfg<DT, MODE, 1, 2>(a, stream);
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
    if (a.cpl != 2 && a.cpl != 4 && a.cpl != 8) return hipErrorInvalidValue;
    if (a.P > kDecMaxPairs || a.E > kDecMaxE) return hipErrorInvalidValue;
    if (dtype == kBF16) return launch_dt<kBF16>(mode, a, stream);
    if (dtype == kF16) return launch_dt<kF16>(mode, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
