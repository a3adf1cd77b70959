// Expert-grouped GEMMs, LDS-DMA variant (gfx950).
//
// Same products and epilogues as moe_mfma_gemm (moe_gemm.hip); what changes
// is how tiles reach the matrix cores:
//  * Both operands go global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
//    staging, no v_perm). One wave instruction moves 1 KB: lane l lands at
//    byte 16*l, so each lane is pointed at the global chunk that belongs at
//    its (swizzled) LDS position.
//  * Weights stored [K,N] (N contiguous) stay row-major in LDS; the MFMA B
//    fragments are read with ds_read_b64_tr_b16, which transposes inside each
//    16-lane group: if lane j addresses B[k0 + j/4][n0 + 4*(j%4)], lane i
//    receives B[k0 .. k0+3][n0 + i]. Two such reads give the 8 consecutive K
//    values of one column that v_mfma_f32_32x32x16 expects.
//  * Buffer resources return zeros for rows / columns outside the operand,
//    which covers row, column and K tails without branches.
//  * NST-stage LDS ring: while stage kt is consumed by the MFMAs the loads of
//    stages kt+1 .. kt+NST-1 are in flight; one s_waitcnt + s_barrier per K
//    tile hands stage kt over and stage kt-1 back.
// LDS layouts (BK = 32 or 64 bf16/f16 per stage):
//  A and [N,K] weights: BK*2-byte rows, 16-byte chunk c of row r stored at
//                       a_swz(r, c) (conflict-free b128 reads).
//  [K,N] weights      : one sub-tile per tensor (gate and up apart), rows of
//                       SUBN*2 bytes (one per k), chunk c of row k stored at
//                       kn_swz(k, c), so the 4 rows of a transposed read hit
//                       disjoint banks.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define CM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

constexpr uint32_t kOob = 0x80000000u;  // buffer offset past every resource (operands are < 2 GiB)

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource (V#) of a raw byte range: base, stride 0, num_records =
// bytes, dword3 0x00020000 (gfx9 data format); loads past num_records
// return zeros. Made wave-uniform so it lives in SGPRs.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, long long bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)b);
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((b >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane((int32_t)bytes);
    r[3] = 0x00020000;
    return r;
}

// One wave instruction: 64 lanes x 16 bytes from the buffer into LDS at
// lds_off + 16*lane. Issued as inline asm so that the compiler neither waits
// for it before unrelated LDS reads nor tracks it: stage hand-over is done
// with the explicit s_waitcnt / s_barrier below.
__device__ __forceinline__ void dma16(const i32x4& r, uint32_t lds_off, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_off), "v"(voff), "s"(r)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" : : : "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)(p));
}

// Rows of K-contiguous tiles (A, [N,K] weights) hold ACH 16-byte chunks
// (ACH = BK / 8); chunk c of row r is stored at a_swz(r, c). 16 lanes of a
// ds_read_b128 read 16 consecutive rows at one logical chunk and land in 16
// distinct bank groups.
template <int ACH>
__device__ __forceinline__ int a_swz(int r, int c) {
    if constexpr (ACH == 8) return (c ^ r ^ (r >> 3)) & 7;
    else return (c ^ (r >> 2)) & 3;
}

// [K,N] sub-tile rows of BCH 16-byte chunks: chunk c of k-row r is stored at
// kn_swz(r, c). A transposed read touches 4 consecutive rows x 4 consecutive
// chunks (c multiple of 4 first) per 32 lanes; the xor sends them to 16
// distinct bank groups (rows are 256 B apart for BCH >= 16, 128 B for 8).
template <int BCH>
__device__ __forceinline__ int kn_swz(int r, int c) {
    if constexpr (BCH >= 16) return c ^ ((r & 3) << 2);
    else return c ^ (((r >> 1) & 1) << 2);
}

// Bijective remap of the hardware dispatch order (workgroup w runs on XCD
// w % 8) to a logical tile id that is contiguous per XCD.
__device__ __forceinline__ void lds_tile_coords(int n_tiles, int& mt, int& nt) {
    const int nwg = gridDim.x;
    const int w = blockIdx.x;
    const int per = nwg >> 3, rem = nwg & 7, xcd = w & 7, idx = w >> 3;
    const int logical = xcd * per + (xcd < rem ? xcd : rem) + idx;
    mt = logical / n_tiles;
    nt = logical - mt * n_tiles;
}

}  // namespace

template <int DT, int BM, int BN, int BK, int NST, int NW, int MODE>
__global__ __launch_bounds__(64 * NW, 1) void moe_lds_gemm(GemmArgs a) {
    // NW waves: 4 in a 2x2 layout (one per SIMD) or 8 in 2x4 (two per SIMD,
    // so one wave's MFMAs cover the other's LDS, DMA and VALU work)
    static_assert(NW == 4 || NW == 8, "waves");
    constexpr int WGN = NW / 2;
    constexpr int WM = BM / 2, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool SET = (MODE == kDownSet || MODE == kFc2Set);
    constexpr bool BNK = (MODE == kFc2 || MODE == kFc2Set);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    constexpr bool SWAP = !ATOMIC;
    static_assert(BK == 32 || BK == 64, "BK");
    constexpr int ACH = BK / 8;            // 16-byte chunks per K-contiguous row
    constexpr int AROW = BK * 2;           // bytes per K-contiguous row
    constexpr int RPA = 1024 / AROW;       // K-contiguous rows per DMA instruction
    constexpr int KSTEPS = BK / 16;
    constexpr int A_BYTES = BM * AROW;
    constexpr int B_BYTES = BN * AROW;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int A_INS = A_BYTES / (1024 * NW);  // DMA instructions per wave per stage
    constexpr int B_INS = B_BYTES / (1024 * NW);
    constexpr int LOADS = A_INS + B_INS;
    // [K,N] weights: gate and up (DUAL) get separate sub-tiles, so that every
    // DMA instruction reads one tensor through one (uniform) buffer resource.
    constexpr int NSUB = DUAL ? 2 : 1;
    constexpr int SUBN = BN / NSUB;        // columns per sub-tile
    constexpr int BROW = SUBN * 2;         // bytes per k-row of a sub-tile
    constexpr int BCH = SUBN / 8;          // 16-byte chunks per k-row
    constexpr int RPI = 1024 / BROW;       // k-rows per DMA instruction
    constexpr int SUB_BYTES = BK * BROW;
    constexpr int SUB_INS = SUB_BYTES / (1024 * NW);  // per wave, per sub-tile
    static_assert(A_INS * 1024 * NW == A_BYTES && SUB_INS * 1024 * NW == SUB_BYTES, "DMA split");
    static_assert(!DUAL || (WN % 64) == 0, "gate/up pairs must stay inside one wave");
    static_assert(BNK || BCH >= 8, "[K,N] tiles need >= 8 chunks per row for the swizzle");
    static_assert(BNK || SUB_INS * NSUB == B_INS, "B tile split");
    static_assert(LOADS * (NST - 2) < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) char smem[NST * STAGE];
    __shared__ int32_t s_tok[ATOMIC ? BM : 1];
    __shared__ float s_w[ATOMIC ? BM : 1];

    int mt, nt;
    lds_tile_coords(a.n_tiles, mt, nt);
    if (mt >= *a.num_tiles) return;
    const int r0 = a.tile_row[mt];
    const int grp = a.tile_exp[mt];
    const int m_valid = min(BM, a.offsets[grp + 1] - r0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int N = a.N;

    int seg_exp[SET ? kSetMaxK : 1];
    int n_seg = 1;
    if constexpr (SET) {
        const int base = a.n_experts + 1;
        int key = grp;
        n_seg = 0;
        for (int s = a.k_top - 1; s >= 0; --s) {
            seg_exp[s] = key % base;
            key /= base;
        }
        for (int s = 0; s < a.k_top; ++s) n_seg += seg_exp[s] < a.n_experts;
    } else {
        seg_exp[0] = grp;
    }
    const int K = SET ? n_seg * a.seg_len : a.K;
    const int a_pitch = SET ? a.k_top * a.seg_len : a.K;

    const i32x4 rA = make_rsrc(a.A, a.a_bytes);
    const uint32_t smem_base = __builtin_amdgcn_readfirstlane(lds_addr(smem));

    // ---- per-lane DMA sources. A: instruction i of this wave covers rows
    // RPA*q .. RPA*q+RPA-1, q = NW*i + wave.
    uint32_t a_row[A_INS];
    int a_kc[A_INS];
#pragma unroll
    for (int i = 0; i < A_INS; ++i) {
        const int r = RPA * (NW * i + wave) + lane / ACH;
        a_kc[i] = a_swz<ACH>(r, lane % ACH) * 8;  // k offset of the chunk that lands at this lane's slot
        if (r < m_valid) {
            const int src = GATHER ? a.sorted_pair[r0 + r] / a.k_top : r0 + r;
            a_row[i] = (uint32_t)src * (uint32_t)a_pitch * 2u;
        } else {
            a_row[i] = kOob;
        }
    }
    // B: [K,N] sub-tiles: instruction i (i % SUB_INS within sub-tile i / SUB_INS)
    // covers k-rows RPI*q .. RPI*q+RPI-1; [N,K] tiles: like A.
    uint32_t b_col[B_INS];  // byte offset of the column chunk (or n-row start for [N,K])
    int b_r[B_INS];         // k-row in tile ([K,N]) / k offset of the chunk ([N,K])
#pragma unroll
    for (int i = 0; i < B_INS; ++i) {
        if constexpr (BNK) {
            const int r = RPA * (NW * i + wave) + lane / ACH;
            const int n = nt * BN + r;
            b_r[i] = a_swz<ACH>(r, lane % ACH) * 8;
            b_col[i] = n < N ? (uint32_t)n * (uint32_t)a.ldb * 2u : kOob;
        } else {
            const int q = NW * (i % SUB_INS) + wave;
            const int r = RPI * q + lane / BCH;
            const int c = kn_swz<BCH>(r, lane % BCH);
            const int col = nt * SUBN + c * 8;
            b_r[i] = r;
            b_col[i] = col < N ? (uint32_t)col * 2u : kOob;
        }
    }

    auto issue = [&](int stage, int k0) {
        const uint32_t sA = smem_base + stage * STAGE;
        const uint32_t sB = sA + A_BYTES;
#pragma unroll
        for (int i = 0; i < A_INS; ++i) {
            const int kc = k0 + a_kc[i];
            const uint32_t off = (a_row[i] == kOob || kc >= K) ? kOob : a_row[i] + (uint32_t)kc * 2u;
            dma16(rA, sA + (NW * i + wave) * 1024, off);
        }
        int kk = k0, klim = K, e = seg_exp[0];
        if constexpr (SET) {
            const int s = k0 / a.seg_len;
            e = seg_exp[s < kSetMaxK ? s : 0];
            kk = k0 - s * a.seg_len;
            klim = a.seg_len;
        }
        const long long eoff = (long long)e * a.strideB;
        const i32x4 r0s = make_rsrc(reinterpret_cast<const uint16_t*>(a.B0) + eoff, a.strideB * 2);
        i32x4 r1s = r0s;
        if constexpr (DUAL) r1s = make_rsrc(reinterpret_cast<const uint16_t*>(a.B1) + eoff, a.strideB * 2);
#pragma unroll
        for (int i = 0; i < B_INS; ++i) {
            uint32_t off;
            if constexpr (BNK) {
                const int kc = kk + b_r[i];
                off = (b_col[i] == kOob || kc >= klim) ? kOob : b_col[i] + (uint32_t)kc * 2u;
                dma16(r0s, sB + (NW * i + wave) * 1024, off);
            } else {
                const int kr = kk + b_r[i];
                off = (b_col[i] == kOob || kr >= klim) ? kOob : b_col[i] + (uint32_t)kr * (uint32_t)a.ldb * 2u;
                const int sub = i / SUB_INS;  // compile-time after unrolling
                dma16(sub ? r1s : r0s, sB + sub * SUB_BYTES + (NW * (i % SUB_INS) + wave) * 1024, off);
            }
        }
    };

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // fragment addresses (bytes inside a stage) that do not depend on kk
    const int lr = lane & 31, lh = lane >> 5;
    int a_frag_row[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a_frag_row[mb] = wm * WM + mb * 32 + lr;
    // [K,N] transposed read: lane (g = lane/16, j = lane%16) addresses
    // B[kbase + j/4][p + 4*(j%4)] of its sub-tile, p = block column + 16*(g&1).
    // DUAL: block nb is the gate (even) or up (odd) half of logical columns
    // wn*WN/2 + (nb/2)*32 of the tile.
    const int tj = lane & 15, tg = lane >> 4;
    int b_tr_col[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        b_tr_col[nb] = (DUAL ? wn * (WN / 2) + (nb >> 1) * 32 : wn * WN + nb * 32) + 16 * (tg & 1) + 4 * (tj & 3);
    }
    const int tr_k = 8 * (tg >> 1) + (tj >> 2);  // + kk*16 (+4 for the second read)

    // Fragments of one k16 step: MB A rows blocks and NB B column blocks.
    auto load_frags = [&](const char* sA, const char* sB, int kk, u32x4 (&af)[MB], u32x4 (&bfr)[NB]) {
        const int c = kk * 2 + lh;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int r = a_frag_row[mb];
            af[mb] = *reinterpret_cast<const u32x4*>(sA + r * AROW + a_swz<ACH>(r, c) * 16);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if constexpr (BNK) {
                const int r = wn * WN + nb * 32 + lr;
                bfr[nb] = *reinterpret_cast<const u32x4*>(sB + r * AROW + a_swz<ACH>(r, c) * 16);
            } else {
                const int p = b_tr_col[nb];
                const int kr = kk * 16 + tr_k;  // kr & 3 == (tj >> 2); kr + 4 keeps the swizzle
                const int cc = kn_swz<BCH>(kr, p >> 3);
                const char* base = sB + (DUAL ? (nb & 1) * SUB_BYTES : 0) + cc * 16 + (p & 7) * 2;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(CM_LDS(base + kr * BROW)));
                const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(CM_LDS(base + (kr + 4) * BROW)));
                u32x4 v;
                v[0] = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
                v[1] = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
                v[2] = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
                v[3] = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
                bfr[nb] = v;
            }
        }
    };
    auto mfma_step = [&](const u32x4 (&af)[MB], const u32x4 (&bfr)[NB]) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (SWAP) acc[mb][nb] = mfma32<DT>(bfr[nb], af[mb], acc[mb][nb]);
                else acc[mb][nb] = mfma32<DT>(af[mb], bfr[nb], acc[mb][nb]);
            }
    };
    // LDS read instructions per k16 step (ds_read_b128 for A and [N,K] B,
    // two ds_read_b64_tr_b16 per [K,N] B block).
    constexpr int DS_PER_STEP = MB + (BNK ? NB : 2 * NB);
    constexpr int MFMA_PER_STEP = MB * NB;
    // Pin the schedule of one region: one MFMA, then one LDS read, while
    // reads remain, then the remaining MFMAs (masks: 0x8 MFMA, 0x100 DS read).
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < MFMA_PER_STEP; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < DS_PER_STEP) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    // KSTEPS k16 steps per stage; the fragments of step kk+1 are read while
    // the MFMAs of step kk run (two register sets).
    auto compute = [&](int stage) {
        const char* sA = smem + stage * STAGE;
        const char* sB = sA + A_BYTES;
        u32x4 af0[MB], bf0[NB], af1[MB], bf1[NB];
        load_frags(sA, sB, 0, af0, bf0);
        __builtin_amdgcn_sched_barrier(0);
        load_frags(sA, sB, 1, af1, bf1);
        mfma_step(af0, bf0);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KSTEPS == 4) {
            load_frags(sA, sB, 2, af0, bf0);
            mfma_step(af1, bf1);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
            load_frags(sA, sB, 3, af1, bf1);
            mfma_step(af0, bf0);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
        }
        mfma_step(af1, bf1);
        __builtin_amdgcn_sched_barrier(0);
    };

    if constexpr (ATOMIC) {
        if (tid < BM) {
            const int p = a.sorted_pair[r0 + (tid < m_valid ? tid : 0)];
            s_tok[tid] = p / a.k_top;
            s_w[tid] = a.routing_w[p];
        }
    }

    // Stage hand-over, one barrier per K tile: wait for this wave's DMA of
    // stage kt (the NST-2 newer stages may stay in flight) and for its own
    // LDS reads of stage kt-1, then the barrier makes both block-wide; only
    // after it is stage kt-1's slot refilled with tile kt+NST-1.
    const int nk = (K + BK - 1) / BK;
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < nk) issue(s, s * BK);
    for (int kt = 0; kt < nk; ++kt) {
        const int newer = min(NST - 2, nk - 1 - kt);  // stages issued after kt and before this wait
        if constexpr (NST >= 4) {
            if (newer >= 2) wait_vm<2 * LOADS>();
            else if (newer == 1) wait_vm<LOADS>();
            else wait_vm<0>();
        } else if constexpr (NST == 3) {
            if (newer >= 1) wait_vm<LOADS>();
            else wait_vm<0>();
        } else {
            wait_vm<0>();
        }
        wait_lgkm0();
        block_barrier();
        const int ahead = kt + NST - 1;
        if (ahead < nk) issue(ahead % NST, ahead * BK);
        compute(kt % NST);
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (ATOMIC) {
        float* C = reinterpret_cast<float*>(a.C);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ml = wm * WM + mb * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
                if (ml >= m_valid) continue;
                const long long rowoff = (long long)s_tok[ml] * N;
                const float w = s_w[ml];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int col = nt * BN + wn * WN + nb * 32 + lr;
                    if (col < N) unsafeAtomicAdd(C + rowoff + col, w * acc[mb][nb][i]);
                }
            }
        }
    } else {
        const int nsub = 4 * lh;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = wm * WM + mb * 32 + lr;
            if (ml >= m_valid) continue;
            const int r = r0 + ml;
            if constexpr (MODE == kGateUp || MODE == kFc1) {
                const int p = a.sorted_pair[r];
                const int dst = a.pair_dest ? a.pair_dest[p] : r;
                const float wscale = a.fold_w ? a.routing_w[p] : 1.0f;
                uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)dst * N;
                constexpr int PAIRS = DUAL ? NB / 2 : NB;
#pragma unroll
                for (int q = 0; q < PAIRS; ++q) {
                    const int colbase = DUAL ? nt * (BN / 2) + ((wn * WN) / 64 + q) * 32 : nt * BN + wn * WN + q * 32;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = colbase + 8 * g + nsub;
                        if (col >= N) continue;
                        float h[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if constexpr (DUAL) {
                                h[j] = act_fast(acc[mb][2 * q][4 * g + j], a.act) * acc[mb][2 * q + 1][4 * g + j];
                            } else {
                                h[j] = act_fast(acc[mb][q][4 * g + j], a.act);
                            }
                            h[j] *= wscale;
                        }
                        u32x2 v;
                        v[0] = (uint32_t)Elem<DT>::from_f32(h[0]) | ((uint32_t)Elem<DT>::from_f32(h[1]) << 16);
                        v[1] = (uint32_t)Elem<DT>::from_f32(h[2]) | ((uint32_t)Elem<DT>::from_f32(h[3]) << 16);
                        *reinterpret_cast<u32x2*>(C + col) = v;
                    }
                }
            } else {
                const int tok = a.tok_sorted[r];
                uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)tok * N;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int colbase = nt * BN + wn * WN + nb * 32;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = colbase + 8 * g + nsub;
                        if (col >= N) continue;
                        const u32x2 old = *reinterpret_cast<const u32x2*>(C + col);
                        float h[4];
                        h[0] = Elem<DT>::to_f32((uint16_t)(old[0] & 0xffffu)) + acc[mb][nb][4 * g + 0];
                        h[1] = Elem<DT>::to_f32((uint16_t)(old[0] >> 16)) + acc[mb][nb][4 * g + 1];
                        h[2] = Elem<DT>::to_f32((uint16_t)(old[1] & 0xffffu)) + acc[mb][nb][4 * g + 2];
                        h[3] = Elem<DT>::to_f32((uint16_t)(old[1] >> 16)) + acc[mb][nb][4 * g + 3];
                        u32x2 v;
                        v[0] = (uint32_t)Elem<DT>::from_f32(h[0]) | ((uint32_t)Elem<DT>::from_f32(h[1]) << 16);
                        v[1] = (uint32_t)Elem<DT>::from_f32(h[2]) | ((uint32_t)Elem<DT>::from_f32(h[3]) << 16);
                        *reinterpret_cast<u32x2*>(C + col) = v;
                    }
                }
            }
        }
    }
}

template <int DT, int MODE>
hipError_t launch_lds_mode(int cfg, const GemmArgs& a, hipStream_t stream) {
    const int nwg = a.m_tiles_max * a.n_tiles;
    if (nwg <= 0) return hipSuccess;
    if constexpr (DT == kF32) {
        return hipErrorInvalidValue;
    } else {
        switch (cfg) {
            case kLds256:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 32, 4, 4, MODE>), dim3(nwg), dim3(256), 0, stream, a);
                break;
            case kLds256x128:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 128, 64, 3, 4, MODE>), dim3(nwg), dim3(256), 0, stream, a);
                break;
            case kLds128:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 128, 128, 64, 4, 4, MODE>), dim3(nwg), dim3(256), 0, stream, a);
                break;
            case kLds256k64:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 64, 2, 4, MODE>), dim3(nwg), dim3(256), 0, stream, a);
                break;
            case kLds256w8:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 64, 2, 8, MODE>), dim3(nwg), dim3(512), 0, stream, a);
                break;
            case kLds256w8k32:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 32, 4, 8, MODE>), dim3(nwg), dim3(512), 0, stream, a);
                break;
            default:
                return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_lds_dt(int mode, int cfg, const GemmArgs& a, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return launch_lds_mode<DT, kGateUp>(cfg, a, stream);
        case kFc1: return launch_lds_mode<DT, kFc1>(cfg, a, stream);
        case kDown: return launch_lds_mode<DT, kDown>(cfg, a, stream);
        case kFc2: return launch_lds_mode<DT, kFc2>(cfg, a, stream);
        case kDownSet: return launch_lds_mode<DT, kDownSet>(cfg, a, stream);
        case kFc2Set: return launch_lds_mode<DT, kFc2Set>(cfg, a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_gemm_lds(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream) {
    if (dtype == kBF16) return launch_lds_dt<kBF16>(mode, cfg, a, stream);
    if (dtype == kF16) return launch_lds_dt<kF16>(mode, cfg, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
