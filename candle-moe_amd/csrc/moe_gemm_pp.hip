// Expert-grouped GEMMs, 8-wave ping-pong schedule (gfx950).
//
// Same products, LDS layouts and epilogues as moe_lds_gemm
// (moe_gemm_lds.hip); what changes is who does what when. A 256x256 block
// tile runs 8 waves, two per SIMD (wave w and w+4 share a SIMD). The waves
// form two groups, 0 (waves 0-3) and 1 (waves 4-7), and every K tile of 64
// is two phases separated by s_barrier:
//
//   phase 2j   : group 0 issues the 32 MFMAs of tile j from registers;
//                group 1 reads its fragments of tile j from LDS.
//   phase 2j+1 : group 1 issues its 32 MFMAs of tile j;
//                group 0 refills the LDS stage of tile j with tile j+2
//                (global->LDS DMA) and reads its fragments of tile j+1.
//
// So on every SIMD one wave keeps the matrix core busy with 32 independent
// back-to-back MFMAs while the other wave does the LDS reads, the DMA
// issue and the address arithmetic, and the two swap at each barrier. A
// wave holds all fragments of one K tile (4 k16 steps x (4 A + 2 B) x 16 B
// = 96 VGPRs) next to its 128x64 f32 accumulator (128 registers). Two LDS
// stages of 64 KB: tile j+2 is issued two phases before group 0 reads it.
//
// DMA offsets: each lane's part of an instruction is fixed for the whole
// K loop (gathered row or column chunk, swizzled LDS slot), so it stays in
// a VGPR and the K position goes into the instruction's SGPR offset. Full K
// tiles never leave the operands for lanes whose row / column is valid;
// lanes outside the operand carry an offset past every buffer, which
// returns zeros. A K tail (K % 64 != 0) is issued with per-lane offsets and
// the same zero fill.
#include "cm_lds.hpp"

namespace cm {

using namespace lds;

template <int DT, int MODE>
__global__ __launch_bounds__(512, 1) void moe_pp_gemm(GemmArgs a) {
    constexpr int BM = 256, BN = 256, BK = 64;
    constexpr int WM = 128, WN = 64, MB = WM / 32, NB = WN / 32;
    constexpr int KSTEPS = BK / 16;
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool SET = (MODE == kDownSet || MODE == kFc2Set);
    constexpr bool BNK = (MODE == kFc2 || MODE == kFc2Set);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    constexpr bool SWAP = !ATOMIC;
    constexpr int ACH = BK / 8;                 // 16-byte chunks per K-contiguous row
    constexpr int AROW = BK * 2;                // bytes per K-contiguous row
    constexpr int RPA = 1024 / AROW;            // K-contiguous rows per DMA instruction
    constexpr int A_BYTES = BM * AROW;
    constexpr int B_BYTES = BN * AROW;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int NLW = 4;                      // waves that issue the DMA (group 0)
    constexpr int A_INS = A_BYTES / (1024 * NLW);
    constexpr int B_INS = B_BYTES / (1024 * NLW);
    constexpr int LOADS = A_INS + B_INS;        // DMA instructions per loading wave per tile
    constexpr int NSUB = DUAL ? 2 : 1;          // [K,N] sub-tiles (gate and up apart)
    constexpr int SUBN = BN / NSUB;
    constexpr int BROW = SUBN * 2;
    constexpr int BCH = SUBN / 8;
    constexpr int RPI = 1024 / BROW;            // k-rows per DMA instruction
    constexpr int SUB_BYTES = BK * BROW;
    constexpr int SUB_INS = SUB_BYTES / (1024 * NLW);
    constexpr int NBV = BNK ? B_INS : 1;        // per-lane B offsets kept
    static_assert(A_INS * 1024 * NLW == A_BYTES && SUB_INS * NSUB == B_INS, "DMA split");
    static_assert(BNK || (BCH >= 16 && (RPI * NLW) % 4 == 0), "[K,N] swizzle must not depend on the instruction");
    static_assert(LOADS < 64, "vmcnt range");
    // per-lane DMA offsets of the loading waves, [wave][quad][lane] x 4 (read
    // back right before each issue, so they do not occupy VGPRs in between)
    constexpr int NOFF = A_INS + NBV;
    constexpr int NQ = (NOFF + 3) / 4;
    __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];
    __shared__ __attribute__((aligned(16))) uint32_t s_voff[NLW * NQ * 64 * 4];
    __shared__ int32_t s_tok[ATOMIC ? BM : 1];
    __shared__ float s_w[ATOMIC ? BM : 1];

    int mt, nt;
    if (!tile_coords(a.n_tiles, *a.num_tiles, mt, nt)) return;
    const int r0 = a.tile_row[mt];
    const int ge = a.tile_exp[mt];  // expert (pair grouping) or expert-set key
    const int m_valid = min(BM, a.offsets[ge + 1] - r0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;      // 0: MFMAs in even phases; 1: MFMAs in odd phases
    const int wl = wave & 3;        // SIMD slot inside the group
    const int wm = grp, wn = wl;    // this wave's 128x64 output sub-tile
    const int N = a.N;

    int seg_exp[SET ? kSetMaxK : 1];
    int n_seg = 1;
    if constexpr (SET) {
        n_seg = decode_set(ge, a.k_top, a.n_experts, seg_exp);
    } else {
        seg_exp[0] = ge;
    }
    const int K = SET ? n_seg * a.seg_len : a.K;
    const int a_pitch = SET ? a.k_top * a.seg_len : a.K;
    const int nk = (K + BK - 1) / BK;
    const bool k_tail = (K % BK) != 0;  // never on the expert-set path (seg_len % 64 == 0)

    const i32x4 rA = make_rsrc(a.A, a.a_bytes);
    const uint32_t smem_base = __builtin_amdgcn_readfirstlane(lds_addr(smem));

    // ---- per-lane DMA offsets of the loading waves (group 0), parked in
    // s_voff. A instruction i of load wave wl covers rows RPA*q .. RPA*q+RPA-1,
    // q = NLW*i + wl.
    // B [N,K]: like A (rows n of the column tile). B [K,N]: instruction i of
    // sub-tile s covers k-rows RPI*q .. RPI*q+RPI-1, q = NLW*i + wl; the
    // lane's column chunk is the same for every i (RPI*NLW is a multiple of
    // 4, so the swizzle row phase r & 3 does not change), only the k-row
    // moves, by RPI*NLW*i, which goes into the SGPR offset.
    if (grp == 0) {
        uint32_t off[NQ * 4];
#pragma unroll
        for (int i = 0; i < NQ * 4; ++i) off[i] = kOob;
#pragma unroll
        for (int i = 0; i < A_INS; ++i) {
            const int r = RPA * (NLW * i + wl) + lane / ACH;
            const int kc = a_swz<ACH>(r, lane % ACH) * 8;  // k offset of the chunk that lands at this lane's slot
            if (r < m_valid) {
                const int src = GATHER ? a.sorted_pair[r0 + r] / a.k_top : r0 + r;
                off[i] = ((uint32_t)src * (uint32_t)a_pitch + (uint32_t)kc) * 2u;
            }
        }
#pragma unroll
        for (int i = 0; i < NBV; ++i) {
            if constexpr (BNK) {
                const int r = RPA * (NLW * i + wl) + lane / ACH;
                const int n = nt * BN + r;
                const int kc = a_swz<ACH>(r, lane % ACH) * 8;
                off[A_INS + i] = n < N ? ((uint32_t)n * (uint32_t)a.ldb + (uint32_t)kc) * 2u : kOob;
            } else {
                const int r = RPI * wl + lane / BCH;
                const int c = kn_swz<BCH>(r, lane % BCH);
                const int col = nt * SUBN + c * 8;
                off[A_INS + i] = col < N ? ((uint32_t)col + (uint32_t)r * (uint32_t)a.ldb) * 2u : kOob;
            }
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            u32x4 v = {off[4 * q], off[4 * q + 1], off[4 * q + 2], off[4 * q + 3]};
            *reinterpret_cast<u32x4*>(&s_voff[((wl * NQ + q) * 64 + lane) * 4]) = v;
        }
    }

    // Issue the DMA of K tile t into stage t & 1 (group 0 only).
    auto issue_tile = [&](int t) {
        const int k0 = t * BK;
        const uint32_t sA = smem_base + (t & 1) * STAGE;
        const uint32_t sB = sA + A_BYTES;
        const bool tail = k_tail && t == nk - 1;
        int kk = k0, e = seg_exp[0];
        if constexpr (SET) {
            const int s = k0 / a.seg_len;
            e = seg_exp[s < kSetMaxK ? s : 0];
            kk = k0 - s * a.seg_len;
        }
        uint32_t a_voff[A_INS], b_voff[NBV];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(&s_voff[((wl * NQ + q) * 64 + lane) * 4]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int i = 4 * q + c;
                if (i < A_INS) a_voff[i] = v[c];
                else if (i < A_INS + NBV) b_voff[i - A_INS] = v[c];
            }
        }
        const long long eoff = (long long)e * a.strideB;
        const i32x4 rB0 = make_rsrc(reinterpret_cast<const uint16_t*>(a.B0) + eoff, a.strideB * 2);
        i32x4 rB1 = rB0;
        if constexpr (DUAL) rB1 = make_rsrc(reinterpret_cast<const uint16_t*>(a.B1) + eoff, a.strideB * 2);
        if (!tail) {
#pragma unroll
            for (int i = 0; i < A_INS; ++i) dma16s(rA, sA + (NLW * i + wl) * 1024, a_voff[i], (uint32_t)k0 * 2u);
#pragma unroll
            for (int i = 0; i < B_INS; ++i) {
                if constexpr (BNK) {
                    dma16s(rB0, sB + (NLW * i + wl) * 1024, b_voff[i], (uint32_t)kk * 2u);
                } else {
                    const int sub = i / SUB_INS, ii = i % SUB_INS;
                    const uint32_t soff = (uint32_t)(kk + RPI * NLW * ii) * (uint32_t)a.ldb * 2u;
                    dma16s(sub ? rB1 : rB0, sB + sub * SUB_BYTES + (NLW * ii + wl) * 1024, b_voff[0], soff);
                }
            }
        } else {
            // K tail: per-lane offsets, chunks at k >= K read as zeros
#pragma unroll
            for (int i = 0; i < A_INS; ++i) {
                const int r = RPA * (NLW * i + wl) + lane / ACH;
                const int kc = k0 + a_swz<ACH>(r, lane % ACH) * 8;
                const uint32_t off = (a_voff[i] == kOob || kc >= K) ? kOob : a_voff[i] + (uint32_t)k0 * 2u;
                dma16(rA, sA + (NLW * i + wl) * 1024, off);
            }
#pragma unroll
            for (int i = 0; i < B_INS; ++i) {
                if constexpr (BNK) {
                    const int r = RPA * (NLW * i + wl) + lane / ACH;
                    const int kc = kk + a_swz<ACH>(r, lane % ACH) * 8;
                    const uint32_t off = (b_voff[i] == kOob || kc >= K) ? kOob : b_voff[i] + (uint32_t)kk * 2u;
                    dma16(rB0, sB + (NLW * i + wl) * 1024, off);
                } else {
                    const int sub = i / SUB_INS, ii = i % SUB_INS;
                    const int kr = kk + RPI * (NLW * ii + wl) + lane / BCH;
                    const uint32_t off = (b_voff[0] == kOob || kr >= K)
                                             ? kOob
                                             : b_voff[0] + (uint32_t)(kk + RPI * NLW * ii) * (uint32_t)a.ldb * 2u;
                    dma16(sub ? rB1 : rB0, sB + sub * SUB_BYTES + (NLW * ii + wl) * 1024, off);
                }
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

    // Fragment addresses. A (and [N,K] B) rows R + 32*mb, R = wm*128 + lr
    // (n: wn*64 + lr): with 8 chunks per row, a_swz(R + 32*mb, 2*kk + lh) =
    // s0 ^ 2*kk ^ 4*(mb & 1), s0 = lh ^ (lr & 7) ^ (lr >> 3), so four base
    // addresses (x = kk ^ 2*(mb & 1)) plus immediate row offsets cover all
    // 16 reads. [K,N] transposed reads: lane (tg, tj) addresses
    // B[kr][p + 4*(tj%4)] of its sub-tile with kr = 16*kk + tr_k (+4 for the
    // second read), p = block column + 16*(tg&1); the swizzle depends on
    // kr & 3 = tr_k & 3 only, so k steps are immediate offsets too. DUAL:
    // block nb is the gate (even) or up (odd) sub-tile at the same columns.
    const int lr = lane & 31, lh = lane >> 5;
    const int tj = lane & 15, tg = lane >> 4;
    const int s0 = (lh ^ (lr & 7) ^ (lr >> 3)) & 7;
    uint32_t a_base[4], bnk_base[BNK ? 4 : 1];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        a_base[x] = (uint32_t)((wm * WM + lr) * AROW + ((s0 ^ (2 * x)) << 4));
        if constexpr (BNK) bnk_base[x] = (uint32_t)(A_BYTES + (wn * WN + lr) * AROW + ((s0 ^ (2 * x)) << 4));
    }
    constexpr int NTRB = BNK ? 1 : (DUAL ? 1 : NB);
    uint32_t tr_base[NTRB];
    const int tr_k = 8 * (tg >> 1) + (tj >> 2);
#pragma unroll
    for (int v = 0; v < NTRB; ++v) {
        const int p = (DUAL ? wn * (WN / 2) : wn * WN + v * 32) + 16 * (tg & 1) + 4 * (tj & 3);
        const int cc = kn_swz<BCH>(tr_k, p >> 3);
        tr_base[v] = (uint32_t)(A_BYTES + cc * 16 + (p & 7) * 2 + tr_k * BROW);
    }

    u32x4 af[KSTEPS][MB], bfr[KSTEPS][NB];
    // All fragments of one K tile of this wave's sub-tile.
    auto load_frags = [&](int stage) {
        const char* st = smem + stage * STAGE;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                af[kk][mb] = *reinterpret_cast<const u32x4*>(st + a_base[kk ^ (2 * (mb & 1))] + mb * 32 * AROW);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (BNK) {
                    bfr[kk][nb] = *reinterpret_cast<const u32x4*>(st + bnk_base[kk ^ (2 * nb)] + nb * 32 * AROW);
                } else {
                    const char* base = st + tr_base[DUAL ? 0 : nb] + (DUAL ? nb * SUB_BYTES : 0) + kk * 16 * BROW;
                    bfr[kk][nb] = tr_pair(base, base + 4 * BROW);
                }
            }
        }
    };
    auto mfma_tile = [&]() {
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if constexpr (SWAP) acc[mb][nb] = mfma32<DT>(bfr[kk][nb], af[kk][mb], acc[mb][nb]);
                    else acc[mb][nb] = mfma32<DT>(af[kk][mb], bfr[kk][nb], acc[mb][nb]);
                }
    };

    if constexpr (ATOMIC) {
        if (tid < BM) {
            const int p = a.sorted_pair[r0 + (tid < m_valid ? tid : 0)];
            s_tok[tid] = p / a.k_top;
            s_w[tid] = a.routing_w[p];
        }
    }

    if (nk > 0) {
        // prologue: tiles 0 and 1 in flight, group 0 reads tile 0
        if (grp == 0) {
            issue_tile(0);
            if (nk > 1) {
                issue_tile(1);
                wait_vm<LOADS>();
            } else {
                wait_vm<0>();
            }
        }
        block_barrier();
        // Separate code per group, so that each wave's fragment registers
        // have one straight-line producer and consumer.
        if (grp == 0) {
            load_frags(0);
            wait_lgkm0();
            block_barrier();
            for (int j = 0; j < nk; ++j) {
                // phase 2j: MFMAs of tile j; this wave's DMA of tile j+1 (issued one
                // phase ago) must land before the barrier that hands tile j+1 over
                __builtin_amdgcn_sched_barrier(0);
                mfma_tile();
                __builtin_amdgcn_sched_barrier(0);
                if (j + 1 < nk) wait_vm<0>();
                block_barrier();
                // phase 2j+1: refill stage j & 1 (both groups have read tile j) with
                // tile j+2, read the fragments of tile j+1
                if (j + 1 < nk) {
                    if (j + 2 < nk) issue_tile(j + 2);
                    load_frags((j + 1) & 1);
                    wait_lgkm0();
                    block_barrier();
                }
            }
        } else {
            block_barrier();
            for (int j = 0; j < nk; ++j) {
                // phase 2j: read the fragments of tile j
                load_frags(j & 1);
                wait_lgkm0();
                block_barrier();
                // phase 2j+1: MFMAs of tile j
                __builtin_amdgcn_sched_barrier(0);
                mfma_tile();
                __builtin_amdgcn_sched_barrier(0);
                if (j + 1 < nk) block_barrier();
            }
        }
    }

    // (s_tok holds the pair path's tokens only: the expert-set epilogue reads
    // its rows from tok_sorted)
    tile_epilogue<DT, MODE, BN, WM, WN, MB, NB>(a, acc, r0, m_valid, nt, wm, wn, lane, ATOMIC ? s_tok : nullptr,
                                                s_w);
}

template <int DT>
static hipError_t launch_pp_dt(int mode, const GemmArgs& a, hipStream_t stream) {
    const int nwg = a.m_tiles_max * a.n_tiles;
    if (nwg <= 0) return hipSuccess;
    switch (mode) {
        case kGateUp: hipLaunchKernelGGL((moe_pp_gemm<DT, kGateUp>), dim3(nwg), dim3(512), 0, stream, a); break;
        case kFc1: hipLaunchKernelGGL((moe_pp_gemm<DT, kFc1>), dim3(nwg), dim3(512), 0, stream, a); break;
        case kDown: hipLaunchKernelGGL((moe_pp_gemm<DT, kDown>), dim3(nwg), dim3(512), 0, stream, a); break;
        case kFc2: hipLaunchKernelGGL((moe_pp_gemm<DT, kFc2>), dim3(nwg), dim3(512), 0, stream, a); break;
        case kDownSet: hipLaunchKernelGGL((moe_pp_gemm<DT, kDownSet>), dim3(nwg), dim3(512), 0, stream, a); break;
        case kFc2Set: hipLaunchKernelGGL((moe_pp_gemm<DT, kFc2Set>), dim3(nwg), dim3(512), 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_gemm_pp(int mode, int dtype, const GemmArgs& a, hipStream_t stream) {
    if (dtype == kBF16) return launch_pp_dt<kBF16>(mode, a, stream);
    if (dtype == kF16) return launch_pp_dt<kF16>(mode, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
