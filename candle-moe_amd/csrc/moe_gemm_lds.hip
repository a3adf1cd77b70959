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
#include "cm_lds.hpp"

namespace cm {

using namespace lds;

template <int DT, int BM, int BN, int BK, int NST, int NW, int MODE, int WGM = 2, int OCC = 1, bool W8 = false,
          bool PK = false>
__global__ __launch_bounds__(64 * NW, OCC) void moe_lds_gemm(GemmArgs a) {
    // NW waves in WGM rows: 4 in a 2x2 layout (one per SIMD), 8 in 2x4 (two
    // per SIMD, so one wave's MFMAs cover the other's LDS, DMA and VALU work),
    // or all side by side along N (WGM = 1) for 32-row tiles, where the
    // weight panels dominate and the row block is shared by every wave.
    static_assert(NW == 4 || NW == 8, "waves");
    static_assert(WGM == 1 || WGM == 2, "wave rows");
    constexpr int WGN = NW / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN, MB = WM / 32, NB = WN / 32;
    static_assert(MB >= 1 && NB >= 1, "wave tile");
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool SET = (MODE == kDownSet || MODE == kFc2Set);
    constexpr bool BNK = (MODE == kFc2 || MODE == kFc2Set || MODE == kFc2Rows);
    // KC: 16-bit weights stored K-contiguous ([N,K] per expert): Nomic's fc2
    // in the API layout, or every GEMM on pre-packed weights (PK)
    constexpr bool KC = BNK || PK;
    static_assert(!(W8 && PK), "fp8 codes are K-contiguous already");
    constexpr bool ROWS = (MODE == kDownRows || MODE == kFc2Rows);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    constexpr bool SWAP = !ATOMIC;
    static_assert(BK == 32 || BK == 64, "BK");
    constexpr int ACH = BK / 8;            // 16-byte chunks per K-contiguous row
    constexpr int AROW = BK * 2;           // bytes per K-contiguous row
    constexpr int RPA = 1024 / AROW;       // K-contiguous rows per DMA instruction
    constexpr int KSTEPS = BK / 16;
    constexpr int A_BYTES = BM * AROW;
    // W8: fp8 e4m3 weights, K-contiguous ([N,K] per expert, one byte per
    // element), each n-row of a B sub-tile BK bytes of KCH 16-byte chunks
    constexpr int KROW = BK;
    constexpr int KCH = KROW / 16;
    constexpr int KRPI = 1024 / KROW;  // fp8 n-rows per DMA instruction
    constexpr int B_BYTES = W8 ? BN * KROW : BN * AROW;
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
    static_assert(KC || BCH >= 8, "[K,N] tiles need >= 8 chunks per row for the swizzle");
    static_assert(KC || W8 || SUB_INS * NSUB == B_INS, "B tile split");
    // K-contiguous 16-bit sub-tiles (gate / up apart for DUAL): SUBN n-rows of
    // AROW bytes each
    constexpr int KSUB_BYTES = SUBN * AROW;
    constexpr int KSUB_INS = KSUB_BYTES / (1024 * NW);
    static_assert(!KC || (KSUB_INS * 1024 * NW == KSUB_BYTES && KSUB_INS * NSUB == B_INS), "K-contiguous B split");
    constexpr int W8_SUB_BYTES = SUBN * KROW;
    constexpr int W8_SUB_INS = W8_SUB_BYTES / (1024 * NW);
    static_assert(!W8 || (!BNK && KCH == 4 && W8_SUB_INS * 1024 * NW == W8_SUB_BYTES && W8_SUB_INS * NSUB == B_INS),
                  "fp8 B tile");
    static_assert(LOADS * (NST - 2) < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) char smem[NST * STAGE];
    __shared__ int32_t s_tok[(ATOMIC || SET) ? BM : 1];
    __shared__ float s_w[ATOMIC ? BM : 1];
    __shared__ float s_sc[W8 ? BN : 1];
    // fp8 expert sets: unit u_j[col] of segment j's column (its expert's
    // column scale, or 1 for an all-zero column), [kSetMaxK][BN]
    constexpr bool W8SET = W8 && SET;
    __shared__ __attribute__((aligned(16))) float s_unit[W8SET ? kSetMaxK * BN : 4];
    // staged (row-contiguous) epilogue of the large tiles, see staged_epilogue
    constexpr bool STAGED = SWAP && BM >= 128;
    static_assert(!STAGED || NST * STAGE >= BM * (DUAL ? BN / 2 : BN) * 2, "output tile fits the stages");
    __shared__ int32_t s_dst[STAGED ? BM : 1];

    // workgroup -> (output tile, K split); every workgroup first clears its
    // share of zero_f32 (the accumulator of the GEMM that follows)
    clear_share(a.zero_f32, a.zero_n);
    constexpr bool FIXUP = BM <= 32 || NW == 8;  // kernels that carry the split-K fixup
    int tile, ks, nsplit, fix_slot0, fix_ctr;
    if (FIXUP && a.tail_cus > 0) {
        if (!tail_item(*a.num_tiles * a.n_tiles, a.tail_cus, (a.K + BK - 1) / BK, tile, ks, nsplit, fix_slot0,
                       fix_ctr))
            return;
    } else {
        const int live = *a.num_tiles * a.n_tiles;
        nsplit = adaptive_split(a.ksplit, a.split_target, live, (a.K + BK - 1) / BK);
        const int lg = xcd_logical(live * nsplit);
        if (lg < 0) return;
        tile = lg / nsplit;
        ks = lg - tile * nsplit;
        fix_slot0 = tile * nsplit;
        fix_ctr = tile;
    }
    const int mt = tile / a.n_tiles, nt = tile - mt * a.n_tiles;
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
        n_seg = decode_set(grp, a.k_top, a.n_experts, seg_exp);
    } else {
        seg_exp[0] = grp;
    }
    const int K = SET ? n_seg * a.seg_len : a.K;
    const int a_pitch = SET ? a.k_top * a.seg_len : a.K;

    const i32x4 rA = make_rsrc(a.A, a.a_bytes);
    const uint32_t smem_base = __builtin_amdgcn_readfirstlane(lds_addr(smem));

    // ---- per-lane DMA offsets, fixed for the whole K loop (gathered row or
    // column chunk and the chunk's swizzled slot); the K position of a full
    // tile goes into the instruction's SGPR offset. A: instruction i of this
    // wave covers rows RPA*q .. RPA*q+RPA-1, q = NW*i + wave. Gathered rows
    // (gate/up, fc1) past the group's end (r >= m_valid) are not masked: row
    // i of a product depends on row i of A only and those rows are never
    // stored, and every load stays in range (the sorted-pair index is clamped
    // to the array; an A offset past a_bytes, or wrapped, reads zeros;
    // offsets stay multiples of 16 bytes), so the first DMA waits for the
    // tile table and the gather only, not for the group's end (offsets[grp +
    // 1]), loaded alongside. Contiguous rows (the other modes) need no gather
    // and stay masked (kOob lanes fetch nothing), which saves their
    // partly filled tiles the traffic of the rows past the group.
    uint32_t a_off[A_INS];
#pragma unroll
    for (int i = 0; i < A_INS; ++i) {
        const int r = RPA * (NW * i + wave) + lane / ACH;
        const int kc = a_swz<ACH>(r, lane % ACH) * 8;  // k offset of the chunk that lands at this lane's slot
        if constexpr (GATHER) {
            const int src = a.sorted_pair[min(r0 + r, a.sorted_n - 1)] / a.k_top;
            a_off[i] = ((uint32_t)src * (uint32_t)a_pitch + (uint32_t)kc) * 2u;
        } else {
            a_off[i] = r < m_valid ? ((uint32_t)(r0 + r) * (uint32_t)a_pitch + (uint32_t)kc) * 2u : kOob;
        }
    }
    // B [N,K]: like A over the column tile's rows n. B [K,N]: instruction i
    // (i % SUB_INS within sub-tile i / SUB_INS) covers k-rows RPI*q ..
    // RPI*q+RPI-1 of the tile, q = NW*(i % SUB_INS) + wave.
    uint32_t b_off[B_INS];
#pragma unroll
    for (int i = 0; i < B_INS; ++i) {
        if constexpr (W8) {
            // n-row r of sub-tile i / W8_SUB_INS; the lane's slot receives the
            // chunk a_swz(r, slot) of that row (byte offsets: one byte per k)
            const int q = NW * (i % W8_SUB_INS) + wave;
            const int r = KRPI * q + lane / KCH;
            const int n = nt * SUBN + r;
            const int kc = a_swz<KCH>(r, lane % KCH) * 16;
            b_off[i] = n < N ? (uint32_t)n * (uint32_t)a.ldb + (uint32_t)kc : kOob;
        } else if constexpr (KC) {
            // n-row r of sub-tile i / KSUB_INS (the only one unless DUAL)
            const int r = RPA * (NW * (i % KSUB_INS) + wave) + lane / ACH;
            const int n = nt * SUBN + r;
            const int kc = a_swz<ACH>(r, lane % ACH) * 8;
            b_off[i] = n < N ? ((uint32_t)n * (uint32_t)a.ldb + (uint32_t)kc) * 2u : kOob;
        } else {
            const int q = NW * (i % SUB_INS) + wave;
            const int r = RPI * q + lane / BCH;
            const int c = kn_swz<BCH>(r, lane % BCH);
            const int col = nt * SUBN + c * 8;
            b_off[i] = col < N ? ((uint32_t)col + (uint32_t)r * (uint32_t)a.ldb) * 2u : kOob;
        }
    }

    // fp8 weights: this thread's column scale of the tile (256 threads, 256
    // columns: gate then up for kGateUp), loaded now, staged in LDS for the
    // epilogue after the K loop
    float sc_pre = 1.0f;
    if constexpr (W8 && !SET) {
        static_assert(BN <= 64 * NW, "one scale per thread");
        const int c = DUAL ? nt * SUBN + tid % SUBN : nt * BN + tid;
        const float* src = (DUAL && tid >= SUBN) ? a.scale1 : a.scale0;
        if (tid < BN && c < N) sc_pre = src[(long long)grp * N + c];
    }

    // Weight buffer resources of the current expert; on the expert-set path
    // the expert changes every seg_len of K (tracked as K advances, issue
    // calls come in increasing k0).
    int seg = 0, seg_k0 = 0;
    auto weights_rsrc = [&](int e, i32x4& r0s, i32x4& r1s) {
        constexpr int BES = W8 ? 1 : 2;  // bytes per weight element
        const long long eoff = (long long)e * a.strideB * BES;
        r0s = make_rsrc(reinterpret_cast<const char*>(a.B0) + eoff, a.strideB * BES);
        r1s = r0s;
        if constexpr (DUAL) r1s = make_rsrc(reinterpret_cast<const char*>(a.B1) + eoff, a.strideB * BES);
    };
    i32x4 rB0, rB1;
    weights_rsrc(seg_exp[0], rB0, rB1);

    // DMA instructions lo .. hi-1 of this wave's LOADS for the tile at k0
    // (A instructions first, then B).
    auto issue_range = [&](int stage, int k0, int lo, int hi) {
        const uint32_t sA = smem_base + stage * STAGE;
        const uint32_t sB = sA + A_BYTES;
        int kk = k0, klim = K;
        if constexpr (SET) {
            if (k0 >= seg_k0 + a.seg_len) {
                while (k0 >= seg_k0 + a.seg_len) {
                    ++seg;
                    seg_k0 += a.seg_len;
                }
                weights_rsrc(seg_exp[seg < kSetMaxK ? seg : 0], rB0, rB1);
            }
            kk = k0 - seg_k0;
            klim = a.seg_len;
        }
        // a tile that lies inside the operands in K takes the SGPR-offset path;
        // a K tail checks every lane's chunk against K
        const uint32_t sa = (uint32_t)k0 * 2u;
        const uint32_t sb = W8 ? (uint32_t)kk : (KC ? (uint32_t)kk * 2u : (uint32_t)kk * (uint32_t)a.ldb * 2u);
        if (k0 + BK <= K && kk + BK <= klim) {
            // the tile lies inside the operands in K: one SGPR offset for all lanes
#pragma unroll
            for (int i = 0; i < A_INS; ++i)
                if (i >= lo && i < hi) dma16s(rA, sA + (NW * i + wave) * 1024, a_off[i], sa);
#pragma unroll
            for (int i = 0; i < B_INS; ++i) {
                if (A_INS + i < lo || A_INS + i >= hi) continue;
                if constexpr (W8) {
                    const int sub = i / W8_SUB_INS;
                    dma16s(sub ? rB1 : rB0, sB + sub * W8_SUB_BYTES + (NW * (i % W8_SUB_INS) + wave) * 1024, b_off[i],
                           sb);
                } else if constexpr (KC) {
                    const int sub = i / KSUB_INS;
                    dma16s(sub ? rB1 : rB0, sB + sub * KSUB_BYTES + (NW * (i % KSUB_INS) + wave) * 1024, b_off[i], sb);
                } else {
                    const int sub = i / SUB_INS;  // compile-time after unrolling
                    dma16s(sub ? rB1 : rB0, sB + sub * SUB_BYTES + (NW * (i % SUB_INS) + wave) * 1024, b_off[i], sb);
                }
            }
        } else {
            // K tail: every lane's chunk is checked against the operand's K
#pragma unroll
            for (int i = 0; i < A_INS; ++i) {
                if (i < lo || i >= hi) continue;
                const int r = RPA * (NW * i + wave) + lane / ACH;
                const bool in = k0 + a_swz<ACH>(r, lane % ACH) * 8 < K;
                dma16s(rA, sA + (NW * i + wave) * 1024, in ? a_off[i] : kOob, sa);
            }
#pragma unroll
            for (int i = 0; i < B_INS; ++i) {
                if (A_INS + i < lo || A_INS + i >= hi) continue;
                if constexpr (W8) {
                    // (K is a multiple of 16: a chunk lies wholly inside or outside)
                    const int sub = i / W8_SUB_INS;
                    const int r = KRPI * (NW * (i % W8_SUB_INS) + wave) + lane / KCH;
                    const bool in = kk + a_swz<KCH>(r, lane % KCH) * 16 < klim;
                    dma16s(sub ? rB1 : rB0, sB + sub * W8_SUB_BYTES + (NW * (i % W8_SUB_INS) + wave) * 1024,
                           in ? b_off[i] : kOob, sb);
                } else if constexpr (KC) {
                    const int sub = i / KSUB_INS;
                    const int r = RPA * (NW * (i % KSUB_INS) + wave) + lane / ACH;
                    const bool in = kk + a_swz<ACH>(r, lane % ACH) * 8 < klim;
                    dma16s(sub ? rB1 : rB0, sB + sub * KSUB_BYTES + (NW * (i % KSUB_INS) + wave) * 1024,
                           in ? b_off[i] : kOob, sb);
                } else {
                    const int sub = i / SUB_INS;
                    const bool in = kk + RPI * (NW * (i % SUB_INS) + wave) + lane / BCH < klim;
                    dma16s(sub ? rB1 : rB0, sB + sub * SUB_BYTES + (NW * (i % SUB_INS) + wave) * 1024,
                           in ? b_off[i] : kOob, sb);
                }
            }
        }
    };
    auto issue = [&](int stage, int k0) { issue_range(stage, k0, 0, LOADS); };

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
            if constexpr (KC) {
                // DUAL: block nb is gate (even) or up (odd) of logical
                // columns wn*WN/2 + (nb/2)*32 of the tile
                const int sub = DUAL ? (nb & 1) : 0;
                const int r = (DUAL ? wn * (WN / 2) + (nb >> 1) * 32 : wn * WN + nb * 32) + lr;
                bfr[nb] = *reinterpret_cast<const u32x4*>(sB + sub * KSUB_BYTES + r * AROW + a_swz<ACH>(r, c) * 16);
            } else {
                const int p = b_tr_col[nb];
                const int kr = kk * 16 + tr_k;  // kr & 3 == (tj >> 2); kr + 4 keeps the swizzle
                const int cc = kn_swz<BCH>(kr, p >> 3);
                const char* base = sB + (DUAL ? (nb & 1) * SUB_BYTES : 0) + cc * 16 + (p & 7) * 2;
                bfr[nb] = tr_pair(base + kr * BROW, base + (kr + 4) * BROW);
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
    // fp8 expert sets: per-column unit changes of the accumulators. Lane l
    // holds, for block nb and register group g, columns wn*WN + nb*32 + 8g +
    // 4(l/32) .. +3 (the swapped MFMA layout), the same for every mb.
    auto scale_acc = [&](auto&& factor4) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = wn * WN + nb * 32 + 8 * g + 4 * lh;
                const f32x4 f = factor4(col);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) acc[mb][nb][4 * g + jj] *= f[jj];
            }
    };
    auto rescale_units = [&](int j) {
        scale_acc([&](int col) {
            const f32x4 up = *reinterpret_cast<const f32x4*>(s_unit + (j - 1) * BN + col);
            const f32x4 un = *reinterpret_cast<const f32x4*>(s_unit + j * BN + col);
            // reciprocal to ~1 ulp: the units cancel to that accuracy in
            // the end, far below the fp8 codes' own rounding
            return f32x4{up[0] * __builtin_amdgcn_rcpf(un[0]), up[1] * __builtin_amdgcn_rcpf(un[1]),
                         up[2] * __builtin_amdgcn_rcpf(un[2]), up[3] * __builtin_amdgcn_rcpf(un[3])};
        });
    };
    auto to_absolute = [&](int j) {
        scale_acc([&](int col) { return *reinterpret_cast<const f32x4*>(s_unit + j * BN + col); });
    };
    // LDS read instructions per k16 step (ds_read_b128 for A and [N,K] B,
    // two ds_read_b64_tr_b16 per [K,N] B block).
    constexpr int DS_PER_STEP = MB + ((KC || W8) ? NB : 2 * NB);
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
    // 8 waves: the waves of row group 1 issue the whole DMA of the next tile
    // after their first k16 step's MFMAs (ds >= 0 only for them), so that the
    // two waves sharing a SIMD do not both stall on the memory pipeline right
    // after the barrier (2 % on the prefill GEMMs; issuing later leaves the
    // DMA too little time before the next barrier).
    auto dma_slice = [&](int ds, int dk, int step) {
        if constexpr (NW == 8) {
            if (step == 0 && ds >= 0) issue_range(ds, dk, 0, LOADS);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // A wave whose rows all lie past the group's end (the last row tile of a
    // group) reads no fragments and issues no MFMAs; it still issues its DMA
    // share and meets every barrier. On a half-empty tile this leaves the
    // matrix core of each SIMD to the other wave.
    // (one wave row: every wave holds the tile's rows, and m_valid >= 1; as a
    // constant the compiler keeps the accumulators in place across the loop)
    const bool rows_live = WGM == 1 || wm * WM < m_valid;
    // fp8 weights: all LDS reads of a stage first (A fragments and the raw
    // fp8 bytes of every k16 step), then per step the conversion and the
    // MFMAs, so that the LDS latency of later steps runs under the
    // conversions and MFMAs of earlier ones (converting right after each read
    // serialises read, wait, conversion and MFMA step by step).
    auto compute_w8 = [&](int stage) {
        if (!rows_live) return;
        const char* sA = smem + stage * STAGE;
        const char* sB = sA + A_BYTES;
        u32x4 af[KSTEPS][MB];
        u32x2 braw[KSTEPS][NB];
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
            const int c = kk * 2 + lh;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int r = a_frag_row[mb];
                af[kk][mb] = *reinterpret_cast<const u32x4*>(sA + r * AROW + a_swz<ACH>(r, c) * 16);
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int sub = DUAL ? (nb & 1) : 0;
                const int r = DUAL ? wn * (WN / 2) + (nb >> 1) * 32 + lr : wn * WN + nb * 32 + lr;
                // 8 fp8 weights: k = 16 kk + 8 lh .. +7 of n-row r
                braw[kk][nb] = *reinterpret_cast<const u32x2*>(sB + sub * W8_SUB_BYTES + r * KROW +
                                                                a_swz<KCH>(r, kk) * 16 + lh * 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // every read issued before the first conversion
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
            u32x4 bfr[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) bfr[nb] = fp8x8_to<DT>(braw[kk][nb]);  // exact in DT
            mfma_step(af[kk], bfr);
        }
    };
    // fp8 weights on the 8-wave kernel: the 16-bit loop's schedule (two
    // register sets, one LDS read per MFMA); each B block is read as the
    // lane's 8 raw code bytes (one ds_read_b64, half the 16-bit block's bytes)
    // and converted right before its step's MFMAs
    auto load_w8 = [&](const char* sA, const char* sB, int kk, u32x4 (&af)[MB], u32x2 (&br)[NB]) {
        const int c = kk * 2 + lh;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int r = a_frag_row[mb];
            af[mb] = *reinterpret_cast<const u32x4*>(sA + r * AROW + a_swz<ACH>(r, c) * 16);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int sub = DUAL ? (nb & 1) : 0;
            const int r = DUAL ? wn * (WN / 2) + (nb >> 1) * 32 + lr : wn * WN + nb * 32 + lr;
            br[nb] = *reinterpret_cast<const u32x2*>(sB + sub * W8_SUB_BYTES + r * KROW + a_swz<KCH>(r, kk) * 16 +
                                                     lh * 8);
        }
    };
    auto compute_w8i = [&](int stage, int ds, int dk) {
        if (!rows_live) {
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) dma_slice(ds, dk, st);
            return;
        }
        const char* sA = smem + stage * STAGE;
        const char* sB = sA + A_BYTES;
        u32x4 af0[MB], af1[MB], bfr[NB];
        u32x2 br0[NB], br1[NB];
        auto cvt = [&](const u32x2 (&br)[NB]) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) bfr[nb] = fp8x8_to<DT>(br[nb]);  // exact in DT
        };
        load_w8(sA, sB, 0, af0, br0);
        __builtin_amdgcn_sched_barrier(0);
        load_w8(sA, sB, 1, af1, br1);
        cvt(br0);
        mfma_step(af0, bfr);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, 0);
        load_w8(sA, sB, 2, af0, br0);
        cvt(br1);
        mfma_step(af1, bfr);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, 1);
        load_w8(sA, sB, 3, af1, br1);
        cvt(br0);
        mfma_step(af0, bfr);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, 2);
        cvt(br1);
        mfma_step(af1, bfr);
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, KSTEPS - 1);
    };
    auto compute = [&](int stage, int ds, int dk) {
        if (!rows_live) {
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) dma_slice(ds, dk, st);
            return;
        }
        const char* sA = smem + stage * STAGE;
        const char* sB = sA + A_BYTES;
        u32x4 af0[MB], bf0[NB], af1[MB], bf1[NB];
        load_frags(sA, sB, 0, af0, bf0);
        __builtin_amdgcn_sched_barrier(0);
        load_frags(sA, sB, 1, af1, bf1);
        mfma_step(af0, bf0);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, 0);
        if constexpr (KSTEPS == 4) {
            load_frags(sA, sB, 2, af0, bf0);
            mfma_step(af1, bf1);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
            dma_slice(ds, dk, 1);
            load_frags(sA, sB, 3, af1, bf1);
            mfma_step(af0, bf0);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
            dma_slice(ds, dk, 2);
        }
        mfma_step(af1, bf1);
        __builtin_amdgcn_sched_barrier(0);
        dma_slice(ds, dk, KSTEPS - 1);
    };

    if constexpr (ATOMIC) {
        if (tid < BM) {
            const int p = a.sorted_pair[r0 + (tid < m_valid ? tid : 0)];
            s_tok[tid] = p / a.k_top;
            s_w[tid] = a.routing_w[p];
        }
    }
    // expert-set down / fc2: the output row (token) of every tile row, staged
    // in LDS now (no registers to spare) for the epilogue
    if constexpr (W8SET) {
        // loaded next to s_tok's rows, whose wait the DMA waits for anyway
        if (tid < BN) {
            const int c = nt * BN + tid;
            for (int j = 0; j < n_seg; ++j) {
                const float sj = c < N ? a.scale0[(long long)seg_exp[j] * N + c] : 0.0f;
                s_unit[j * BN + tid] = sj > 0.0f ? sj : 1.0f;
            }
        }
    }
    if constexpr (SET) {
        if (tid < BM) s_tok[tid] = a.tok_sorted[r0 + (tid < m_valid ? tid : 0)];
    }
    // gate/up, fc1: the epilogue's output rows and routing weights (two
    // dependent reads per row), loaded now so that they are long done when the
    // K loop ends.
    // (pair-row down / fc2: the row's pair and its routing weight)
    int pre_dst[MB];
    float pre_w[MB];
    if constexpr (GATHER || ROWS) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = wm * WM + mb * 32 + (lane & 31);
            const int r = r0 + (ml < m_valid ? ml : 0);
            const int p = a.sorted_pair[r];
            if constexpr (ROWS) {
                pre_dst[mb] = p;
                pre_w[mb] = a.routing_w[p];
            } else {
                pre_dst[mb] = a.pair_dest ? a.pair_dest[p] : r;
                pre_w[mb] = a.fold_w ? a.routing_w[p] : 1.0f;
            }
        }
    }

    // Stage hand-over, one barrier per K tile: wait for this wave's DMA of
    // stage kt (the NST-2 newer stages may stay in flight) and for its own
    // LDS reads of stage kt-1, then the barrier makes both block-wide; only
    // after it is stage kt-1's slot refilled with tile kt+NST-1.
    // this split's K tiles: [kt0, kt0 + nk) of nk_all
    const int nk_all = (K + BK - 1) / BK;
    const int per_split = (nk_all + nsplit - 1) / nsplit;
    const int kt0 = min(nk_all, ks * per_split);
    const int nk = min(nk_all, kt0 + per_split) - kt0;

    if constexpr (NW == 4 && !GATHER && !W8) {
        // 4-wave down / fc2 kernels: hand-over one k16 step early. The
        // barrier of tile kt+1 sits before the MFMAs of tile kt's last k16
        // step, whose fragments are already in registers, so the MFMAs issued
        // before the barrier keep the matrix cores busy while the waves meet,
        // and the first fragments of tile kt+1 are read while the last step's
        // MFMAs run. Measured: Nomic T=4096 fc2 (expert sets, 128x256 tile) 120 ->
        // 107 us; the gathering gate/up / fc1 GEMMs got 2-5 % slower and the
        // 8-wave kernels, whose second wave per SIMD covers those reads,
        // moved within 1.5 % either way: they keep the loop below.
        //   [tile kt: steps 0 .. KSTEPS-2, fragments of the next step read
        //    under each step's MFMAs] -> wait for this wave's DMA of tile kt+1
        //   and its LDS reads of tile kt -> barrier -> DMA of tile kt+NST into
        //   tile kt's slot -> fragments of tile kt+1 step 0 under the MFMAs of
        //   tile kt's last step.
        // wait for the DMA of the tile with `newer` of this wave's tiles
        // issued after it
        auto wait_tile = [&](int newer) { wait_stage<LOADS, NST - 2>(newer); };
        u32x4 af0[MB], bf0[NB], af1[MB], bf1[NB];
#pragma unroll
        for (int s = 0; s < NST - 1; ++s)
            if (s < nk) issue(s, (kt0 + s) * BK);
        if (nk > 0) {
            wait_tile(min(NST - 2, nk - 1));
            wait_lgkm0();
            block_barrier();
            if (NST - 1 < nk) issue(NST - 1, (kt0 + NST - 1) * BK);
            if (rows_live) load_frags(smem, smem + A_BYTES, 0, af0, bf0);
        }
        for (int kt = 0; kt < nk; ++kt) {
            const int st = kt % NST;
            const char* sA = smem + st * STAGE;
            const char* sB = sA + A_BYTES;
            if (rows_live) {
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
            }
            wait_tile(kt + 1 < nk ? min(NST - 2, nk - 2 - kt) : 0);
            wait_lgkm0();
            block_barrier();
            const int nx = kt + NST;
            if (nx < nk) issue(st, (kt0 + nx) * BK);
            if (rows_live) {
                // (the last tile reads a stale stage: in bounds, unused)
                const char* nA = smem + ((kt + 1) % NST) * STAGE;
                load_frags(nA, nA + A_BYTES, 0, af0, bf0);
                mfma_step(af1, bf1);
                interleave();
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
    // fp8 expert sets: segment of the split's first K tile, and the K tile
    // at which the next one starts (segments are seg_kt whole K tiles)
    const int seg_kt = W8SET ? a.seg_len / BK : 1;
    int seg_cur = W8SET ? kt0 / seg_kt : 0;
    int seg_next = W8SET ? (seg_cur + 1) * seg_kt : 0;
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < nk) issue(s, (kt0 + s) * BK);
    for (int kt = 0; kt < nk; ++kt) {
        const int newer = min(NST - 2, nk - 1 - kt);  // stages issued after kt and before this wait
        wait_stage<LOADS, NST - 2>(newer);
        wait_lgkm0();
        block_barrier();
        const int ahead = kt + NST - 1;
        // row group 1 issues after its first k16 step (the decode kernels'
        // compute_w8 has no DMA slot)
        const bool late = NW == 8 && (!W8 || KSTEPS == 4) && wm == 1;
        if (ahead < nk && !late) issue(ahead % NST, (kt0 + ahead) * BK);
        if constexpr (W8SET) {
            // fp8 expert sets: the accumulators hold the current segment's
            // column units; entering segment j they are rescaled by
            // u_{j-1} / u_j (the K tiles of a segment never straddle one:
            // seg_len is a multiple of BK)
            if (kt0 + kt == seg_next) {
                if (kt > 0 && rows_live) rescale_units(seg_cur + 1);
                ++seg_cur;
                seg_next += seg_kt;
            }
        }
        if constexpr (W8 && NW == 8 && KSTEPS == 4)
            compute_w8i(kt % NST, (late && ahead < nk) ? ahead % NST : -1, (kt0 + ahead) * BK);
        else if constexpr (W8) compute_w8(kt % NST);
        else compute(kt % NST, (late && ahead < nk) ? ahead % NST : -1, (kt0 + ahead) * BK);
    }
    }

    if constexpr (W8SET) {
        // to absolute values: the unit of the segment of this split's last K tile
        if (rows_live && nk > 0) to_absolute(((kt0 + nk - 1) * BK) / a.seg_len);
    }
    if constexpr (FIXUP) {
        // split K: the last split to finish a tile sums all partials in split
        // order and alone runs the epilogue (one atomic per output element and
        // pair, as without splits: the result does not depend on the order in
        // which splits finish)
        // loads in flight per batch: the atomic-combine kernels keep their
        // row table in registers and have less room
        constexpr int FIX_BATCH = (ATOMIC || MB * NB < 2) ? 4 : 8;
        if (nsplit > 1 &&
            !splitk_fixup<MB, NB, NW, FIX_BATCH, (BM <= 32)>(a, acc, fix_slot0, fix_ctr, ks, nsplit, wave, lane))
            return;
    }
    // fp8 weights: the tile's column scales, staged in LDS
    const float* sc0 = nullptr;
    const float* sc1 = nullptr;
    if constexpr (W8 && !SET) {
        if (tid < BN) s_sc[tid] = sc_pre;
        __syncthreads();
        sc0 = s_sc;
        if constexpr (DUAL) sc1 = s_sc + SUBN;
    }
    if constexpr (STAGED) {
        if (!SET || a.overwrite) {
            // output row of every tile row (gate/up, fc1: the pair's inter row;
            // pair rows: the pair; expert sets: the token, already in s_tok)
            if constexpr (GATHER || ROWS) {
                if (wn == 0 && lane < 32) {
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) s_dst[wm * WM + mb * 32 + lane] = pre_dst[mb];
                }
            }
            __syncthreads();  // every wave is done with the stages
            staged_epilogue<DT, MODE, BM, BN, WM, WN, MB, NB, NW, W8 && !SET>(a, acc, smem, SET ? s_tok : s_dst,
                                                                             m_valid, nt, wm, wn, lane, pre_w, sc0,
                                                                             sc1);
            return;
        }
        if constexpr (SET && BN == 256 && NST * STAGE >= BM * (BN / 2) * 4) {
            __syncthreads();  // every wave is done with the stages
            staged_epilogue_acc<DT, BM, BN, WM, WN, MB, NB, NW>(a, acc, smem, s_tok, m_valid, nt, wm, wn, lane);
            return;
        }
    }
    tile_epilogue<DT, MODE, BN, WM, WN, MB, NB>(a, acc, r0, m_valid, nt, wm, wn, lane, s_tok, s_w,
                                                (GATHER || ROWS) ? pre_dst : nullptr,
                                                (GATHER || ROWS) ? pre_w : nullptr, sc0, sc1);
}

template <int DT, int MODE, bool PK>
hipError_t launch_lds_mode(int cfg, const GemmArgs& a, hipStream_t stream) {
    // one workgroup per (row tile, column tile, K split)
    // tail balance: each XCD's range plus up to tail_cus split workgroups
    const long long tiles = (long long)a.m_tiles_max * a.n_tiles;
    const long long nwg_l = a.tail_cus > 0 ? 8 * ((tiles + 7) / 8 + a.tail_cus)
                                           : split_grid(tiles, a);
    if (nwg_l > 0x7fffffffLL) return hipErrorInvalidValue;
    const int nwg = (int)nwg_l;
    if (nwg <= 0) return hipSuccess;
    if constexpr (DT == kF32) {
        return hipErrorInvalidValue;
    } else {
        switch (cfg) {
            case kLds128:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 128, 128, 64, 4, 4, MODE, 2, 1, false, PK>), dim3(nwg), dim3(256),
                                   0, stream, a);
                break;
            case kLds256w8:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 64, 2, 8, MODE, 2, 1, false, PK>), dim3(nwg), dim3(512),
                                   0, stream, a);
                break;
            case kLdsRows32:
                if constexpr (MODE == kDown || MODE == kFc2 || MODE == kFc1) {
                    if (a.narrow) {
                        hipLaunchKernelGGL((moe_lds_gemm<DT, 32, 128, 64, 4, 4, MODE, 1, 1, false, PK>), dim3(nwg),
                                           dim3(256), 0, stream, a);
                        break;
                    }
                }
                hipLaunchKernelGGL((moe_lds_gemm<DT, 32, 256, 64, 4, 4, MODE, 1, 1, false, PK>), dim3(nwg), dim3(256),
                                   0, stream, a);
                break;
            // two workgroups per CU (72 KB of LDS, at most 256 VGPRs each): one
            // workgroup's barrier and DMA issue overlap the other's MFMAs
            case kLds128x256o2:
                hipLaunchKernelGGL((moe_lds_gemm<DT, 128, 256, 32, 3, 4, MODE, 2, 2, false, PK>), dim3(nwg),
                                   dim3(256), 0, stream, a);
                break;
            default:
                return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

// fp8-weight GEMMs, pair-path modes only: the 32-row kernel (decode; down /
// fc2 also on 128-column tiles, a.narrow) or the
// 8-wave 256x256 kernel with 3 LDS stages (48 KB each: the fp8 B tile is half
// the 16-bit one) for larger batches
template <int DT, int MODE>
static hipError_t launch_w8_mode(int cfg, const GemmArgs& a, hipStream_t stream) {
    const long long tiles = (long long)a.m_tiles_max * a.n_tiles;
    if (cfg == kLds256w8) {
        if constexpr (MODE == kGateUp || MODE == kFc1 || MODE == kDownRows || MODE == kDownSet) {
            const long long nwg = a.tail_cus > 0 ? 8 * ((tiles + 7) / 8 + a.tail_cus) : tiles;
            if (nwg > 0x7fffffffLL) return hipErrorInvalidValue;
            if (nwg <= 0) return hipSuccess;
            hipLaunchKernelGGL((moe_lds_gemm<DT, 256, 256, 64, 3, 8, MODE, 2, 1, true>), dim3((int)nwg), dim3(512), 0,
                               stream, a);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    if (cfg != kLdsRows32) return hipErrorInvalidValue;
    const long long nwg_l = split_grid(tiles, a);
    if (nwg_l > 0x7fffffffLL) return hipErrorInvalidValue;
    if (nwg_l <= 0) return hipSuccess;
    // 4 LDS stages of 20 KB, one workgroup per CU (6 or 7 stages, and two
    // workgroups per CU, measured slower)
    constexpr int kW8Nst = 4, kW8Occ = 1;
    if constexpr (MODE == kDown || MODE == kFc1) {
        if (a.narrow) {  // 128-column tiles (n_tiles counts those)
            hipLaunchKernelGGL((moe_lds_gemm<DT, 32, 128, 64, kW8Nst, 4, MODE, 1, kW8Occ, true>),
                               dim3((int)nwg_l), dim3(256), 0, stream, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((moe_lds_gemm<DT, 32, 256, 64, kW8Nst, 4, MODE, 1, kW8Occ, true>), dim3((int)nwg_l),
                       dim3(256), 0, stream, a);
    return hipGetLastError();
}
template <int DT>
static hipError_t launch_w8_dt(int mode, int cfg, const GemmArgs& a, hipStream_t stream) {
    // [N,K] fp8 weights for every GEMM: fc2 (Nomic) runs the down kernels
    switch (mode) {
        case kGateUp: return launch_w8_mode<DT, kGateUp>(cfg, a, stream);
        case kFc1: return launch_w8_mode<DT, kFc1>(cfg, a, stream);
        case kDown: return launch_w8_mode<DT, kDown>(cfg, a, stream);
        case kFc2: return launch_w8_mode<DT, kDown>(cfg, a, stream);
        case kDownRows: return launch_w8_mode<DT, kDownRows>(cfg, a, stream);
        case kFc2Rows: return launch_w8_mode<DT, kDownRows>(cfg, a, stream);
        case kDownSet: return launch_w8_mode<DT, kDownSet>(cfg, a, stream);
        case kFc2Set: return launch_w8_mode<DT, kDownSet>(cfg, a, stream);
        default: return hipErrorInvalidValue;
    }
}
hipError_t launch_moe_gemm_w8(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream) {
    if (cfg == kW8Gemv) return launch_w8_gemv(mode, dtype, a, stream);
    if (dtype == kBF16) return launch_w8_dt<kBF16>(mode, cfg, a, stream);
    if (dtype == kF16) return launch_w8_dt<kF16>(mode, cfg, a, stream);
    return hipErrorInvalidValue;
}

template <int DT, bool PK>
static hipError_t launch_lds_dt(int mode, int cfg, const GemmArgs& a, hipStream_t stream) {
    // (pre-packed weights: every B is [N,K]; Nomic's fc2 is [N,K] either
    // way, so its modes need no packed instances)
    switch (mode) {
        case kGateUp: return launch_lds_mode<DT, kGateUp, PK>(cfg, a, stream);
        case kFc1: return launch_lds_mode<DT, kFc1, PK>(cfg, a, stream);
        case kDown: return launch_lds_mode<DT, kDown, PK>(cfg, a, stream);
        case kFc2: return launch_lds_mode<DT, kFc2, false>(cfg, a, stream);
        case kDownSet: return launch_lds_mode<DT, kDownSet, PK>(cfg, a, stream);
        case kFc2Set: return launch_lds_mode<DT, kFc2Set, false>(cfg, a, stream);
        case kDownRows: return launch_lds_mode<DT, kDownRows, PK>(cfg, a, stream);
        case kFc2Rows: return launch_lds_mode<DT, kFc2Rows, false>(cfg, a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_gemm_lds(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream) {
    if (dtype == kBF16) return a.packed ? launch_lds_dt<kBF16, true>(mode, cfg, a, stream)
                                        : launch_lds_dt<kBF16, false>(mode, cfg, a, stream);
    if (dtype == kF16) return a.packed ? launch_lds_dt<kF16, true>(mode, cfg, a, stream)
                                       : launch_lds_dt<kF16, false>(mode, cfg, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
