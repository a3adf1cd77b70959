// Expert-grouped GEMMs of the fused MoE layer.
//
// Four products, one per GemmMode (/root/reference/kernels/moe.cu:193-449 for
// the f32 reference kernels, /root/reference/kernels/qwen3_moe.cu and
// nomic_moe.cu for the 16-bit ones):
//   kGateUp  Qwen3 gate+up : inter[r] = act(x_t . G_e) * (x_t . U_e)
//   kFc1     Nomic fc1     : inter[r] = act(x_t . G_e)
//   kDown    Qwen3 down    : acc[t]  += w_p * (inter[r] . D_e)
//   kFc2     Nomic fc2     : acc[t]  += w_p * (inter[r] . U_e^T)
// where r runs over expert-sorted pairs p = t*k + j of expert e and acc is
// an f32 [T,N] accumulator that a final pass adds to the caller's output.
// Expert-set path (few distinct expert sets, e.g. E=8, k=2): tokens are
// grouped by the sorted set of their k experts, GEMM1 writes w_p * h for
// pair p into slot rank(j) of its token's row of inter [T, k*I], and
//   kDownSet / kFc2Set : out[t] += [w h_1 | .. | w h_k] . [B_e1; ..; B_ek]
//                        (out[t] = ... with a.overwrite)
// one GEMM over K = k*I whose weight block switches expert every I rows, so
// each output row is written exactly once: no atomics, no f32 accumulator.
//
// moe_mfma_gemm (bf16 / f16): 256 threads = 4 waves in a 2x2 layout, block
// tile BM x BN, K staged 64 at a time through a 2-stage LDS ring.
//  * A rows are gathered per tile row (token of the pair) with 16-byte loads.
//  * Weights stored [K,N] (N contiguous) are loaded as 8x8 blocks and
//    transposed in registers with v_perm_b32 so LDS holds every operand
//    K-contiguous; [N,K] weights (Nomic fc2) are copied as they are.
//  * LDS rows are 128 B with an XOR swizzle of the 16-byte chunk index by
//    row bits [2:0] and [5:3], so fragment reads and transposed writes hit
//    distinct banks.
//  * v_mfma_f32_32x32x16_{bf16,f16}. For stores the weight fragment is the
//    MFMA A operand, so each lane owns 4 consecutive output columns of one
//    row (one 8-byte store); for the f32 atomics the operands stay in order,
//    so a register of the wave spans 32 consecutive columns (coalesced).
//  * gate and up column blocks are interleaved every 32 columns, so the
//    SwiGLU product is formed in registers.
//  * Workgroup ids are remapped so each XCD walks a contiguous range of
//    tiles, column tiles of one row tile adjacent (A reuse in that XCD's L2).
// moe_simt_gemm: f32 (and any shape the MFMA path does not take), 64x64
// tiles with 4x4 outputs per thread.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

constexpr int kBK = 64;  // K elements per LDS stage

__device__ __forceinline__ int swz(int row, int c) { return row * 128 + (((c ^ row ^ (row >> 3)) & 7) << 4); }

__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int DT, int BM, int BN, int MODE>
__global__ __launch_bounds__(256, 1) void moe_mfma_gemm(GemmArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2, MB = WM / 32, NB = WN / 32;
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool SET = (MODE == kDownSet || MODE == kFc2Set);
    constexpr bool BNK = (MODE == kFc2 || MODE == kFc2Set);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    // ATOMIC epilogues keep the MFMA operands unswapped, so one register of a
    // wave covers 32 consecutive output columns of 2 rows (coalesced atomics);
    // the others swap them, so a lane owns 4 consecutive columns of one row.
    constexpr bool SWAP = !ATOMIC;
    constexpr int A_ITEMS = BM * 8 / 256;
    constexpr int B_ITEMS = BNK ? (BN * 8 / 256) : ((BN + 255) / 256);  // 16-B chunks or 8x8 blocks
    constexpr int B_REGS = BNK ? B_ITEMS : B_ITEMS * 8;
    constexpr int STAGE = (BM + BN) * 128;
    static_assert(!DUAL || (WN % 64) == 0, "gate/up pairs must stay inside one wave");
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
    __shared__ int32_t s_tok[ATOMIC ? BM : 1];
    __shared__ float s_w[ATOMIC ? BM : 1];

    int mt, nt;
    if (!tile_coords(a.n_tiles, *a.num_tiles, mt, nt)) return;
    const int r0 = a.tile_row[mt];
    const int grp = a.tile_exp[mt];  // expert, or expert-set key
    const int m_valid = min(BM, a.offsets[grp + 1] - r0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int N = a.N;

    // Experts feeding this tile: one, or the k digits of the set key (ascending;
    // digit E marks a dropped slot and sorts last, so only the first n_seg count).
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
    const int K = SET ? n_seg * a.seg_len : a.K;          // reduction length of this tile
    const int a_pitch = SET ? a.k_top * a.seg_len : a.K;  // A row pitch

    const uint16_t* Ab = reinterpret_cast<const uint16_t*>(a.A);
    const uint16_t* B0 = reinterpret_cast<const uint16_t*>(a.B0);
    const uint16_t* B1 = reinterpret_cast<const uint16_t*>(a.B1);

    // A: thread owns chunk (tid & 7) of rows (tid >> 3) + 32 i.
    const int a_c = tid & 7;
    long long a_off[A_ITEMS];
#pragma unroll
    for (int i = 0; i < A_ITEMS; ++i) {
        const int r = (tid >> 3) + 32 * i;
        const int rr = r < m_valid ? r : 0;
        if constexpr (GATHER) {
            const int tok = a.sorted_pair[r0 + rr] / a.k_top;
            a_off[i] = (long long)tok * a_pitch;
        } else {
            a_off[i] = (long long)(r0 + rr) * a_pitch;
        }
    }
    if constexpr (ATOMIC) {
        if (tid < BM) {
            const int p = a.sorted_pair[r0 + (tid < m_valid ? tid : 0)];
            s_tok[tid] = p / a.k_top;
            s_w[tid] = a.routing_w[p];
        }
    }
    // B: element offsets inside one expert's matrix (k offset added per stage).
    long long b_off[B_ITEMS];
    bool b_ok[B_ITEMS], b_up[B_ITEMS];
    int b_kb[B_ITEMS], b_q[B_ITEMS];
#pragma unroll
    for (int i = 0; i < B_ITEMS; ++i) {
        const int item = tid + 256 * i;
        b_up[i] = false;
        if constexpr (BNK) {
            const int row = item >> 3, c = item & 7;
            const int col = nt * BN + row;
            b_ok[i] = col < N;
            b_off[i] = (long long)(b_ok[i] ? col : 0) * a.ldb + c * 8;
            b_kb[i] = c;
            b_q[i] = row;
        } else {
            const int q = item % (BN / 8), kb = item / (BN / 8);
            const int nr = q * 8;
            int col;
            if constexpr (DUAL) {
                col = nt * (BN / 2) + (nr >> 6) * 32 + (nr & 31);
                b_up[i] = ((nr >> 5) & 1) != 0;
            } else {
                col = nt * BN + nr;
            }
            b_ok[i] = (item < BN) && (col < N);
            b_off[i] = (long long)kb * 8 * a.ldb + (b_ok[i] ? col : 0);
            b_kb[i] = kb;
            b_q[i] = q;
        }
    }

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    u32x4 ra[A_ITEMS];
    u32x4 rb[B_REGS];
    const u32x4 zero4 = {0u, 0u, 0u, 0u};

    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_ITEMS; ++i) {
            const bool ok = (k0 + a_c * 8) < K;
            ra[i] = ok ? *reinterpret_cast<const u32x4*>(Ab + a_off[i] + k0 + a_c * 8) : zero4;
        }
        // expert matrix and K offset inside it for this stage
        int kk = k0, klim = K, e = seg_exp[0];
        if constexpr (SET) {
            const int s = k0 / a.seg_len;
            e = seg_exp[s < kSetMaxK ? s : 0];
            kk = k0 - s * a.seg_len;
            klim = a.seg_len;
        }
        const uint16_t* g0 = B0 + (long long)e * a.strideB;
        const uint16_t* g1 = DUAL ? B1 + (long long)e * a.strideB : g0;
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            const bool ok = b_ok[i] && (k0 < K) && (kk + b_kb[i] * 8) < klim;
            if constexpr (BNK) {
                rb[i] = ok ? *reinterpret_cast<const u32x4*>(g0 + b_off[i] + kk) : zero4;
            } else {
                const uint16_t* src = (b_up[i] ? g1 : g0) + b_off[i] + (long long)kk * a.ldb;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    rb[i * 8 + j] = ok ? *reinterpret_cast<const u32x4*>(src + (long long)j * a.ldb) : zero4;
            }
        }
    };
    auto store_tiles = [&](int stage) {
        char* sA = smem + stage * STAGE;
        char* sB = sA + BM * 128;
#pragma unroll
        for (int i = 0; i < A_ITEMS; ++i) {
            const int r = (tid >> 3) + 32 * i;
            *reinterpret_cast<u32x4*>(sA + swz(r, a_c)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            if constexpr (BNK) {
                *reinterpret_cast<u32x4*>(sB + swz(b_q[i], b_kb[i])) = rb[i];
            } else {
                if (tid + 256 * i < BN) {
                    // rb[i*8 + j] holds row k = kb*8 + j, columns q*8 .. q*8+7.
                    // Transposed: n-row q*8 + c gets k-values kb*8 .. kb*8+7.
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        u32x4 o;
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const uint32_t lo = rb[i * 8 + 2 * d][c >> 1];
                            const uint32_t hi = rb[i * 8 + 2 * d + 1][c >> 1];
                            o[d] = (c & 1) ? pack_hi(lo, hi) : pack_lo(lo, hi);
                        }
                        *reinterpret_cast<u32x4*>(sB + swz(b_q[i] * 8 + c, b_kb[i])) = o;
                    }
                }
            }
        }
    };
    auto compute = [&](int stage) {
        const char* sA = smem + stage * STAGE;
        const char* sB = sA + BM * 128;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int c = kk * 2 + (lane >> 5);
            u32x4 af[MB], bf[NB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                af[mb] = *reinterpret_cast<const u32x4*>(sA + swz(wm * WM + mb * 32 + (lane & 31), c));
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                bf[nb] = *reinterpret_cast<const u32x4*>(sB + swz(wn * WN + nb * 32 + (lane & 31), c));
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if constexpr (SWAP) acc[mb][nb] = mfma32<DT>(bf[nb], af[mb], acc[mb][nb]);
                    else acc[mb][nb] = mfma32<DT>(af[mb], bf[nb], acc[mb][nb]);
                }
        }
    };

    const int nk = (K + kBK - 1) / kBK;
    if (nk > 0) {
        load_tiles(0);
        store_tiles(0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_tiles((kt + 1) * kBK);
        compute(cur);
        if (kt + 1 < nk) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (ATOMIC) {
        // lane owns column (lane & 31) of rows 8*(i/4) + 4*(lane/32) + i%4
        float* C = reinterpret_cast<float*>(a.C);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ml = wm * WM + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (ml >= m_valid) continue;
                const long long rowoff = (long long)s_tok[ml] * N;
                const float w = s_w[ml];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int col = nt * BN + wn * WN + nb * 32 + (lane & 31);
                    if (col < N) unsafeAtomicAdd(C + rowoff + col, w * acc[mb][nb][i]);
                }
            }
        }
    } else {
        // lane owns row (lane & 31) and 4 consecutive columns per register group
        const int nsub = 4 * (lane >> 5);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = wm * WM + mb * 32 + (lane & 31);
            if (ml >= m_valid) continue;
            const int r = r0 + ml;
            if constexpr (MODE == kGateUp || MODE == kFc1) {
                const int p = a.sorted_pair[r];
                const int dst = a.pair_dest ? a.pair_dest[p] : r;
                const float wscale = a.fold_w ? a.routing_w[p] : 1.0f;
                uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)dst * N;
                constexpr int PAIRS = DUAL ? NB / 2 : NB;
                with_act(a.act, [&](auto act_c) {
                    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
                    for (int q = 0; q < PAIRS; ++q) {
                        const int colbase =
                            DUAL ? nt * (BN / 2) + ((wn * WN) / 64 + q) * 32 : nt * BN + wn * WN + q * 32;
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int col = colbase + 8 * g + nsub;
                            if (col >= N) continue;
                            float h[4];
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                if constexpr (DUAL) {
                                    h[j] = act_t<ACT>(acc[mb][2 * q][4 * g + j]) * acc[mb][2 * q + 1][4 * g + j];
                                } else {
                                    h[j] = act_t<ACT>(acc[mb][q][4 * g + j]);
                                }
                                h[j] *= wscale;
                            }
                            u32x2 v;
                            v[0] = pack2<DT>(h[0], h[1]);
                            v[1] = pack2<DT>(h[2], h[3]);
                            *reinterpret_cast<u32x2*>(C + col) = v;
                        }
                    }
                });
            } else {
                // expert-set down projection: each token's row is written once
                const int tok = a.tok_sorted[r];
                uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)tok * N;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int colbase = nt * BN + wn * WN + nb * 32;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = colbase + 8 * g + nsub;
                        if (col >= N) continue;
                        // overwrite: add to +0 instead of the old value (no read)
                        u32x2 old = {0u, 0u};
                        if (!a.overwrite) old = *reinterpret_cast<const u32x2*>(C + col);
                        float h[4];
                        h[0] = Elem<DT>::to_f32((uint16_t)(old[0] & 0xffffu)) + acc[mb][nb][4 * g + 0];
                        h[1] = Elem<DT>::to_f32((uint16_t)(old[0] >> 16)) + acc[mb][nb][4 * g + 1];
                        h[2] = Elem<DT>::to_f32((uint16_t)(old[1] & 0xffffu)) + acc[mb][nb][4 * g + 2];
                        h[3] = Elem<DT>::to_f32((uint16_t)(old[1] >> 16)) + acc[mb][nb][4 * g + 3];
                        u32x2 v;
                        v[0] = pack2<DT>(h[0], h[1]);
                        v[1] = pack2<DT>(h[2], h[3]);
                        *reinterpret_cast<u32x2*>(C + col) = v;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ SIMT
template <int DT, int MODE>
__global__ __launch_bounds__(256) void moe_simt_gemm(GemmArgs a) {
    constexpr int TM = 64, TN = 64, TK = 16;
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool BNK = (MODE == kFc2);
    typedef typename Elem<DT>::storage S;
    __shared__ float sA[TK][TM + 4];
    __shared__ float sB[DUAL ? 2 : 1][TK][TN + 4];
    __shared__ long long s_row[TM];

    int mt, nt;
    if (!tile_coords(a.n_tiles, *a.num_tiles, mt, nt)) return;
    const int r0 = a.tile_row[mt];
    const int e = a.tile_exp[mt];
    const int m_valid = min(TM, a.offsets[e + 1] - r0);
    const int K = a.K, N = a.N;
    const int tid = threadIdx.x;
    const int ty = tid >> 4, tx = tid & 15;
    const S* A = reinterpret_cast<const S*>(a.A);
    const S* B0 = reinterpret_cast<const S*>(a.B0) + (long long)e * a.strideB;
    const S* B1 = DUAL ? reinterpret_cast<const S*>(a.B1) + (long long)e * a.strideB : nullptr;
    if (tid < TM) {
        const int rr = tid < m_valid ? tid : 0;
        if constexpr (GATHER) s_row[tid] = (long long)(a.sorted_pair[r0 + rr] / a.k_top) * K;
        else s_row[tid] = (long long)(r0 + rr) * K;
    }
    __syncthreads();
    const int n0 = nt * TN;
    float acc[DUAL ? 2 : 1][4][4] = {};
    for (int k0 = 0; k0 < K; k0 += TK) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int li = tid + 256 * i;  // 0..1023
            const int m = li >> 4, kk = li & 15;
            sA[kk][m] = (k0 + kk < K) ? Elem<DT>::to_f32(A[s_row[m] + k0 + kk]) : 0.0f;
            const int bk = li >> 6, bn = li & 63;
#pragma unroll
            for (int d = 0; d < (DUAL ? 2 : 1); ++d) {
                const S* B = d ? B1 : B0;
                float v = 0.0f;
                if (k0 + bk < K && n0 + bn < N) {
                    if constexpr (BNK) v = Elem<DT>::to_f32(B[(long long)(n0 + bn) * a.ldb + k0 + bk]);
                    else v = Elem<DT>::to_f32(B[(long long)(k0 + bk) * a.ldb + n0 + bn]);
                }
                sB[d][bk][bn] = v;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = sA[kk][ty * 4 + i];
#pragma unroll
            for (int d = 0; d < (DUAL ? 2 : 1); ++d) {
#pragma unroll
                for (int j = 0; j < 4; ++j) bv[j] = sB[d][kk][tx * 4 + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[d][i][j] = fmaf(av[i], bv[j], acc[d][i][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ml = ty * 4 + i;
        if (ml >= m_valid) continue;
        const int r = r0 + ml;
        if constexpr (MODE == kGateUp || MODE == kFc1) {
            S* C = reinterpret_cast<S*>(a.C) + (long long)r * N;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = n0 + tx * 4 + j;
                if (col >= N) continue;
                float h = act_f32(acc[0][i][j], a.act);
                if constexpr (DUAL) h *= acc[DUAL ? 1 : 0][i][j];
                C[col] = Elem<DT>::from_f32(h);
            }
        } else {
            const int p = a.sorted_pair[r];
            const float w = a.routing_w[p];
            float* C = reinterpret_cast<float*>(a.C) + (long long)(p / a.k_top) * N;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = n0 + tx * 4 + j;
                if (col < N) unsafeAtomicAdd(C + col, w * acc[0][i][j]);
            }
        }
    }
}

// -------------------------------------------------------------- helpers
__global__ void fill_zero_u32(uint32_t* __restrict__ p, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

__global__ void fill_zero_u32x4(u32x4* __restrict__ p, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = z;
}

template <int DT>
__global__ void finalize_kernel(typename Elem<DT>::storage* __restrict__ out, const float* __restrict__ acc,
                                long long n, int overwrite) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = Elem<DT>::from_f32(overwrite ? acc[i] : Elem<DT>::to_f32(out[i]) + acc[i]);
}

// 16-bit output, 8 elements per thread and iteration (two 16-byte
// accumulator loads, one 16-byte store); out 16-byte aligned, n % 8 == 0.
template <int DT>
__global__ void finalize_vec8_kernel(uint16_t* __restrict__ out, const float* __restrict__ acc, long long n8,
                                     int overwrite) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const f32x4 a0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(acc) + 2 * i);
        const f32x4 a1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(acc) + 2 * i + 1);
        u32x4* o = reinterpret_cast<u32x4*>(out) + i;
        u32x4 old = {0u, 0u, 0u, 0u};
        if (!overwrite) old = *o;
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x0 = j < 2 ? a0[2 * j] : a1[2 * j - 4];
            const float x1 = j < 2 ? a0[2 * j + 1] : a1[2 * j - 3];
            const float y0 = overwrite ? x0 : Elem<DT>::to_f32((uint16_t)(old[j] & 0xffffu)) + x0;
            const float y1 = overwrite ? x1 : Elem<DT>::to_f32((uint16_t)(old[j] >> 16)) + x1;
            v[j] = pack2<DT>(y0, y1);
        }
        *o = v;
    }
}

static unsigned grid_for(long long n, int block) {
    long long g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (unsigned)g;
}

__global__ void fill_zero_u16(uint16_t* __restrict__ p, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

// Zero nbytes (a multiple of 2) with a fill kernel rather than hipMemsetAsync.
hipError_t launch_fill_zero_bytes(void* p, long long nbytes, hipStream_t stream) {
    if (nbytes <= 0) return hipSuccess;
    if (((uintptr_t)p % 16) == 0 && nbytes % 16 == 0) {
        const long long n = nbytes / 16;
        hipLaunchKernelGGL(fill_zero_u32x4, dim3(grid_for(n, 256)), dim3(256), 0, stream,
                           reinterpret_cast<u32x4*>(p), n);
    } else if (((uintptr_t)p % 4) == 0 && nbytes % 4 == 0) {
        const long long n = nbytes / 4;
        hipLaunchKernelGGL(fill_zero_u32, dim3(grid_for(n, 256)), dim3(256), 0, stream,
                           reinterpret_cast<uint32_t*>(p), n);
    } else {
        const long long n = nbytes / 2;
        hipLaunchKernelGGL(fill_zero_u16, dim3(grid_for(n, 256)), dim3(256), 0, stream,
                           reinterpret_cast<uint16_t*>(p), n);
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero_f32(float* p, long long n, hipStream_t stream) {
    return launch_fill_zero_bytes(p, n * 4, stream);
}

// Pair rows -> token rows: one thread per 8 consecutive columns of a token
// (16-byte loads of its k rows, f32 sums in slot order, one 16-byte store).
template <int DT>
__global__ void pair_rows_sum8_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ rows,
                                      const uint32_t* __restrict__ idx, int E, int T, int k, int H, int overwrite) {
    const int h8 = H / 8;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < (long long)T * h8;
         i += (long long)gridDim.x * blockDim.x) {
    const long long t = i / h8, c = (i - t * h8) * 8;
    float s[8];
    if (overwrite) {
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] = 0.0f;
    } else {
        const u32x4 o = *reinterpret_cast<const u32x4*>(out + t * H + c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[2 * j] = Elem<DT>::to_f32((uint16_t)(o[j] & 0xffffu));
            s[2 * j + 1] = Elem<DT>::to_f32((uint16_t)(o[j] >> 16));
        }
    }
    for (int j = 0; j < k; ++j) {
        if (idx[t * k + j] >= (uint32_t)E) continue;  // dropped pair: no row
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows + (t * k + j) * H + c));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            s[2 * q] += Elem<DT>::to_f32((uint16_t)(v[q] & 0xffffu));
            s[2 * q + 1] += Elem<DT>::to_f32((uint16_t)(v[q] >> 16));
        }
    }
    u32x4 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = pack2<DT>(s[2 * q], s[2 * q + 1]);
    *reinterpret_cast<u32x4*>(out + t * H + c) = r;
    }
}
template <int DT>
__global__ void pair_rows_sum_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ rows,
                                     const uint32_t* __restrict__ idx, int E, int T, int k, int H, int overwrite) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < (long long)T * H;
         i += (long long)gridDim.x * blockDim.x) {
        const long long t = i / H, c = i - t * H;
        float s = overwrite ? 0.0f : Elem<DT>::to_f32(out[i]);
        for (int j = 0; j < k; ++j)
            if (idx[t * k + j] < (uint32_t)E) s += Elem<DT>::to_f32(rows[(t * k + j) * H + c]);
        out[i] = Elem<DT>::from_f32(s);
    }
}

hipError_t launch_pair_rows_sum(void* out, int dtype, const void* rows, const uint32_t* idx, int E, int T, int k,
                                int H, bool overwrite, hipStream_t stream) {
    if (T <= 0 || H <= 0) return hipSuccess;
    if (dtype != kBF16 && dtype != kF16) return hipErrorInvalidValue;
    const int ow = overwrite ? 1 : 0;
    uint16_t* o = reinterpret_cast<uint16_t*>(out);
    const uint16_t* rw = reinterpret_cast<const uint16_t*>(rows);
    const dim3 b(256);
    if (H % 8 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)rows % 16) == 0) {
        const dim3 g(grid_for((long long)T * (H / 8), 256));
        if (dtype == kBF16)
            hipLaunchKernelGGL(pair_rows_sum8_kernel<kBF16>, g, b, 0, stream, o, rw, idx, E, T, k, H, ow);
        else
            hipLaunchKernelGGL(pair_rows_sum8_kernel<kF16>, g, b, 0, stream, o, rw, idx, E, T, k, H, ow);
    } else {
        const dim3 g(grid_for((long long)T * H, 256));
        if (dtype == kBF16)
            hipLaunchKernelGGL(pair_rows_sum_kernel<kBF16>, g, b, 0, stream, o, rw, idx, E, T, k, H, ow);
        else
            hipLaunchKernelGGL(pair_rows_sum_kernel<kF16>, g, b, 0, stream, o, rw, idx, E, T, k, H, ow);
    }
    return hipGetLastError();
}

hipError_t launch_finalize(void* out, int dtype, const float* acc, long long n, bool overwrite, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 g(grid_for(n, 256)), b(256);
    const int ow = overwrite ? 1 : 0;
    if ((dtype == kBF16 || dtype == kF16) && n % 8 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)acc % 16) == 0) {
        const long long n8 = n / 8;
        const dim3 g8(grid_for(n8, 256));
        if (dtype == kBF16)
            hipLaunchKernelGGL(finalize_vec8_kernel<kBF16>, g8, b, 0, stream, reinterpret_cast<uint16_t*>(out), acc, n8,
                               ow);
        else
            hipLaunchKernelGGL(finalize_vec8_kernel<kF16>, g8, b, 0, stream, reinterpret_cast<uint16_t*>(out), acc, n8,
                               ow);
        return hipGetLastError();
    }
    if (dtype == kBF16)
        hipLaunchKernelGGL(finalize_kernel<kBF16>, g, b, 0, stream, reinterpret_cast<uint16_t*>(out), acc, n, ow);
    else if (dtype == kF16)
        hipLaunchKernelGGL(finalize_kernel<kF16>, g, b, 0, stream, reinterpret_cast<uint16_t*>(out), acc, n, ow);
    else
        hipLaunchKernelGGL(finalize_kernel<kF32>, g, b, 0, stream, reinterpret_cast<float*>(out), acc, n, ow);
    return hipGetLastError();
}

bool mfma_supported(int dtype, int K, int N) {
    return (dtype == kBF16 || dtype == kF16) && (K % 8 == 0) && (N % 8 == 0);
}

int gemm_tile_cols(int mode, int cfg) {
    const int bn = tile_cols(cfg);
    if (is_f32_cfg(cfg) || cfg == kW8Gemv) return mode == kGateUp ? bn / 2 : bn;
    return (mode == kGateUp && cfg != kTileSimt) ? bn / 2 : bn;
}

template <int DT, int MODE>
static hipError_t launch_mode(int cfg, const GemmArgs& a, hipStream_t stream) {
    const int nwg = a.m_tiles_max * a.n_tiles;
    if (nwg <= 0) return hipSuccess;
    if (cfg == kTile128) {
        if constexpr (DT == kF32) {
            return hipErrorInvalidValue;
        } else {
            hipLaunchKernelGGL((moe_mfma_gemm<DT, 128, 128, MODE>), dim3(nwg), dim3(256), 0, stream, a);
        }
    } else {
        if constexpr (MODE == kDownSet || MODE == kFc2Set) {
            return hipErrorInvalidValue;  // the expert-set path is MFMA-only
        } else {
            hipLaunchKernelGGL((moe_simt_gemm<DT, MODE>), dim3(nwg), dim3(256), 0, stream, a);
        }
    }
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_dt(int mode, int cfg, const GemmArgs& a, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return launch_mode<DT, kGateUp>(cfg, a, stream);
        case kFc1: return launch_mode<DT, kFc1>(cfg, a, stream);
        case kDown: return launch_mode<DT, kDown>(cfg, a, stream);
        case kFc2: return launch_mode<DT, kFc2>(cfg, a, stream);
        case kDownSet: return launch_mode<DT, kDownSet>(cfg, a, stream);
        case kFc2Set: return launch_mode<DT, kFc2Set>(cfg, a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_gemm(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream) {
    if (is_lds_cfg(cfg)) return launch_moe_gemm_lds(mode, dtype, cfg, a, stream);
    if (is_f32_cfg(cfg)) return dtype == kF32 ? launch_moe_gemm_f32(mode, cfg, a, stream) : hipErrorInvalidValue;
    if (dtype == kBF16) return launch_dt<kBF16>(mode, cfg, a, stream);
    if (dtype == kF16) return launch_dt<kF16>(mode, cfg, a, stream);
    if (dtype == kF32) return launch_dt<kF32>(mode, cfg, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
