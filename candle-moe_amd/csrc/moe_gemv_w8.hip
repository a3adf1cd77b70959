// Decode GEMMs over fp8 e4m3 weights without LDS staging or K splits across
// workgroups (gfx950).
//
// Few rows per touched expert (decode): the work is the weight stream. The
// 32-row tile kernel stages weights through LDS and splits K across
// workgroups, whose fixed costs (tile-table chain, stage hand-over barriers,
// split-K partials and fixup) took about half of its launch at these sizes.
// Here the weights are K-contiguous ([E][N][K] codes), so each lane loads the
// bytes of one MFMA operand straight from memory:
//  * a wave owns two 16-column blocks (gate/up: 16 gate and the matching 16
//    up columns; fc1 / down / fc2: 32 columns) of one 32-row tile (one
//    expert) over a part of K; the 4 waves of a workgroup split K in KW
//    parts (the fewest of 1, 2, 4 that still give two workgroups per CU,
//    chosen from the row tiles the grouping produced) and the columns in
//    4 / KW groups;
//  * each wave keeps its own loads in flight (a ring of four 64-wide K
//    steps; the first weight steps leave before the row metadata is read)
//    and meets no barrier until the end, where the K parts are summed
//    through LDS in wave order (deterministic) and the first wave of each
//    column group runs the epilogue: one store, or one atomic add, per
//    element and pair, as the tile kernels;
//  * v_mfma_f32_16x16x32: the A operand is the token rows (16 per block, a
//    second block only for tiles of more than 16 rows), the B operand the
//    weight columns. Lane l holds k = 8*(l/16) .. +7 of a 32-wide step in
//    both operands; a 16-byte load gives lane group g (= l/16) the 16 codes
//    k0 + 16g .. +15 of its column, which feed two MFMAs (the first 8 and the
//    last 8 of each group): the same permutation of K in both operands, so
//    the products and sums are those of the plain order.
// Buffer resources return zeros past each operand; rows past the tile's
// group, columns past N and K positions past K (or past this wave's share)
// are pointed past the resource, so they add exact zeros.
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

constexpr int kGvWaves = 4;  // waves per workgroup: KW along K x 4/KW along N
constexpr int kGvRing = 4;   // K steps in flight per wave
constexpr int kGvStep = 64;  // K per step

// The K loop, reduction and epilogue of one wave's column blocks over the
// tile's RB row blocks of 16 (2 only when the tile holds more than 16 rows).
// wv: the weight half of the load ring, whose first steps the caller issued
// before the row metadata arrived.
template <int DT, int MODE, int KW, int RB>
__device__ __forceinline__ void gemv_rows(const GemmArgs& a, int r0, int e, int m_valid, const int (&col)[kGvCB],
                                          const int (&pr)[2], u32x4 (&wv)[kGvRing][kGvCB], int s0, int s1,
                                          const __amdgpu_buffer_rsrc_t& rw0, const __amdgpu_buffer_rsrc_t& rw1,
                                          const uint32_t (&woff)[kGvCB], f32x4* red) {
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool ATOMIC = (MODE == kDown);
    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kq = wave % KW, cw = wave / KW;
    const int g = lane >> 4, li = lane & 15;
    const int K = a.K, N = a.N;

    // token rows of this lane (one per row block): gathered for gate/up and
    // fc1, the tile's own rows of the intermediate for down / fc2
    uint32_t xoff[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int m = rb * 16 + li;
        const int src = GATHER ? pr[rb] / a.k_top : r0 + m;
        xoff[rb] = m < m_valid ? ((uint32_t)src * (uint32_t)K + 16u * (uint32_t)g) * 2u : kOob;
    }
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.A), 0, (int)a.a_bytes, 0x00020000);

    f32x4 acc[RB][kGvCB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < kGvCB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 xv[kGvRing][RB][2];
    // step s into ring slot i (steps past this wave's share, or K positions
    // past K, load zeros; K is a multiple of 16)
    auto in_k = [&](int s) { return s < s1 && s * kGvStep + 16 * g < K; };
    auto load_w = [&](int i, int s) {
        const bool in = in_k(s);
#pragma unroll
        for (int cb = 0; cb < kGvCB; ++cb)
            wv[i][cb] = __builtin_amdgcn_raw_buffer_load_b128((cb & 1) ? rw1 : rw0, in ? woff[cb] : kOob,
                                                               s * kGvStep, 0);
    };
    auto load_x = [&](int i, int s) {
        const bool in = in_k(s);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint32_t o = in ? xoff[rb] : kOob;
            xv[i][rb][0] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 2 * s * kGvStep, 0);
            xv[i][rb][1] = __builtin_amdgcn_raw_buffer_load_b128(rx, o + 16u, 2 * s * kGvStep, 0);
        }
    };
    auto compute = [&](int i) {
        u32x4 wl[kGvCB], wh[kGvCB];
#pragma unroll
        for (int cb = 0; cb < kGvCB; ++cb) {
            wl[cb] = fp8x8_to<DT>(u32x2{wv[i][cb][0], wv[i][cb][1]});  // exact in DT
            wh[cb] = fp8x8_to<DT>(u32x2{wv[i][cb][2], wv[i][cb][3]});
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < kGvCB; ++cb) {
                acc[rb][cb] = mfma16<DT>(xv[i][rb][0], wl[cb], acc[rb][cb]);
                acc[rb][cb] = mfma16<DT>(xv[i][rb][1], wh[cb], acc[rb][cb]);
            }
    };
#pragma unroll
    for (int i = 0; i < kGvRing; ++i) load_x(i, s0 + i);
    for (int s = s0; s < s1; s += kGvRing) {
#pragma unroll
        for (int i = 0; i < kGvRing; ++i) {
            compute(i);
            load_w(i, s + i + kGvRing);
            load_x(i, s + i + kGvRing);
        }
    }

    // the K parts of a column group, summed in wave order
    constexpr int NBLK = RB * kGvCB;
    if constexpr (KW > 1) {
        if (kq > 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < kGvCB; ++cb)
                    red[((cw * (KW - 1) + kq - 1) * NBLK + rb * kGvCB + cb) * 64 + lane] = acc[rb][cb];
        }
        __syncthreads();
        if (kq != 0) return;
#pragma unroll
        for (int q = 1; q < KW; ++q)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < kGvCB; ++cb)
                    acc[rb][cb] += red[((cw * (KW - 1) + q - 1) * NBLK + rb * kGvCB + cb) * 64 + lane];
    }

    // epilogue: lane l holds column li of each block, rows 4g .. 4g+3 of each
    // row block (the 16x16 MFMA result layout)
    const long long soff = (long long)e * N;
    if constexpr (ATOMIC) {
        float* C = reinterpret_cast<float*>(a.C);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = rb * 16 + 4 * g + j;
                if (m >= m_valid) continue;
                const int p = a.sorted_pair[r0 + m];
                const long long rowoff = (long long)(p / a.k_top) * N;
                const float w = a.routing_w[p];
#pragma unroll
                for (int cb = 0; cb < kGvCB; ++cb) {
                    if (col[cb] >= N) continue;
                    const float sc = a.scale0[soff + col[cb]];
                    unsafeAtomicAdd(C + rowoff + col[cb], w * (sc * acc[rb][cb][j]));
                }
            }
    } else {
        with_act(a.act, [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
            constexpr int NOUT = DUAL ? kGvCB / 2 : kGvCB;  // output blocks
            float s0v[NOUT], s1v[NOUT];
#pragma unroll
            for (int ob = 0; ob < NOUT; ++ob) {
                const int c = col[DUAL ? 2 * ob : ob];
                s0v[ob] = c < N ? a.scale0[soff + c] : 0.0f;
                s1v[ob] = (DUAL && c < N) ? a.scale1[soff + c] : 0.0f;
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int m = rb * 16 + 4 * g + j;
                    if (m >= m_valid) continue;
                    const int r = r0 + m;
                    const int p = a.sorted_pair[r];
                    const int dst = a.pair_dest ? a.pair_dest[p] : r;
                    const float ws = a.fold_w ? a.routing_w[p] : 1.0f;
                    uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)dst * N;
#pragma unroll
                    for (int ob = 0; ob < NOUT; ++ob) {
                        const int c = col[DUAL ? 2 * ob : ob];
                        if (c >= N) continue;
                        float h;
                        if constexpr (DUAL)
                            h = act_t<ACT>(s0v[ob] * acc[rb][2 * ob][j]) * (s1v[ob] * acc[rb][2 * ob + 1][j]);
                        else
                            h = act_t<ACT>(s0v[ob] * acc[rb][ob][j]);
                        C[c] = (uint16_t)(pack2<DT>(h * ws, 0.0f) & 0xffffu);
                    }
                }
        });
    }
}

// Workgroup t of a launch whose 4 waves split K in KW parts: one 32-row
// tile x gv_wg_cols(MODE, KW) output columns; wave (kq, cw) = (wave % KW,
// wave / KW) takes K part kq of column group cw.
template <int DT, int MODE, int KW>
__device__ __forceinline__ void gemv_wg(const GemmArgs& a, int t, int n_tiles, f32x4* red) {
    constexpr bool DUAL = (MODE == kGateUp);
    static_assert(!DUAL || kGvCB % 2 == 0, "gate / up block pairs");
    const int mt = t / n_tiles, nt = t - mt * n_tiles;
    const int r0 = a.tile_row[mt];
    const int e = a.tile_exp[mt];

    const int lane = (int)(threadIdx.x & 63u);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int kq = wave % KW, cw = wave / KW;
    const int g = lane >> 4, li = lane & 15;
    const int N = a.N;
    // this wave's weight columns (one per block; DUAL: even blocks gate, odd
    // blocks up, block pair q: output columns 16q ..)
    constexpr int PWC = DUAL ? 8 * kGvCB : 16 * kGvCB;
    int col[kGvCB];
    uint32_t woff[kGvCB];
#pragma unroll
    for (int cb = 0; cb < kGvCB; ++cb) {
        col[cb] = nt * (PWC * (kGvWaves / KW)) + cw * PWC + (DUAL ? (cb >> 1) : cb) * 16 + li;
        woff[cb] = col[cb] < N ? (uint32_t)col[cb] * (uint32_t)a.ldb + 16u * (uint32_t)g : kOob;
    }
    const long long wbytes = a.strideB;  // one byte per code
    const __amdgpu_buffer_rsrc_t rw0 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(reinterpret_cast<const char*>(a.B0) + (long long)e * wbytes), 0, (int)wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw1 =
        DUAL ? __builtin_amdgcn_make_buffer_rsrc(
                   const_cast<char*>(reinterpret_cast<const char*>(a.B1) + (long long)e * wbytes), 0, (int)wbytes,
                   0x00020000)
             : rw0;
    const int nks = (a.K + kGvStep - 1) / kGvStep;
    const int s0 = kq * nks / KW, s1 = (kq + 1) * nks / KW;
    // the first weight steps go out before the row metadata is read (they
    // depend on the expert only)
    u32x4 wv[kGvRing][kGvCB];
#pragma unroll
    for (int i = 0; i < kGvRing; ++i) {
        const int s = s0 + i;
        const bool in = s < s1 && s * kGvStep + 16 * g < a.K;
#pragma unroll
        for (int cb = 0; cb < kGvCB; ++cb)
            wv[i][cb] = __builtin_amdgcn_raw_buffer_load_b128((cb & 1) ? rw1 : rw0, in ? woff[cb] : kOob,
                                                               s * kGvStep, 0);
    }
    // rows: the group's end and this lane's pairs (rows li and 16 + li,
    // clamped to the array: rows past the group are masked afterwards)
    const int m_valid = min(32, a.offsets[e + 1] - r0);
    int pr[2];
    pr[0] = a.sorted_pair[min(r0 + li, a.sorted_n - 1)];
    pr[1] = a.sorted_pair[min(r0 + 16 + li, a.sorted_n - 1)];
    if (m_valid > 16)
        gemv_rows<DT, MODE, KW, 2>(a, r0, e, m_valid, col, pr, wv, s0, s1, rw0, rw1, woff, red);
    else
        gemv_rows<DT, MODE, KW, 1>(a, r0, e, m_valid, col, pr, wv, s0, s1, rw0, rw1, woff, red);
}

// The grid covers the most workgroups any split can take (m_tiles_max x
// gv_wg_cols(MODE, 4) columns); the split is chosen here from the live row
// tiles the grouping produced (gv_pick_kw), and workgroups past that
// split's count exit.
template <int DT, int MODE>
__global__ __launch_bounds__(64 * kGvWaves, 3) void moe_w8_gemv(GemmArgs a) {
    // every workgroup first clears its share of zero_f32 (the accumulator of
    // the GEMM that follows)
    clear_share(a.zero_f32, a.zero_n);
    const int tiles = *a.num_tiles;
    const int kw = gv_pick_kw(MODE, a.N, tiles);
    const int n_tiles = (a.N + gv_wg_cols(MODE, kw) - 1) / gv_wg_cols(MODE, kw);
    const int t = (int)blockIdx.x;
    if (t >= tiles * n_tiles) return;
    __shared__ f32x4 red[(kGvWaves - 1) * 2 * kGvCB * 64];
    if (kw == 1) gemv_wg<DT, MODE, 1>(a, t, n_tiles, red);
    else if (kw == 2) gemv_wg<DT, MODE, 2>(a, t, n_tiles, red);
    else gemv_wg<DT, MODE, 4>(a, t, n_tiles, red);
}

template <int DT, int MODE>
hipError_t launch_mode(const GemmArgs& a, hipStream_t stream) {
    // n_tiles: the column tiles of the split with the most workgroups (K in 4)
    const long long nwg = (long long)a.m_tiles_max * a.n_tiles;
    if (nwg > 0x7fffffffLL) return hipErrorInvalidValue;
    if (nwg <= 0) return hipSuccess;
    hipLaunchKernelGGL((moe_w8_gemv<DT, MODE>), dim3((int)nwg), dim3(64 * kGvWaves), 0, stream, a);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_dt(int mode, const GemmArgs& a, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return launch_mode<DT, kGateUp>(a, stream);
        case kFc1: return launch_mode<DT, kFc1>(a, stream);
        case kDown:
        case kFc2:  // fc2 codes are [E][H][I] like down's: the same kernel
            return launch_mode<DT, kDown>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_w8_gemv(int mode, int dtype, const GemmArgs& a, hipStream_t stream) {
    if (dtype == kBF16) return launch_dt<kBF16>(mode, a, stream);
    if (dtype == kF16) return launch_dt<kF16>(mode, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace cm
