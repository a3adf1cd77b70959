// Expert-grouped GEMMs in f32 (gfx950 has no f32 MFMA rate above its vector
// FMA rate, so f32 runs on the vector ALUs, as the reference's f32 path does).
//
// moe_f32_gemm<BM, MODE>: BM x 128 block tile (BM = 128 for batches, 32 for
// decode), 256 threads; thread (ty, tx) = (tid / 16, tid % 16) owns rows
// ty*BM/16 .. +BM/16 and panel columns 4tx .. 4tx+3 and 64+4tx .. 64+4tx+3.
// For the gate/up GEMM the 128-column weight panel is 64 gate columns then
// the same 64 up columns, so a thread holds gate and up of 4 output columns
// (64 output columns per workgroup). K goes in chunks of 16:
// the next chunk's A rows and weight panel are fetched with 16-byte loads
// into registers while the current chunk is consumed from LDS, then stored
// to the other LDS buffer; one barrier per chunk.
//  * A rows are gathered (gate/up, fc1: the pair's token row) or sorted rows
//    (down, fc2: the intermediate in pair order), stored k-major in LDS.
//  * [K,N] weights (gate, up, down) are copied row by row; [N,K] weights (the
//    Nomic fc2 operand) are transposed into the same k-major layout.
//  * Decode tiles (BM = 32) split K over up to 16 workgroups per tile; the
//    splits meet in an ordered fixup (device-coherent partials, an arrival
//    counter, the last split sums in split order), so results stay
//    deterministic.
//  * Epilogues as the other kernels: act(gate) * up or act(x) into the
//    intermediate; w * acc added with one f32 atomic per element and pair
//    into the accumulator (down, fc2).
// Requires K % 4 == 0, N % 4 == 0 and 16-byte aligned operands (checked on
// the host; other shapes take moe_simt_gemm).
#include "cm_lds.hpp"

namespace cm {

using namespace lds;

template <int BM, int MODE>
__global__ __launch_bounds__(256, 2) void moe_f32_gemm(GemmArgs a) {
    constexpr int BN = 128, TK = 16;
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool BNK = (MODE == kFc2);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    constexpr int BNO = DUAL ? BN / 2 : BN;       // output columns per workgroup
    constexpr int RM = BM / 16;                   // rows per thread
    constexpr int A_VEC = BM * TK / 4;            // float4 of one A chunk
    constexpr int A_PER = (A_VEC + 255) / 256;    // per thread
    constexpr int B_VEC = BN * TK / 4;            // float4 of one weight panel chunk
    constexpr int B_PER = B_VEC / 256;
    constexpr int NACC = RM * 8;                  // accumulators per thread
    static_assert(B_PER * 256 == B_VEC && NACC % 4 == 0, "f32 tile");
    __shared__ __attribute__((aligned(16))) float sA[2][TK][BM + 4];
    __shared__ __attribute__((aligned(16))) float sB[2][TK][BN + 4];
    __shared__ long long s_row[BM];
    __shared__ int s_last;

    clear_share(a.zero_f32, a.zero_n);
    const int live = *a.num_tiles * a.n_tiles;
    const int nsplit = adaptive_split(a.ksplit, a.split_target, live, (a.K + TK - 1) / TK);
    const int lg = xcd_logical(live * nsplit);
    if (lg < 0) return;
    const int tile = lg / nsplit, ks = lg - tile * nsplit;
    const int mt = tile / a.n_tiles, nt = tile - mt * a.n_tiles;
    const int r0 = a.tile_row[mt];
    const int e = a.tile_exp[mt];
    const int m_valid = min(BM, a.offsets[e + 1] - r0);
    const int K = a.K, N = a.N, n0 = nt * BNO;
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    const float* A = reinterpret_cast<const float*>(a.A);
    const float* B0 = reinterpret_cast<const float*>(a.B0) + (long long)e * a.strideB;
    const float* B1 = DUAL ? reinterpret_cast<const float*>(a.B1) + (long long)e * a.strideB : nullptr;
    for (int m = tid; m < BM; m += 256) {
        const int rr = m < m_valid ? m : 0;
        s_row[m] = GATHER ? (long long)(a.sorted_pair[r0 + rr] / a.k_top) * K : (long long)(r0 + rr) * K;
    }
    __syncthreads();

    // this split's K chunks
    const int nk_all = (K + TK - 1) / TK;
    const int per_split = (nk_all + nsplit - 1) / nsplit;
    const int kc0 = min(nk_all, ks * per_split);
    const int nk = min(nk_all, kc0 + per_split) - kc0;

    f32x4 ra[A_PER], rb[B_PER];
    auto fetch = [&](int kc) {
        const int k0 = kc * TK;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int li = tid + 256 * i;
            const int m = li >> 2, q = li & 3;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (li < A_VEC && k0 + 4 * q < K) v = *reinterpret_cast<const f32x4*>(A + s_row[m] + k0 + 4 * q);
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int li = tid + 256 * i;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if constexpr (BNK) {
                const int n = li >> 2, q = li & 3;
                if (n0 + n < N && k0 + 4 * q < K)
                    v = *reinterpret_cast<const f32x4*>(B0 + (long long)(n0 + n) * a.ldb + k0 + 4 * q);
            } else {
                const int kr = li >> 5, c4 = li & 31;
                // panel column 4*c4: DUAL = gate (c4 < 16) or up (c4 >= 16) column
                const float* B = (DUAL && c4 >= 16) ? B1 : B0;
                const int col = n0 + 4 * (DUAL ? (c4 & 15) : c4);
                if (k0 + kr < K && col < N) v = *reinterpret_cast<const f32x4*>(B + (long long)(k0 + kr) * a.ldb + col);
            }
            rb[i] = v;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int li = tid + 256 * i;
            if (li < A_VEC) {
                const int m = li >> 2, q = li & 3;
#pragma unroll
                for (int j = 0; j < 4; ++j) sA[buf][4 * q + j][m] = ra[i][j];
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int li = tid + 256 * i;
            if constexpr (BNK) {
                const int n = li >> 2, q = li & 3;
#pragma unroll
                for (int j = 0; j < 4; ++j) sB[buf][4 * q + j][n] = rb[i][j];
            } else {
                const int kr = li >> 5, c4 = li & 31;
                *reinterpret_cast<f32x4*>(&sB[buf][kr][4 * c4]) = rb[i];
            }
        }
    };

    float acc[RM][8];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;

    if (nk > 0) {
        fetch(kc0);
        stash(0);
    }
    __syncthreads();
    for (int c = 0; c < nk; ++c) {
        const int buf = c & 1;
        if (c + 1 < nk) fetch(kc0 + c + 1);
#pragma unroll 4
        for (int kk = 0; kk < TK; ++kk) {
            float av[RM];
#pragma unroll
            for (int i = 0; i < RM; ++i) av[i] = sA[buf][kk][ty * RM + i];
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sB[buf][kk][4 * tx]);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sB[buf][kk][64 + 4 * tx]);
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = fmaf(av[i], b0[j], acc[i][j]);
                    acc[i][4 + j] = fmaf(av[i], b1[j], acc[i][4 + j]);
                }
        }
        if (c + 1 < nk) stash(buf ^ 1);
        __syncthreads();
    }

    if (nsplit > 1) {
        // ordered fixup: thread-owned partials, 16 bytes per store, lanes contiguous
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, 0x7ffffff0, 0x00020000);
        constexpr uint32_t SLOT = 256u * NACC * 4u;  // bytes per split
        float* flat = &acc[0][0];
        const uint32_t mine = (uint32_t)(tile * nsplit + ks) * SLOT + (uint32_t)tid * 16u;
#pragma unroll
        for (int q = 0; q < NACC / 4; ++q) {
            const u32x4 v = {__float_as_uint(flat[4 * q]), __float_as_uint(flat[4 * q + 1]),
                             __float_as_uint(flat[4 * q + 2]), __float_as_uint(flat[4 * q + 3])};
            __builtin_amdgcn_raw_buffer_store_b128(v, pr, mine + q * 4096u, 0, kCachePolicyDevice);
        }
        // stores -> barrier -> release increment at agent scope, and an
        // acquire fence in the last split (as splitk_fixup): its partial
        // loads see every split's stores
        __syncthreads();
        if (tid == 0) {
            s_last = __hip_atomic_fetch_add(a.counters + tile, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                     nsplit - 1;
            if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
        if (!s_last) return;
        for (int s2 = 0; s2 < nsplit; ++s2) {
            const uint32_t src = (uint32_t)(tile * nsplit + s2) * SLOT + (uint32_t)tid * 16u;
#pragma unroll
            for (int q = 0; q < NACC / 4; ++q) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(pr, src + q * 4096u, 0, kCachePolicyDevice);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    flat[4 * q + j] = s2 == 0 ? __uint_as_float(v[j]) : flat[4 * q + j] + __uint_as_float(v[j]);
            }
        }
        if (tid == 0) __hip_atomic_store(a.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

#pragma unroll
    for (int i = 0; i < RM; ++i) {
        const int ml = ty * RM + i;
        if (ml >= m_valid) continue;
        const int r = r0 + ml;
        if constexpr (DUAL) {
            // acc[i][0..3]: gate, acc[i][4..7]: up of output columns n0 + 4tx ..
            float* C = reinterpret_cast<float*>(a.C) + (long long)r * N;
            const int col = n0 + 4 * tx;
            if (col < N) {
                f32x4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = act_f32(acc[i][j], a.act) * acc[i][4 + j];
                *reinterpret_cast<f32x4*>(C + col) = v;
            }
        } else if constexpr (!ATOMIC) {
            float* C = reinterpret_cast<float*>(a.C) + (long long)r * N;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = n0 + 64 * h + 4 * tx;
                if (col >= N) continue;
                f32x4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = act_f32(acc[i][4 * h + j], a.act);
                *reinterpret_cast<f32x4*>(C + col) = v;
            }
        } else {
            const int p = a.sorted_pair[r];
            const float w = a.routing_w[p];
            float* C = reinterpret_cast<float*>(a.C) + (long long)(p / a.k_top) * N;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = n0 + 64 * h + 4 * tx;
                if (col >= N) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j) unsafeAtomicAdd(C + col + j, w * acc[i][4 * h + j]);
            }
        }
    }
}

template <int MODE>
static hipError_t launch_f32_mode(int cfg, const GemmArgs& a, hipStream_t stream) {
    const long long nwg_l = split_grid((long long)a.m_tiles_max * a.n_tiles, a);
    if (nwg_l > 0x7fffffffLL) return hipErrorInvalidValue;
    const int nwg = (int)nwg_l;
    if (nwg <= 0) return hipSuccess;
    if (cfg == kF32Rows32)
        hipLaunchKernelGGL((moe_f32_gemm<32, MODE>), dim3(nwg), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((moe_f32_gemm<128, MODE>), dim3(nwg), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_moe_gemm_f32(int mode, int cfg, const GemmArgs& a, hipStream_t stream) {
    switch (mode) {
        case kGateUp: return launch_f32_mode<kGateUp>(cfg, a, stream);
        case kFc1: return launch_f32_mode<kFc1>(cfg, a, stream);
        case kDown: return launch_f32_mode<kDown>(cfg, a, stream);
        case kFc2: return launch_f32_mode<kFc2>(cfg, a, stream);
        default: return hipErrorInvalidValue;  // the expert-set path is MFMA-only
    }
}

}  // namespace cm
