// Grouping of (token, slot) pairs by expert: histogram, exclusive scan and a
// stable scatter into expert-sorted order, plus the row-tile table the
// grouped GEMMs are launched over.
//
// Semantics follow /root/reference/kernels/preprocessing.cuh:5-59 (counts,
// offsets[E] = valid pairs, offsets[E+1] = largest group, pairs with an
// out-of-range expert dropped) with two differences: the order inside an
// expert is ascending pair id (the reference's LDS-atomic order is not
// deterministic), and the multi-block path scans per-block counts instead of
// aliasing counts and offsets (/root/reference/kernels/preprocessing.cuh:296-298).
//
// Three launches, all multi-workgroup, no host synchronisation:
//   1. grouping_hist   : each workgroup histograms kGroupChunk pairs in LDS
//   2. grouping_scan   : one workgroup turns the per-block counts into
//                        per-block bases, expert offsets and the tile table
//   3. grouping_scatter: each workgroup re-reads its chunk and ranks pairs
//                        stably with wave ballots (64-lane peer masks)
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

constexpr int kGroupThreads = 256;

__global__ __launch_bounds__(kGroupThreads) void grouping_hist(const uint32_t* __restrict__ idx, long long P,
                                                               int E, int32_t* __restrict__ block_counts) {
    extern __shared__ int32_t s_cnt[];  // [4 waves][E]
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * E; i += kGroupThreads) s_cnt[i] = 0;
    __syncthreads();
    const long long base = (long long)blockIdx.x * kGroupChunk;
    const long long end = base + kGroupChunk < P ? base + kGroupChunk : P;
    int32_t* mine = s_cnt + wave * E;
    for (long long p = base + threadIdx.x; p < end; p += kGroupThreads) {
        const uint32_t e = __builtin_nontemporal_load(idx + p);
        if (e < (uint32_t)E) atomicAdd(mine + e, 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kGroupThreads)
        block_counts[(long long)blockIdx.x * E + e] = s_cnt[e] + s_cnt[E + e] + s_cnt[2 * E + e] + s_cnt[3 * E + e];
}

// One workgroup. block_counts[b][e] becomes the number of expert-e pairs in
// blocks < b (its base inside the expert's segment).
__global__ __launch_bounds__(kGroupThreads) void grouping_scan(int nblocks, int E, int BM,
                                                               int32_t* __restrict__ block_counts,
                                                               int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ tile_row,
                                                               int32_t* __restrict__ tile_exp,
                                                               int32_t* __restrict__ num_tiles) {
    extern __shared__ int32_t s_tot[];  // [E] totals, then [E] tile bases
    int32_t* s_tb = s_tot + E;
    for (int e = threadIdx.x; e < E; e += kGroupThreads) {
        int32_t run = 0;
        for (int b = 0; b < nblocks; ++b) {
            const long long o = (long long)b * E + e;
            const int32_t c = block_counts[o];
            block_counts[o] = run;
            run += c;
        }
        s_tot[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t sum = 0, mx = 0, tiles = 0;
        for (int e = 0; e < E; ++e) {
            const int32_t c = s_tot[e];
            offsets[e] = sum;
            s_tb[e] = tiles;
            mx = c > mx ? c : mx;
            sum += c;
            tiles += (c + BM - 1) / BM;
        }
        offsets[E] = sum;
        offsets[E + 1] = mx;
        *num_tiles = tiles;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kGroupThreads) {
        const int32_t c = s_tot[e];
        const int32_t nt = (c + BM - 1) / BM;
        const int32_t o = offsets[e];
        const int32_t tb = s_tb[e];
        for (int i = 0; i < nt; ++i) {
            tile_row[tb + i] = o + i * BM;
            tile_exp[tb + i] = e;
        }
    }
}

__global__ __launch_bounds__(kGroupThreads) void grouping_scatter(const uint32_t* __restrict__ idx, long long P,
                                                                  int E, int ebits,
                                                                  const int32_t* __restrict__ block_counts,
                                                                  const int32_t* __restrict__ offsets,
                                                                  int32_t* __restrict__ sorted_pair) {
    extern __shared__ int32_t s_mem[];
    int32_t* s_run = s_mem;           // [E] next free position per expert
    int32_t* s_wc = s_mem + E;        // [4][E] per-wave counts of the current step
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    for (int e = threadIdx.x; e < E; e += kGroupThreads) {
        s_run[e] = offsets[e] + block_counts[(long long)blockIdx.x * E + e];
        s_wc[e] = s_wc[E + e] = s_wc[2 * E + e] = s_wc[3 * E + e] = 0;
    }
    __syncthreads();
    const long long base = (long long)blockIdx.x * kGroupChunk;
    const long long end = base + kGroupChunk < P ? base + kGroupChunk : P;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (long long s = base; s < end; s += kGroupThreads) {
        const long long p = s + threadIdx.x;
        const uint32_t e = p < end ? idx[p] : 0xffffffffu;
        const bool active = e < (uint32_t)E;
        // Lanes of this wave holding the same expert: AND of per-bit ballots.
        uint64_t peers = __ballot(active);
        for (int b = 0; b < ebits; ++b) {
            const bool bit = (e >> b) & 1u;
            const uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const int rank = __popcll(peers & lt_mask);
        if (active && rank == 0) s_wc[wave * E + e] = __popcll(peers);
        __syncthreads();
        if (active) {
            int32_t pos = s_run[e] + rank;
            for (int w = 0; w < wave; ++w) pos += s_wc[w * E + e];
            sorted_pair[pos] = (int32_t)p;
        }
        __syncthreads();
        for (int ee = threadIdx.x; ee < E; ee += kGroupThreads) {
            s_run[ee] += s_wc[ee] + s_wc[E + ee] + s_wc[2 * E + ee] + s_wc[3 * E + ee];
            s_wc[ee] = s_wc[E + ee] = s_wc[2 * E + ee] = s_wc[3 * E + ee] = 0;
        }
        __syncthreads();
    }
}

hipError_t launch_grouping(const uint32_t* idx, long long P, int E, int BM, const GroupingBufs& b,
                           hipStream_t stream) {
    const int nb = grouping_blocks(P);
    int ebits = 0;
    while ((1 << ebits) < E) ++ebits;
    if (nb > 0) {
        hipLaunchKernelGGL(grouping_hist, dim3(nb), dim3(kGroupThreads), 4 * E * sizeof(int32_t), stream, idx, P,
                           E, b.block_counts);
    }
    hipLaunchKernelGGL(grouping_scan, dim3(1), dim3(kGroupThreads), 2 * E * sizeof(int32_t), stream, nb, E, BM,
                       b.block_counts, b.offsets, b.tile_row, b.tile_exp, b.num_tiles);
    if (nb > 0) {
        hipLaunchKernelGGL(grouping_scatter, dim3(nb), dim3(kGroupThreads), 5 * E * sizeof(int32_t), stream, idx, P,
                           E, ebits, b.block_counts, b.offsets, b.sorted_pair);
    }
    return hipGetLastError();
}

}  // namespace cm
