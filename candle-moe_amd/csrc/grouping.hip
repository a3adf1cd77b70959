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
// Up to kGroupSmallMax items one workgroup does everything (small_body).
// Beyond that, three phases, no host synchronisation:
//   1. hist_body   : each workgroup histograms kGroupChunk items in LDS
//   2. scan_body   : one workgroup turns the per-block counts into per-block
//                    bases (one wave-wide scan per bin), the bin offsets and
//                    the tile table
//   3. scatter_body: each workgroup re-reads its chunk and ranks items
//                    stably: 64-lane peer masks from ballots inside a wave,
//                    per-wave running counts in LDS, one barrier to turn the
//                    per-wave counts into bases
// The same code groups tokens by their expert set (TOK = true) for the
// expert-set down projection. The pair grouping and the token grouping share
// three launches (grouping_hist_k, grouping_mid_k, grouping_scatter_k), each
// workgroup serving one of the two jobs; a small job runs whole in the
// middle launch, so decode groupings take one launch.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

constexpr int kGroupThreads = 256;
constexpr int kScanStageMax = 8192;  // block counts staged in LDS by the scan (32 KB)

// Token t's expert set: its k ids with ids >= E replaced by E, sorted
// ascending (stable in j); the key reads them as base-(E+1) digits, most
// significant first. rank[j] is slot j's position in that order.
__device__ __forceinline__ int token_set_key(const uint32_t* __restrict__ idx, long long t, int k, int E,
                                             int (&rank)[kSetMaxK]) {
    int ex[kSetMaxK];
    for (int j = 0; j < k; ++j) {
        const uint32_t v = idx[t * k + j];
        ex[j] = v < (uint32_t)E ? (int)v : E;
    }
    int key = 0;
    for (int j = 0; j < k; ++j) {
        int r = 0;
        for (int i = 0; i < k; ++i) r += (ex[i] < ex[j]) || (ex[i] == ex[j] && i < j);
        rank[j] = r;
    }
    // digits in sorted order: position r holds the slot with rank r
    for (int r = 0; r < k; ++r) {
        int d = E;
        for (int j = 0; j < k; ++j) d = (rank[j] == r) ? ex[j] : d;
        key = key * (E + 1) + d;
    }
    return key;
}

// Bin of item i: the expert of pair i (TOK = false, -1 if dropped), or the
// expert-set key of token i (TOK = true).
template <bool TOK>
__device__ __forceinline__ int item_bin(const uint32_t* __restrict__ idx, long long i, int k, int E,
                                        int (&rank)[kSetMaxK]) {
    if constexpr (TOK) {
        return token_set_key(idx, i, k, E, rank);
    } else {
        const uint32_t e = __builtin_nontemporal_load(idx + i);
        return e < (uint32_t)E ? (int)e : -1;
    }
}

// Histogram of block blk of job j into s_cnt ([4 waves][nbins] of LDS).
template <bool TOK>
__device__ void hist_body(const GroupJob& j, int blk, int32_t* s_cnt) {
    const uint32_t* __restrict__ idx = j.idx;
    const long long P = j.items;
    const int k = j.k, E = j.E, nbins = j.nbins;
    int32_t* __restrict__ block_counts = j.b.block_counts;
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * nbins; i += kGroupThreads) s_cnt[i] = 0;
    __syncthreads();
    constexpr int IPT = kGroupChunk / kGroupThreads;  // items per thread
    const long long base = (long long)blk * kGroupChunk;
    int32_t* mine = s_cnt + wave * nbins;
    int rank[kSetMaxK];
    // the bins of all IPT items first, so that their loads are in flight
    // together, then the LDS counts
    int bin[IPT];
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const long long p = base + s * kGroupThreads + threadIdx.x;
        bin[s] = p < P ? item_bin<TOK>(idx, p, k, E, rank) : -1;
    }
#pragma unroll
    for (int s = 0; s < IPT; ++s)
        if (bin[s] >= 0) atomicAdd(mine + bin[s], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads)
        block_counts[(long long)blk * nbins + e] =
            s_cnt[e] + s_cnt[nbins + e] + s_cnt[2 * nbins + e] + s_cnt[3 * nbins + e];
}

// Exclusive scans of u[0..n) and v[0..n) in place (one workgroup of
// kGroupThreads), returning the totals; s_part is 8 ints of scratch. Each
// thread scans a contiguous run of ceil(n / threads) entries of both; the
// per-thread sums are scanned inside each wave by shuffles and across the 4
// waves through LDS (two barriers).
__device__ void block_exclusive_scan2(int32_t* u, int32_t* v, int n, int32_t* s_part, int32_t& total_u,
                                      int32_t& total_v) {
    constexpr int NW = kGroupThreads / 64;
    const int per = (n + kGroupThreads - 1) / kGroupThreads;
    const int lo = threadIdx.x * per;
    const int hi = lo + per < n ? lo + per : n;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int32_t ru = 0, rv = 0;
    for (int i = lo; i < hi; ++i) {
        ru += u[i];
        rv += v[i];
    }
    int32_t iu = ru, iv = rv;  // inclusive within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t tu = __shfl_up(iu, d), tv = __shfl_up(iv, d);
        if (lane >= d) {
            iu += tu;
            iv += tv;
        }
    }
    if (lane == 63) {
        s_part[wave] = iu;
        s_part[NW + wave] = iv;
    }
    __syncthreads();
    int32_t bu = iu - ru, bv = iv - rv;
    total_u = 0;
    total_v = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int32_t wu = s_part[w], wv = s_part[NW + w];
        if (w < wave) {
            bu += wu;
            bv += wv;
        }
        total_u += wu;
        total_v += wv;
    }
    for (int i = lo; i < hi; ++i) {
        const int32_t cu = u[i], cv = v[i];
        u[i] = bu;
        v[i] = bv;
        bu += cu;
        bv += cv;
    }
    __syncthreads();
}

// One workgroup. block_counts[b][e] becomes the number of bin-e items in
// blocks < b (its base inside the bin's segment): bins go round-robin to the
// waves, each scans its bin over the blocks 64 at a time. Then the bin totals
// and tile counts are scanned into offsets and the tile table. Also clears
// zero_n ints at zero_ptr (the split-K arrival counters of the GEMMs).
__device__ void scan_body(const GroupJob& j, int32_t* s_tot) {
    // LDS: [nbins] totals -> offsets, [nbins] tile counts -> bases, [threads],
    // then (when it fits) the [nblocks][nbins] block counts, staged so that each
    // bin is scanned by one thread from LDS; otherwise bins go round-robin to
    // the waves, which scan them from global memory 64 blocks at a time
    const int nblocks = j.nb, nbins = j.nbins, BM = j.BM;
    int32_t* __restrict__ block_counts = j.b.block_counts;
    int32_t* __restrict__ offsets = j.b.offsets;
    int32_t* __restrict__ tile_row = j.b.tile_row;
    int32_t* __restrict__ tile_exp = j.b.tile_exp;
    int32_t* __restrict__ num_tiles = j.b.num_tiles;
    int32_t* __restrict__ zero_ptr = j.b.zero_ptr;
    const int zero_n = j.b.zero_n;
    int32_t* s_tb = s_tot + nbins;
    int32_t* s_part = s_tb + nbins;
    __shared__ int32_t s_max;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ncounts = nblocks * nbins;
    const bool staged = ncounts <= kScanStageMax;
    int32_t* s_bc = s_part + kGroupThreads;
    if (threadIdx.x == 0) s_max = 0;
    for (int i = threadIdx.x; i < zero_n; i += kGroupThreads) zero_ptr[i] = 0;
    if (staged) {
        for (int i = threadIdx.x; i < ncounts; i += kGroupThreads) s_bc[i] = block_counts[i];
        __syncthreads();
    }
    // Few bins over many blocks (the pair grouping): each wave scans whole
    // bins, its lanes over the blocks 64 at a time. Otherwise (the token-set
    // grouping: many bins, fewer blocks) one thread per bin walks its column
    // of the staged counts (the LDS reads are independent, only the running
    // sum is serial).
    const bool by_wave = !staged || ((nbins + kGroupThreads / 64 - 1) / (kGroupThreads / 64)) * 2 < nblocks;
    if (staged && !by_wave) {
        for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
            int32_t run = 0;
            for (int b = 0; b < nblocks; ++b) {
                const int32_t c = s_bc[b * nbins + e];
                s_bc[b * nbins + e] = run;
                run += c;
            }
            s_tot[e] = run;
            s_tb[e] = (run + BM - 1) / BM;
        }
    }
    int32_t* bc = staged ? s_bc : block_counts;
    for (int e = wave; e < (by_wave ? nbins : 0); e += kGroupThreads / 64) {
        int32_t carry = 0;
        for (int b0 = 0; b0 < nblocks; b0 += 64) {
            const int b = b0 + lane;
            const long long o = (long long)b * nbins + e;
            const int32_t c = b < nblocks ? bc[o] : 0;
            int32_t incl = c;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int32_t t = __shfl_up(incl, d);
                if (lane >= d) incl += t;
            }
            if (b < nblocks) bc[o] = carry + incl - c;
            carry += __shfl(incl, 63);
        }
        if (lane == 0) {
            s_tot[e] = carry;
            s_tb[e] = (carry + BM - 1) / BM;
        }
    }
    __syncthreads();
    if (staged)
        for (int i = threadIdx.x; i < ncounts; i += kGroupThreads) block_counts[i] = s_bc[i];
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) atomicMax(&s_max, s_tot[e]);
    int32_t total, tiles;
    block_exclusive_scan2(s_tot, s_tb, nbins, s_part, total, tiles);
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        offsets[e] = s_tot[e];
        const int32_t c = (e + 1 < nbins ? s_tot[e + 1] : total) - s_tot[e];
        const int32_t nt = (c + BM - 1) / BM;
        for (int i = 0; i < nt; ++i) {
            tile_row[s_tb[e] + i] = s_tot[e] + i * BM;
            tile_exp[s_tb[e] + i] = e;
        }
    }
    if (threadIdx.x == 0) {
        offsets[nbins] = total;
        offsets[nbins + 1] = s_max;
        *num_tiles = tiles;
    }
}

// Stable scatter of one kGroupChunk block. Wave w ranks items
// [w*64*IPT, (w+1)*64*IPT) of the block, 64 at a time: lanes holding the same
// bin find each other with ballots over the bin's bits, and a per-wave LDS
// count per bin carries the rank from one step to the next. After one barrier
// the per-wave counts become per-wave bases (block base of the bin + counts
// of the waves before), and every item goes to base + its rank.
template <bool TOK>
__device__ void scatter_body(const GroupJob& j, int blk, int32_t* s_wc) {
    constexpr int NW = kGroupThreads / 64;
    constexpr int IPT = kGroupChunk / kGroupThreads;  // items per lane
    // LDS s_wc: [NW][nbins] per-wave counts, then bases
    const uint32_t* __restrict__ idx = j.idx;
    const long long P = j.items;
    const int k = j.k, E = j.E, nbins = j.nbins, ebits = j.ebits;
    const int32_t* __restrict__ block_counts = j.b.block_counts;
    const int32_t* __restrict__ offsets = j.b.offsets;
    int32_t* __restrict__ sorted_pair = j.b.sorted_pair;
    int32_t* __restrict__ pair_dest = j.pair_dest;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < NW * nbins; i += kGroupThreads) s_wc[i] = 0;
    __syncthreads();
    int32_t* mine = s_wc + wave * nbins;
    const long long wbase = (long long)blk * kGroupChunk + wave * 64 * IPT;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int bin[IPT], lrank[IPT];
    int rank[kSetMaxK];
    // the bins first, so that the loads of all IPT items are in flight together
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const long long p = wbase + s * 64 + lane;
        bin[s] = p < P ? item_bin<TOK>(idx, p, k, E, rank) : -1;
    }
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const int b = bin[s];
        const bool active = b >= 0;
        const uint32_t e = active ? (uint32_t)b : 0xffffffffu;
        uint64_t peers = __ballot(active);
        for (int i = 0; i < ebits; ++i) {
            const bool bit = (e >> i) & 1u;
            const uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const int r = __popcll(peers & lt_mask);
        // every lane reads the running count before the bin's first lane
        // stores the new one (LDS instructions of a wave execute in order)
        const int before = active ? mine[b] : 0;
        if (active && r == 0) mine[b] = before + __popcll(peers);
        lrank[s] = before + r;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        int32_t run = offsets[e] + block_counts[(long long)blk * nbins + e];
        for (int w = 0; w < NW; ++w) {
            const int32_t c = s_wc[w * nbins + e];
            s_wc[w * nbins + e] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        if (bin[s] < 0) continue;
        const long long p = wbase + s * 64 + lane;
        const int32_t pos = mine[bin[s]] + lrank[s];
        sorted_pair[pos] = (int32_t)p;
        if constexpr (TOK) {
            (void)token_set_key(idx, p, k, E, rank);
            for (int j = 0; j < k; ++j) pair_dest[p * k + j] = pos * k + rank[j];
        }
    }
}

// All of grouping in one workgroup, for at most kGroupSmallMax items. Wave w
// takes items [w*64*IPT, (w+1)*64*IPT), 64 at a time, reads their bins once
// (all loads in flight together) and ranks them stably as the scatter phase
// does (ballot peer masks, per-wave running counts in LDS); the per-wave
// counts give the bin totals, whose scans give the offsets and the tile
// table, and then per-wave bases, so each item goes to base + its rank. Also
// clears zero_n ints at zero_ptr (the split-K arrival counters of the GEMMs
// that follow).
template <bool TOK>
__device__ void small_body(const GroupJob& j, int32_t* s_mem) {
    constexpr int NW = kGroupThreads / 64;
    constexpr int IPT = kGroupSmallMax / kGroupThreads;  // items per lane
    const uint32_t* __restrict__ idx = j.idx;
    const int P = (int)j.items, k = j.k, E = j.E, nbins = j.nbins, ebits = j.ebits, BM = j.BM;
    int32_t* __restrict__ offsets = j.b.offsets;
    int32_t* __restrict__ sorted_pair = j.b.sorted_pair;
    int32_t* __restrict__ tile_row = j.b.tile_row;
    int32_t* __restrict__ tile_exp = j.b.tile_exp;
    int32_t* __restrict__ num_tiles = j.b.num_tiles;
    int32_t* __restrict__ pair_dest = j.pair_dest;
    int32_t* __restrict__ zero_ptr = j.b.zero_ptr;
    const int zero_n = j.b.zero_n;
    int32_t* s_cnt = s_mem;               // [NW][nbins] per-wave counts, then per-wave bases
    int32_t* s_off = s_mem + NW * nbins;  // [nbins] bin totals -> offsets
    int32_t* s_tb = s_off + nbins;        // [nbins] tile counts -> tile bases
    int32_t* s_part = s_tb + nbins;       // scan scratch
    __shared__ int32_t s_max;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wbase = wave * 64 * IPT;
    int bin[IPT], lrank[IPT];
    int rank[kSetMaxK];
    // the bins first: the loads of all IPT items are in flight together
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const int p = wbase + s * 64 + lane;
        bin[s] = p < P ? item_bin<TOK>(idx, p, k, E, rank) : -1;
    }
    for (int i = threadIdx.x; i < zero_n; i += kGroupThreads) zero_ptr[i] = 0;
    for (int i = threadIdx.x; i < NW * nbins; i += kGroupThreads) s_cnt[i] = 0;
    if (threadIdx.x == 0) s_max = 0;
    __syncthreads();
    int32_t* mine = s_cnt + wave * nbins;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        if (wbase + s * 64 >= P) break;  // wave-uniform
        const int b = bin[s];
        const bool active = b >= 0;
        const uint32_t e = active ? (uint32_t)b : 0xffffffffu;
        uint64_t peers = __ballot(active);
        for (int i = 0; i < ebits; ++i) {
            const bool bit = (e >> i) & 1u;
            const uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const int r = __popcll(peers & lt_mask);
        // every lane reads the running count before the bin's first lane
        // stores the new one (LDS instructions of a wave execute in order)
        const int before = active ? mine[b] : 0;
        if (active && r == 0) mine[b] = before + __popcll(peers);
        lrank[s] = before + r;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        int32_t c = 0;
        for (int w = 0; w < NW; ++w) c += s_cnt[w * nbins + e];
        s_off[e] = c;
        s_tb[e] = (c + BM - 1) / BM;
        atomicMax(&s_max, c);
    }
    __syncthreads();
    int32_t total, tiles;
    block_exclusive_scan2(s_off, s_tb, nbins, s_part, total, tiles);
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        offsets[e] = s_off[e];
        const int32_t c = (e + 1 < nbins ? s_off[e + 1] : total) - s_off[e];
        const int32_t nt = (c + BM - 1) / BM;
        for (int i = 0; i < nt; ++i) {
            tile_row[s_tb[e] + i] = s_off[e] + i * BM;
            tile_exp[s_tb[e] + i] = e;
        }
        // per-wave bases of bin e: its offset plus the counts of earlier waves
        int32_t run = s_off[e];
        for (int w = 0; w < NW; ++w) {
            const int32_t t = s_cnt[w * nbins + e];
            s_cnt[w * nbins + e] = run;
            run += t;
        }
    }
    if (threadIdx.x == 0) {
        offsets[nbins] = total;
        offsets[nbins + 1] = s_max;
        *num_tiles = tiles;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        if (bin[s] < 0) continue;
        const int p = wbase + s * 64 + lane;
        const int32_t pos = mine[bin[s]] + lrank[s];
        sorted_pair[pos] = p;
        if constexpr (TOK) {
            (void)token_set_key(idx, p, k, E, rank);
            for (int jj = 0; jj < k; ++jj) pair_dest[(long long)p * k + jj] = pos * k + rank[jj];
        }
    }
}

// The three launches serve the pair grouping (A) and, on the expert-set path,
// the token grouping (B) together: workgroups [0, A.nb) work on A and the rest
// on B; in the middle launch workgroup 0 is A's scan (or its whole grouping if
// A is small) and workgroup 1 the same for B.
__global__ __launch_bounds__(kGroupThreads) void grouping_hist_k(GroupJob A, GroupJob B) {
    extern __shared__ int32_t s_dyn[];
    const int a_nb = A.small ? 0 : A.nb;
    if ((int)blockIdx.x < a_nb) hist_body<false>(A, blockIdx.x, s_dyn);
    else hist_body<true>(B, blockIdx.x - a_nb, s_dyn);
}
__global__ __launch_bounds__(kGroupThreads) void grouping_mid_k(GroupJob A, GroupJob B, int has_b) {
    extern __shared__ int32_t s_dyn[];
    if (blockIdx.x == 0) {
        if (A.small) small_body<false>(A, s_dyn);
        else scan_body(A, s_dyn);
    } else if (has_b) {
        if (B.small) small_body<true>(B, s_dyn);
        else scan_body(B, s_dyn);
    }
}
__global__ __launch_bounds__(kGroupThreads) void grouping_scatter_k(GroupJob A, GroupJob B) {
    extern __shared__ int32_t s_dyn[];
    const int a_nb = A.small ? 0 : A.nb;
    if ((int)blockIdx.x < a_nb) scatter_body<false>(A, blockIdx.x, s_dyn);
    else scatter_body<true>(B, blockIdx.x - a_nb, s_dyn);
}

static GroupJob make_job(const uint32_t* idx, long long items, int k, int E, int nbins, int BM,
                         const GroupingBufs& b, int32_t* pair_dest) {
    GroupJob j = {};
    j.idx = idx;
    j.items = items;
    j.k = k;
    j.E = E;
    j.nbins = nbins;
    j.BM = BM;
    j.b = b;
    j.pair_dest = pair_dest;
    while ((1 << j.ebits) < nbins) ++j.ebits;
    // one workgroup does everything up to kGroupSmallMax items (LDS of the
    // one-workgroup path: 6 * nbins + threads ints)
    j.small = items <= kGroupSmallMax && (6LL * nbins + kGroupThreads) * 4 <= 64 * 1024;
    j.nb = grouping_blocks(items);
    return j;
}

GroupJob pair_grouping_job(const uint32_t* idx, long long P, int E, int BM, const GroupingBufs& b) {
    return make_job(idx, P, 1, E, E, BM, b, nullptr);
}

GroupJob set_grouping_job(const uint32_t* idx, int T, int k, int E, int nkeys, int BM, const GroupingBufs& b,
                          int32_t* pair_dest) {
    return make_job(idx, T, k, E, nkeys, BM, b, pair_dest);
}

hipError_t launch_groupings(const GroupJob& A, const GroupJob* B, hipStream_t stream) {
    if (B && (B->k < 1 || B->k > kSetMaxK || B->nbins > kSetMaxKeys)) return hipErrorInvalidValue;
    GroupJob b = B ? *B : GroupJob{};
    if (!B) b.small = true;  // nothing of B in the multi-workgroup launches
    const int nb_multi = (A.small ? 0 : A.nb) + (b.small ? 0 : b.nb);
    auto ints = [](long long n) { return (size_t)n * sizeof(int32_t); };
    const int bins_multi = std::max(A.small ? 0 : A.nbins, b.small ? 0 : b.nbins);
    if (nb_multi > 0) {
        hipLaunchKernelGGL(grouping_hist_k, dim3(nb_multi), dim3(kGroupThreads), ints(4LL * bins_multi), stream, A, b);
    }
    auto mid_lds = [&](const GroupJob& j) {
        const long long counts = (long long)j.nb * j.nbins;
        return j.small ? 6LL * j.nbins + kGroupThreads
                       : 2LL * j.nbins + kGroupThreads + (counts <= kScanStageMax ? counts : 0);
    };
    const long long mid = std::max(mid_lds(A), B ? mid_lds(*B) : 0LL);
    hipLaunchKernelGGL(grouping_mid_k, dim3(B ? 2 : 1), dim3(kGroupThreads), ints(mid), stream, A, b, B ? 1 : 0);
    if (nb_multi > 0) {
        hipLaunchKernelGGL(grouping_scatter_k, dim3(nb_multi), dim3(kGroupThreads), ints(4LL * bins_multi), stream, A,
                           b);
    }
    return hipGetLastError();
}

}  // namespace cm
