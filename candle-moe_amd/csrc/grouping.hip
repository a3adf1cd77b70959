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
// Up to kGroupSmallMax items one workgroup does everything (small_body), one
// launch. Beyond that, one launch where the workspace's counters are known
// to start at zero (one_launch_body: the two phases below with a bounded
// wait between them), else two launches, no host synchronisation:
//   1. hist_body   : each workgroup histograms kGroupChunk items in LDS and
//                    stores its per-bin counts
//   2. scatter_body: each workgroup stages every block's counts in LDS (all
//                    loads in flight together), sums each bin over all blocks
//                    and over the blocks before its own (the bin totals give
//                    the offsets by one block-wide scan, which workgroup 0
//                    also writes out with the tile table), then ranks its
//                    items stably -- 64-lane peer masks from ballots inside a
//                    wave, per-wave running counts in LDS, one barrier to
//                    turn the per-wave counts into bases -- and scatters them.
//                    Every workgroup repeats the small scan instead of one
//                    workgroup doing it in a launch of its own in between.
// The same code groups tokens by their expert set (TOK = true, k a template
// parameter so that a token's k ids load together) for the expert-set down
// projection. The pair grouping and the token grouping share the launches,
// each workgroup serving one of the two jobs.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

constexpr int kGroupThreads = 256;


// Token t's expert set: its K ids with ids >= E replaced by E, sorted
// ascending (stable in j); the key reads them as base-(E+1) digits, most
// significant first. rank[j] is slot j's position in that order.
template <int K>
__device__ __forceinline__ int token_set_key_of(const uint32_t (&raw)[K], int E, int (&rank)[K]) {
    int ex[K];
#pragma unroll
    for (int j = 0; j < K; ++j) ex[j] = raw[j] < (uint32_t)E ? (int)raw[j] : E;
    int key = 0;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        int r = 0;
#pragma unroll
        for (int i = 0; i < K; ++i) r += (ex[i] < ex[j]) || (ex[i] == ex[j] && i < j);
        rank[j] = r;
    }
    // digits in sorted order: position r holds the slot with rank r
#pragma unroll
    for (int r = 0; r < K; ++r) {
        int d = E;
#pragma unroll
        for (int j = 0; j < K; ++j) d = (rank[j] == r) ? ex[j] : d;
        key = key * (E + 1) + d;
    }
    return key;
}

// The expert ids of item i (TOK: the K ids of token i; else pair i's id),
// loaded apart from their use so that a caller can have other loads in
// flight before it waits for these.
template <bool TOK, int K>
__device__ __forceinline__ void item_load(const uint32_t* __restrict__ idx, long long i, uint32_t (&raw)[K]) {
    if constexpr (TOK) {
#pragma unroll
        for (int j = 0; j < K; ++j) raw[j] = idx[i * K + j];
    } else {
        raw[0] = __builtin_nontemporal_load(idx + i);
    }
}
// Bin of an item from its ids: the expert of a pair (-1 if dropped), or the
// expert-set key of a token.
template <bool TOK, int K>
__device__ __forceinline__ int item_bin_of(const uint32_t (&raw)[K], int E, int (&rank)[K]) {
    if constexpr (TOK) {
        return token_set_key_of<K>(raw, E, rank);
    } else {
        return raw[0] < (uint32_t)E ? (int)raw[0] : -1;
    }
}
template <bool TOK, int K>
__device__ __forceinline__ int item_bin(const uint32_t* __restrict__ idx, long long i, int E, int (&rank)[K]) {
    uint32_t raw[K];
    item_load<TOK, K>(idx, i, raw);
    return item_bin_of<TOK, K>(raw, E, rank);
}

// Histogram of block blk of job j into s_cnt ([4 waves][nbins] of LDS),
// stored to block_counts (COH: device-coherent stores, read by other
// workgroups of the same launch).
template <bool TOK, int K, bool COH = false>
__device__ void hist_body(const GroupJob& j, int blk, int32_t* s_cnt) {
    const uint32_t* __restrict__ idx = j.idx;
    const long long P = j.items;
    const int E = j.E, nbins = j.nbins;
    int32_t* __restrict__ block_counts = j.b.block_counts;
    const int wave = threadIdx.x >> 6;
    constexpr int IPT = kGroupChunk / kGroupThreads;  // items per thread
    const long long base = (long long)blk * kGroupChunk;
    int32_t* mine = s_cnt + wave * nbins;
    int rank[K];
    // the bins of all IPT items first, so that their loads are in flight
    // together (and under the LDS clear), then the LDS counts
    int bin[IPT];
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const long long p = base + s * kGroupThreads + threadIdx.x;
        bin[s] = p < P ? item_bin<TOK, K>(idx, p, E, rank) : -1;
    }
    for (int i = threadIdx.x; i < 4 * nbins; i += kGroupThreads) s_cnt[i] = 0;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < IPT; ++s)
        if (bin[s] >= 0) atomicAdd(mine + bin[s], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        const int32_t c = s_cnt[e] + s_cnt[nbins + e] + s_cnt[2 * nbins + e] + s_cnt[3 * nbins + e];
        if constexpr (COH)
            __hip_atomic_store(block_counts + (long long)blk * nbins + e, c, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        else
            block_counts[(long long)blk * nbins + e] = c;
    }
}

// Exclusive scans of u[0..n) and v[0..n) in place (one workgroup of
// kGroupThreads), returning the totals and the largest u; s_part is 12 ints
// of scratch. Each
// thread scans a contiguous run of ceil(n / threads) entries of both; the
// per-thread sums are scanned inside each wave by shuffles and across the 4
// waves through LDS (two barriers).
__device__ void block_exclusive_scan2(int32_t* u, int32_t* v, int n, int32_t* s_part, int32_t& total_u,
                                      int32_t& total_v, int32_t& max_u) {
    constexpr int NW = kGroupThreads / 64;
    const int per = (n + kGroupThreads - 1) / kGroupThreads;
    const int lo = threadIdx.x * per;
    const int hi = lo + per < n ? lo + per : n;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int32_t ru = 0, rv = 0, mu = 0;
    for (int i = lo; i < hi; ++i) {
        ru += u[i];
        rv += v[i];
        mu = u[i] > mu ? u[i] : mu;
    }
    // largest u: wave butterfly, then the wave maxima through LDS (one
    // same-address LDS atomic per lane serialises at full latency)
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t t = __shfl_xor(mu, d);
        mu = t > mu ? t : mu;
    }
    if (lane == 0) s_part[2 * NW + wave] = mu;
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
    max_u = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int32_t wu = s_part[w], wv = s_part[NW + w], wm = s_part[2 * NW + w];
        if (w < wave) {
            bu += wu;
            bv += wv;
        }
        total_u += wu;
        total_v += wv;
        max_u = wm > max_u ? wm : max_u;
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

// Stable scatter of one kGroupChunk block, with the scan of the block counts
// done by every workgroup for itself. The counts of all blocks (the previous
// launch's output) give, per bin, the total over all blocks and the base over
// the blocks before this one. Wave w ranks items [w*64*IPT, (w+1)*64*IPT) of
// the block, 64 at a time: lanes holding the same bin find each other with
// ballots over the bin's bits, and a per-wave LDS count per bin carries the
// rank from one step to the next. One block-wide scan of the totals gives the
// bin offsets (workgroup 0 also stores offsets, tile table, tile count, the
// largest bin, and clears zero_n ints at zero_ptr).
// After one more barrier the per-wave counts become per-wave positions and
// every item goes to position + its rank.
// LDS: [NW][nbins] per-wave counts, [nbins] totals, [nbins] tile counts,
// [nbins] bases, [threads] scan scratch.
// Where scatter_body takes the per-block counts from: the previous launch's
// table, this launch's table (written by the other workgroups with
// device-coherent stores before they counted themselves in), or a recount of
// every item by this workgroup alone.
enum CountSrc : int { kCountsPrevLaunch = 0, kCountsCoherent = 1, kCountsRecount = 2 };
template <bool TOK, int K>
__device__ void scatter_body(const GroupJob& j, int blk, int32_t* s_mem, int src = kCountsPrevLaunch) {
    constexpr int NW = kGroupThreads / 64;
    constexpr int IPT = kGroupChunk / kGroupThreads;  // items per lane
    const uint32_t* __restrict__ idx = j.idx;
    const long long P = j.items;
    const int E = j.E, nbins = j.nbins, ebits = j.ebits, BM = j.BM, nblocks = j.nb;
    const int32_t* __restrict__ block_counts = j.b.block_counts;
    int32_t* __restrict__ sorted_pair = j.b.sorted_pair;
    int32_t* __restrict__ pair_dest = j.pair_dest;
    int32_t* s_wc = s_mem;
    int32_t* s_tot = s_wc + NW * nbins;
    int32_t* s_tb = s_tot + nbins;
    int32_t* s_base = s_tb + nbins;
    int32_t* s_part = s_base + nbins;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const long long wbase = (long long)blk * kGroupChunk + wave * 64 * IPT;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int bin[IPT], lrank[IPT];
    int rank[IPT][K];  // slot ranks of each token in its expert set (TOK)
    // Global loads first, all in flight together: this block's items, then
    // the first round of the count table. Bin totals over all blocks and bases
    // over the blocks before this one are summed by groups of G lanes per bin
    // (G a power of two, G * nbins <= threads): lane j of bin e's group adds
    // blocks j, j + G, ... in registers, a butterfly over the group's lanes
    // sums the G parts (no LDS atomics: same-address ones serialise).
    uint32_t raw[IPT][K];
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const long long p = wbase + s * 64 + lane;
        if (p < P) item_load<TOK, K>(idx, p, raw[s]);
    }
    if (src == kCountsRecount) {
        // every block's histogram again, one block at a time (the fallback
        // of the one-launch grouping; per-wave LDS counts in s_wc)
        for (int e = threadIdx.x; e < nbins; e += kGroupThreads) s_tot[e] = s_base[e] = 0;
        constexpr int HIPT = kGroupChunk / kGroupThreads;
        int rk[K];
        for (int b2 = 0; b2 < nblocks; ++b2) {
            int hb[HIPT];
#pragma unroll
            for (int q = 0; q < HIPT; ++q) {
                const long long p = (long long)b2 * kGroupChunk + q * kGroupThreads + threadIdx.x;
                hb[q] = p < P ? item_bin<TOK, K>(idx, p, E, rk) : -1;
            }
            for (int i = threadIdx.x; i < NW * nbins; i += kGroupThreads) s_wc[i] = 0;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < HIPT; ++q)
                if (hb[q] >= 0) atomicAdd(s_wc + wave * nbins + hb[q], 1);
            __syncthreads();
            for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
                int32_t c = 0;
                for (int w = 0; w < NW; ++w) c += s_wc[w * nbins + e];
                s_tot[e] += c;
                if (b2 < blk) s_base[e] += c;
            }
            __syncthreads();
        }
    }
    int G = 1;
    while (G < 64 && 2 * G * nbins <= kGroupThreads) G *= 2;
    const int gj = (int)threadIdx.x & (G - 1), ge = (int)threadIdx.x / G, estep = kGroupThreads / G;
    constexpr int U = 16;
    for (int e0 = 0; src != kCountsRecount && e0 < nbins; e0 += estep) {
        const int e = e0 + ge;
        int32_t tot = 0, bas = 0;
        for (int b0 = gj; b0 < nblocks; b0 += U * G) {
            int32_t c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int b2 = b0 + u * G;
                c[u] = 0;
                if (e < nbins && b2 < nblocks)
                    c[u] = src == kCountsCoherent
                               ? __hip_atomic_load(block_counts + b2 * nbins + e, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : block_counts[b2 * nbins + e];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                tot += c[u];
                bas += (b0 + u * G < blk) ? c[u] : 0;
            }
        }
        for (int m = 1; m < G; m <<= 1) {
            tot += __shfl_xor(tot, m);
            bas += __shfl_xor(bas, m);
        }
        if (e < nbins && gj == 0) {
            s_tot[e] = tot;
            s_base[e] = bas;
        }
    }
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const long long p = wbase + s * 64 + lane;
        bin[s] = p < P ? item_bin_of<TOK, K>(raw[s], E, rank[s]) : -1;
    }
    for (int i = threadIdx.x; i < NW * nbins; i += kGroupThreads) s_wc[i] = 0;
    __syncthreads();
    int32_t* mine = s_wc + wave * nbins;
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
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) s_tb[e] = (s_tot[e] + BM - 1) / BM;
    __syncthreads();
    int32_t total, tiles, largest;
    block_exclusive_scan2(s_tot, s_tb, nbins, s_part, total, tiles, largest);  // s_tot -> offsets
    if (blk == 0) {
        int32_t* __restrict__ offsets = j.b.offsets;
        int32_t* __restrict__ tile_row = j.b.tile_row;
        int32_t* __restrict__ tile_exp = j.b.tile_exp;
        for (int i = threadIdx.x; i < j.b.zero_n; i += kGroupThreads) j.b.zero_ptr[i] = 0;
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
            offsets[nbins + 1] = largest;
            *j.b.num_tiles = tiles;
        }
    }
    // per-wave positions: bin offset + blocks before + waves before
    for (int e = threadIdx.x; e < nbins; e += kGroupThreads) {
        int32_t run = s_tot[e] + s_base[e];
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
#pragma unroll
            for (int jj = 0; jj < K; ++jj) pair_dest[p * K + jj] = pos * K + rank[s][jj];
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
template <bool TOK, int K>
__device__ void small_body(const GroupJob& j, int32_t* s_mem) {
    constexpr int NW = kGroupThreads / 64;
    constexpr int IPT = kGroupSmallMax / kGroupThreads;  // items per lane
    const uint32_t* __restrict__ idx = j.idx;
    const int P = (int)j.items, E = j.E, nbins = j.nbins, ebits = j.ebits, BM = j.BM;
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
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wbase = wave * 64 * IPT;
    int bin[IPT], lrank[IPT];
    int rank[IPT][K];  // slot ranks of each token in its expert set (TOK)
    // the bins first: the loads of all IPT items are in flight together
#pragma unroll
    for (int s = 0; s < IPT; ++s) {
        const int p = wbase + s * 64 + lane;
        bin[s] = p < P ? item_bin<TOK, K>(idx, p, E, rank[s]) : -1;
    }
    for (int i = threadIdx.x; i < zero_n; i += kGroupThreads) zero_ptr[i] = 0;
    for (int i = threadIdx.x; i < NW * nbins; i += kGroupThreads) s_cnt[i] = 0;
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
    }
    __syncthreads();
    int32_t total, tiles, largest;
    block_exclusive_scan2(s_off, s_tb, nbins, s_part, total, tiles, largest);
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
        offsets[nbins + 1] = largest;
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
#pragma unroll
            for (int jj = 0; jj < K; ++jj) pair_dest[(long long)p * K + jj] = pos * K + rank[s][jj];
        }
    }
}

// One-launch multi-workgroup grouping: histogram of this block's chunk,
// stored device-coherently; the workgroup counts itself in at sync[0] and
// waits (at most `spin` polls) until every block of the job has; then the
// scatter as scatter_body, from the counts table. A workgroup whose wait runs
// out (its job's workgroups not all resident, which the host's grid cap makes
// the exception) recounts every item itself instead, so no wait is
// unbounded; spin < 0 makes every workgroup recount (tests). Each workgroup
// then counts itself out at sync[1]; the last one out resets both counters to
// zero for the next launch (every workgroup has counted itself in and
// finished waiting by then). sync must be zero before the first launch.
template <bool TOK, int K>
__device__ void one_launch_body(const GroupJob& j, int blk, int32_t* s_mem, int32_t* sync, int spin) {
    __shared__ int s_ok;
    hist_body<TOK, K, true>(j, blk, s_mem);
    // Publication: every thread's count stores precede the barrier, the
    // barrier precedes thread 0's release increment (agent scope). The poll
    // is relaxed; once it reads the job's total, one acquire fence makes the
    // workgroup synchronise with every increment before it (the increments
    // form one release sequence), so its reads of the count table after the
    // next barrier see every block's counts. (An acquire on every poll would
    // invalidate the XCD's L2 once per poll.)
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(sync, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 0;
        if (spin >= 0) {
            for (int it = 0;; ++it) {
                ok = __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= j.nb;
                if (ok || it >= spin) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
        if (ok) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        s_ok = ok;
    }
    __syncthreads();
    scatter_body<TOK, K>(j, blk, s_mem, s_ok ? kCountsCoherent : kCountsRecount);
    if (threadIdx.x == 0) {
        // (release, and an acquire fence in the last one out: it resets the
        // counters after every other workgroup's poll of sync[0])
        const int out = __hip_atomic_fetch_add(sync + 1, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        if (out == j.nb - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __hip_atomic_store(sync, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
template <int KB>
__global__ __launch_bounds__(kGroupThreads) void grouping_one_k(GroupJob A, GroupJob B, int32_t* sync, int spin) {
    extern __shared__ int32_t s_dyn[];
    const int a_n = A.small ? 1 : A.nb;
    if ((int)blockIdx.x < a_n) {
        if (A.small) small_body<false, 1>(A, s_dyn);
        else one_launch_body<false, 1>(A, blockIdx.x, s_dyn, sync, spin);
    } else if constexpr (KB > 0) {
        if (B.small) small_body<true, KB>(B, s_dyn);
        else one_launch_body<true, KB>(B, blockIdx.x - a_n, s_dyn, sync + 2, spin);
    }
}

// The launches serve the pair grouping (A) and, on the expert-set path, the
// token grouping (B, KB ids per token) together: in each, the first
// workgroups work on A and the rest on B. A job of at most kGroupSmallMax
// items is done whole by one workgroup of the final launch; a larger one
// takes a workgroup per kGroupChunk items in both launches.
template <int KB>
__global__ __launch_bounds__(kGroupThreads) void grouping_hist_k(GroupJob A, GroupJob B) {
    extern __shared__ int32_t s_dyn[];
    const int a_nb = A.small ? 0 : A.nb;
    if ((int)blockIdx.x < a_nb) hist_body<false, 1>(A, blockIdx.x, s_dyn);
    else if constexpr (KB > 0) hist_body<true, KB>(B, blockIdx.x - a_nb, s_dyn);
}
template <int KB>
__global__ __launch_bounds__(kGroupThreads) void grouping_final_k(GroupJob A, GroupJob B) {
    extern __shared__ int32_t s_dyn[];
    const int a_n = A.small ? 1 : A.nb;
    if ((int)blockIdx.x < a_n) {
        if (A.small) small_body<false, 1>(A, s_dyn);
        else scatter_body<false, 1>(A, blockIdx.x, s_dyn);
    } else if constexpr (KB > 0) {
        if (B.small) small_body<true, KB>(B, s_dyn);
        else scatter_body<true, KB>(B, blockIdx.x - a_n, s_dyn);
    }
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

template <int KB>
static hipError_t launch_groupings_k(const GroupJob& A, const GroupJob& B, bool has_b, hipStream_t stream,
                                     int32_t* sync, int max_one, int spin) {
    auto ints = [](long long n) { return (size_t)n * sizeof(int32_t); };
    const bool a_multi = !A.small, b_multi = has_b && !B.small;
    const int nb_multi = (a_multi ? A.nb : 0) + (b_multi ? B.nb : 0);
    if (sync && nb_multi > 0) {
        const int grid = (A.small ? 1 : A.nb) + (has_b ? (B.small ? 1 : B.nb) : 0);
        if (grid <= max_one) {
            auto lds1 = [&](const GroupJob& j) {
                return j.small ? 6LL * j.nbins + kGroupThreads : 7LL * j.nbins + kGroupThreads;
            };
            const long long lds = std::max(lds1(A), has_b ? lds1(B) : 0LL);
            hipLaunchKernelGGL(grouping_one_k<KB>, dim3(grid), dim3(kGroupThreads), ints(lds), stream, A, B, sync,
                               spin);
            return hipGetLastError();
        }
    }
    if (nb_multi > 0) {
        const int bins = std::max(a_multi ? A.nbins : 0, b_multi ? B.nbins : 0);
        hipLaunchKernelGGL(grouping_hist_k<KB>, dim3(nb_multi), dim3(kGroupThreads), ints(4LL * bins), stream, A, B);
    }
    auto final_lds = [&](const GroupJob& j) {
        return j.small ? 6LL * j.nbins + kGroupThreads : 7LL * j.nbins + kGroupThreads;
    };
    const long long lds = std::max(final_lds(A), has_b ? final_lds(B) : 0LL);
    const int grid = (A.small ? 1 : A.nb) + (has_b ? (B.small ? 1 : B.nb) : 0);
    hipLaunchKernelGGL(grouping_final_k<KB>, dim3(grid), dim3(kGroupThreads), ints(lds), stream, A, B);
    return hipGetLastError();
}

hipError_t launch_groupings(const GroupJob& A, const GroupJob* B, hipStream_t stream, int32_t* sync, int max_one,
                            int spin) {
    if (B && (B->k < 1 || B->k > kSetMaxK || B->nbins > kSetMaxKeys)) return hipErrorInvalidValue;
    // the scatter workgroups index the per-block count table with 32-bit ints
    if ((long long)A.nb * A.nbins + 16LL * kGroupThreads >= 0x7fffffffLL ||
        (B && (long long)B->nb * B->nbins + 16LL * kGroupThreads >= 0x7fffffffLL))
        return hipErrorInvalidValue;
    const GroupJob b = B ? *B : GroupJob{};
    switch (B ? B->k : 0) {
        case 0: return launch_groupings_k<0>(A, b, false, stream, sync, max_one, spin);
        case 1: return launch_groupings_k<1>(A, b, true, stream, sync, max_one, spin);
        case 2: return launch_groupings_k<2>(A, b, true, stream, sync, max_one, spin);
        case 3: return launch_groupings_k<3>(A, b, true, stream, sync, max_one, spin);
        case 4: return launch_groupings_k<4>(A, b, true, stream, sync, max_one, spin);
        case 5: return launch_groupings_k<5>(A, b, true, stream, sync, max_one, spin);
        case 6: return launch_groupings_k<6>(A, b, true, stream, sync, max_one, spin);
        case 7: return launch_groupings_k<7>(A, b, true, stream, sync, max_one, spin);
        case 8: return launch_groupings_k<8>(A, b, true, stream, sync, max_one, spin);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace cm
