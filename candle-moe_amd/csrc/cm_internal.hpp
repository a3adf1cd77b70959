// Internal launcher interface between the kernels and the C-ABI dispatcher.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cm {

// ---------------------------------------------------------------- router
// part / part_bytes: workspace of router_ws_bytes() for the K-split form of
// small batches (router_splits() > 1); without it one workgroup per tile.
hipError_t launch_router_topk(const void* x, const void* w, int dtype, float* wo, uint32_t* io, uint32_t* eo, int T,
                              int H, int E, int k, hipStream_t stream, float* part = nullptr,
                              size_t part_bytes = 0);
int router_splits(int T, int H, int E, int dtype);
size_t router_ws_bytes(int T, int H, int E, int dtype);
hipError_t launch_topk_softmax(const void* logits, int in_dtype, void* w, int w_dtype, uint32_t* idx,
                               uint32_t* ei, int T, int E, int k, hipStream_t stream);
// test support: the router's f32 exponential against its f64 one
hipError_t launch_router_exp_check(uint32_t first, uint32_t n, uint32_t* stats, hipStream_t stream);

// -------------------------------------------------------------- grouping
// Pairs p = t*k + j are grouped by expert idx[p] (stable: ascending p inside
// an expert). Pairs whose expert is >= E are dropped, as in
// /root/reference/kernels/preprocessing.cuh:49-52.
struct GroupingBufs {
    int32_t* offsets;       // [E+2]: exclusive scan, [E] = valid pairs, [E+1] = max count
    int32_t* block_counts;  // [nblocks * E]
    int32_t* sorted_pair;   // [P]
    int32_t* tile_row;      // [max_tiles]: first sorted row of the tile
    int32_t* tile_exp;      // [max_tiles]: expert of the tile
    int32_t* num_tiles;     // [1]
    int32_t* zero_ptr;      // ints cleared before the GEMMs run (may be null)
    int zero_n;
};
constexpr int kGroupChunk = 1024;      // items per workgroup of the multi-workgroup grouping
constexpr int kGroupSmallMax = 2048;   // up to this many items: one-workgroup grouping
inline int grouping_blocks(long long P) { return (int)((P + kGroupChunk - 1) / kGroupChunk); }
// Row tiles of a grouping: sum over non-empty groups of ceil(count / BM)
// <= ceil(P / BM) + (number of non-empty groups).
inline long long grouping_max_tiles(long long P, int E, int BM) { return (P + BM - 1) / BM + (P < E ? P : E); }
// Tokens grouped by their expert set: the key of token t is its k expert
// ids sorted ascending (ids >= E become E and sort last), read as base-(E+1)
// digits. b.sorted_pair receives the token of each sorted position,
// pair_dest[t*k + j] = pos(t)*k + rank of slot j in the token's sorted set.
// Polls (each s_sleep 2, ~128 clocks) a one-launch grouping workgroup makes
// for the rest of its job before it recounts on its own (~2 ms).
constexpr int kGroupSpin = 1 << 15;
constexpr int kSetMaxK = 8;
constexpr int kSetMaxKeys = 1024;

// A grouping job: pairs by expert (k = 1, nbins = E) or tokens by expert set
// (nbins = (E+1)^k keys, pair_dest set); small = one workgroup does it all,
// else nb workgroups of kGroupChunk items.
struct GroupJob {
    const uint32_t* idx;
    long long items;
    int k, E, nbins, ebits, BM, nb;
    int small;
    GroupingBufs b;
    int32_t* pair_dest;
};
GroupJob pair_grouping_job(const uint32_t* idx, long long P, int E, int BM, const GroupingBufs& b);
GroupJob set_grouping_job(const uint32_t* idx, int T, int k, int E, int nkeys, int BM, const GroupingBufs& b,
                          int32_t* pair_dest);
size_t a256_bytes(size_t x);  // x rounded up to 256 bytes
// The pair grouping and optionally the token grouping: one launch when both
// have at most kGroupSmallMax items, or when sync (4 ints, zero before the
// first launch, left zero) is given and the launch has at most max_one
// workgroups (one-launch grouping, spin: its wait bound); else two
// (histogram, scan + scatter).
hipError_t launch_groupings(const GroupJob& pairs, const GroupJob* tokens, hipStream_t stream,
                            int32_t* sync = nullptr, int max_one = 0, int spin = 0);

// ----------------------------------------------------------- grouped GEMM
enum GemmMode : int {
    kGateUp = 0,   // Qwen3: inter = act(x.G) * (x.U)      (A gathered from x, B [K,N] x2)
    kFc1 = 1,      // Nomic: inter = act(x.G)              (A gathered from x, B [K,N])
    kDown = 2,     // Qwen3: acc[t] += w * (inter.D)       (A = inter rows, B [K,N], f32 atomics)
    kFc2 = 3,      // Nomic: acc[t] += w * (inter.U^T)     (A = inter rows, B [N,K], f32 atomics)
    kDownSet = 4,  // Qwen3, tokens grouped by expert set: out[t] += [w*h_1 .. w*h_k] . [D_e1; ..; D_ek]
    kFc2Set = 5,   // Nomic, same with the U_e^T blocks
    kDownRows = 6, // Qwen3, pair path without atomics: rows[p] = dtype(w_p * (inter.D))  (rows [T*k, N])
    kFc2Rows = 7,  // Nomic, same with U^T
};

struct GemmArgs {
    const void* A;            // x [T,K] (kGateUp/kFc1) or inter [P,K] (kDown/kFc2)
    const void* B0;           // gate / down / up weights, expert-major
    const void* B1;           // up weights (kGateUp)
    void* C;                  // inter [P,N] (dtype) or f32 accumulator [T,N]
    const float* routing_w;   // [T*k]
    const int32_t* sorted_pair;
    int sorted_n;             // entries of sorted_pair (P)
    const int32_t* tile_row;
    const int32_t* tile_exp;
    const int32_t* num_tiles;
    const int32_t* offsets;
    long long strideB;        // elements between consecutive experts' B matrices
    int ldb;                  // row pitch of B in elements
    int K;                    // reduction length
    int N;                    // logical output columns
    int k_top;                // pair -> token divisor
    int act;                  // activation code
    int n_tiles;              // output column tiles
    int m_tiles_max;          // upper bound on row tiles (grid sizing)
    // expert-set path
    const int32_t* pair_dest; // GEMM1: output row of pair p (NULL: its sorted row)
    const int32_t* tok_sorted;// set GEMM2: token of each sorted row
    int fold_w;               // GEMM1: scale by the routing weight before rounding
    int n_experts;            // E (key digits are base E+1)
    int seg_len;              // set GEMM2: K length of one slot's segment (= I)
    long long a_bytes;        // size of A in bytes (LDS-DMA kernels: buffer range, < 2^31)
    // split-K and fused clears (moe_lds_gemm only)
    int ksplit;               // most workgroups per output tile along K (<= 1: one)
    int split_target;         // > 0: the kernel takes ~split_target / live tiles splits (at most
                              // ksplit; adaptive_split); 0: ksplit
    float* partial;           // ksplit > 1: [tile * splits + split][BM*BN] f32 slots
    int32_t* counters;        // [m_tiles_max*n_tiles] arrival counters: zero on entry, left zero
    float* zero_f32;          // f32 range cleared by this launch's workgroups (null: none)
    long long zero_n;
    int overwrite;            // expert-set down GEMM: out = acc instead of out + acc
    // Tail balance (8-wave 256x256 kernel): CUs per XCD, 0 = off. The tiles
    // of each XCD's last, partly filled round are split along K so that the
    // round's workgroups fill the XCD's CUs; the splits meet in the fixup
    // through partial [8*tail_cus][BM*BN] f32 and counters [8*tail_cus].
    int tail_cus;
    // fp8 weights (launch_moe_gemm_w8): per-output-column f32 scales, [E][N],
    // of B0 and (kGateUp) B1
    const float* scale0;
    const float* scale1;
    // 32-row kernel, kFc1 / kDown / kFc2 with 16-bit weights: 128-column
    // tiles instead of 256 (n_tiles counts those)
    int narrow;
    // 16-bit weights pre-packed K-contiguous ([N,K] per expert, ldb = K) for
    // every GEMM (candle_moe_fused_moe_packed); LDS-DMA kernels only
    int packed;
};
constexpr int kTailMaxSplit = 8;
constexpr int kTailMinKTiles = 8;  // K tiles per tail split at least (shorter splits lose to the fixup)

// Kernel shapes (the codes of candle_moe_set_tile_policy; the missing codes
// belonged to measured variants that are not shipped and are rejected).
// kTileSimt: 64x64 SIMT (f32 and shapes the MFMA kernels do not take).
// kTile128: register-staged MFMA kernel, 128x128 block tile (operands beyond
//   the 2 GiB range of the LDS-DMA kernels' buffer offsets).
// LDS-DMA MFMA kernels (moe_gemm_lds.hip):
//   kLds128: 128x128, 4 waves, BK 64, 4 stages;
//   kLds256w8: 256x256, 8 waves (2 per SIMD), BK 64, 2 stages (prefill);
//   kLdsRows32: 32x256, 4 waves side by side along N, BK 64, 4 stages: few
//     rows per expert (decode), bound by streaming the weights;
//   kLds128x256o2: 128x256, 4 waves, BK 32, 3 stages, two workgroups per CU.
// kW8Gemv (fp8 weights only, moe_gemv_w8.hip): the 32-row tile table, 16
//   output columns (gate/up) or 32 per workgroup over the whole of K, split
//   over its 4 waves; operands loaded straight into registers (decode).
// f32 vector-FMA kernels (moe_gemm_f32.hip): kF32Rows32 (32x128 block tile),
//   kF32Tile128 (128x128).
// The grouping's tile table must be built with the kernel's row tile,
// tile_rows().
// kDecGemv (16-bit weights, moe_gemv_dec.hip): decode GEMMs that group the
//   pairs themselves (no grouping launch), load weights straight into
//   registers and split K only across the waves of a workgroup; the down /
//   fc2 GEMM stores pair rows that the k-row sum adds up.
enum TileCfg : int {
    kTileSimt = 0, kTile128 = 1, kLds128 = 5, kLds256w8 = 7, kLdsRows32 = 12, kLds128x256o2 = 14,
    kF32Rows32 = 15, kF32Tile128 = 16, kW8Gemv = 17, kDecGemv = 18
};
constexpr int kNumTileCfgs = 19;  // codes are < kNumTileCfgs
inline bool is_shipped_cfg(int cfg) {
    return cfg == kTileSimt || cfg == kTile128 || cfg == kLds128 || cfg == kLds256w8 || cfg == kLdsRows32 ||
           cfg == kLds128x256o2 || cfg == kF32Rows32 || cfg == kF32Tile128 || cfg == kW8Gemv || cfg == kDecGemv;
}
inline bool is_f32_cfg(int cfg) { return cfg == kF32Rows32 || cfg == kF32Tile128; }
inline int tile_rows(int cfg) {
    if (cfg == kDecGemv) return 16;
    if (cfg == kLdsRows32 || cfg == kF32Rows32 || cfg == kW8Gemv) return 32;
    if (cfg == kTileSimt) return 64;
    if (cfg == kLds256w8) return 256;
    return 128;  // kTile128, kLds128, kLds128x256o2, kF32Tile128
}
// kW8Gemv: 16-column blocks per wave; output columns of a workgroup whose 4
// waves split K in kw parts; kw for a GEMM of K, N over `tiles` row tiles:
// the fewest K parts (1, 2, 4) that still give 512 workgroups (two per CU),
// else 4.
constexpr int kGvCB = 2;
__host__ __device__ inline int gv_wg_cols(int mode, int kw) {
    return (mode == kGateUp ? 8 * kGvCB : 16 * kGvCB) * (4 / kw);
}
__host__ __device__ inline int gv_pick_kw(int mode, int N, long long tiles) {
    for (int kw = 1; kw < 4; kw *= 2)
        if (tiles * ((N + gv_wg_cols(mode, kw) - 1) / gv_wg_cols(mode, kw)) >= 512) return kw;
    return 4;
}
inline int tile_cols(int cfg) {
    if (cfg == kTileSimt) return 64;
    if (cfg == kW8Gemv) return 16 * kGvCB;
    if (cfg == kLds256w8 || cfg == kLdsRows32 || cfg == kLds128x256o2) return 256;
    return 128;  // kTile128, kLds128, f32 kernels
}
// (kW8Gemv shares the LDS-DMA kernels' 32-bit buffer offsets and fused
// accumulator clear)
inline bool is_lds_cfg(int cfg) {
    return cfg == kLds128 || cfg == kLds256w8 || cfg == kLdsRows32 || cfg == kLds128x256o2 || cfg == kW8Gemv;
}
// Workgroups of a launch over at most `tiles` output tiles: with adaptive K
// splits live tiles * splits stays within split_target when it splits.
inline long long split_grid(long long tiles, const GemmArgs& a) {
    if (a.ksplit <= 1) return tiles;
    if (a.split_target <= 0) return tiles * a.ksplit;
    return tiles > a.split_target ? tiles : a.split_target;
}
// K tile of the LDS-DMA kernels
inline int tile_bk(int cfg) {
    if (is_f32_cfg(cfg)) return 16;
    return cfg == kLds128x256o2 ? 32 : 64;
}

bool mfma_supported(int dtype, int K, int N);
// Logical output columns covered by one workgroup of the chosen kernel.
int gemm_tile_cols(int mode, int cfg);
hipError_t launch_moe_gemm(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream);
hipError_t launch_moe_gemm_lds(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream);
// GEMMs over OCP fp8 e4m3 weights stored K-contiguous ([E][N][K] bytes, ldb
// = K, strideB = N*K) with per-output-column scales (scale0 / scale1), on the
// 32-row kernel (tile_rows(kLdsRows32)); 16-bit activations; modes kGateUp,
// kFc1, kDown, kFc2.
// cfg: kW8Gemv or kLdsRows32 (decode), or kLds256w8
hipError_t launch_moe_gemm_w8(int mode, int dtype, int cfg, const GemmArgs& a, hipStream_t stream);
// kW8Gemv (moe_gemv_w8.hip): modes kGateUp, kFc1, kDown, kFc2 (pair path,
// f32 atomics for kDown / kFc2)
hipError_t launch_w8_gemv(int mode, int dtype, const GemmArgs& a, hipStream_t stream);
hipError_t launch_moe_gemm_f32(int mode, int cfg, const GemmArgs& a, hipStream_t stream);

// Decode GEMMs (moe_gemv_dec.hip) over 16-bit weights (API layout or
// pre-packed) or fp8 codes. Every workgroup groups the P pairs itself (P <=
// kDecMaxPairs, E <= kDecMaxE), counts the touched experts U and splits K
// into ks = min(cap / (U * nblk), ks_lim) slices (at least 1), so that the U
// * nblk * ks items (expert, column block of 16 * cpl columns, slice) fill
// one round of cap workgroups; the grid is max(cap, max_groups * nblk) and
// workgroup w takes item w. ks goes to meta[0] (gate/up, fc1) or meta[1]
// (down, fc2) for the finishing launch. Modes: kGateUp, kFc1 (ks == 1: inter
// [P, N] by pair in the dtype; ks > 1: f32 partials), kDownRows, kFc2Rows
// (always f32 partials of the unweighted sums). Partials: part[(s * P + p) *
// NC + c], NC = 2N for kGateUp (gate at c, up at N + c), else N.
constexpr int kDecMaxPairs = 1024;
constexpr int kDecMaxE = 4096;
constexpr int kDecMaxSlices = 16;
struct DecArgs {
    const void* A;            // x [T, K] (kGateUp / kFc1) or inter [P, K] (kDownRows / kFc2Rows)
    const void* B0;           // gate / fc1 / down / fc2 weights, expert-major
    const void* B1;           // up weights (kGateUp)
    void* C;                  // inter [P, N] (dtype; kGateUp / kFc1 when ks == 1)
    float* part;              // f32 partials, ks_lim * P * NC floats
    int* meta;                // [2] slices of the last gate/up and down launches
    const uint32_t* idx;      // [P] expert of pair p (>= E: dropped)
    int P, E, K, N, k_top, act;
    long long strideB;        // elements per expert matrix
    int ldb;                  // row pitch of B: N for [K,N] weights, K for [N,K] (kFc2Rows)
    long long a_bytes;        // bytes of A (< 2^31)
    int nblk;                 // column blocks of 16 * cpl columns
    int cap;                  // workgroups of one round (the items' target)
    int ks_lim;               // most K slices (1 .. kDecMaxSlices)
    int max_groups;           // touched experts at most
    int rows_max;             // > 16: row chunks of 32 (two MFMA row blocks), else 16
    int cpl;                  // columns per lane: 2, 4 or 8
    int packed;               // every B [N,K] (pre-packed weights, ldb = K)
    int w8;                   // fp8 e4m3 codes [E][N][K] (ldb = K) with f32 scales [E][N]
    const float* scale0;      // (w8) gate / fc1 column scales (kGateUp / kFc1 with ks == 1)
    const float* scale1;      // (w8) up column scales
};
hipError_t launch_dec_gemv(int mode, int dtype, const DecArgs& a, hipStream_t stream);
// Finishing the K slices of a decode GEMM (fixed slice order: deterministic),
// ks = meta[0] (gate/up, fc1) or meta[1] (down, fc2), as the GEMM stored it.
// kGateUp / kFc1 (nothing to do when ks == 1): inter[p] = dtype(act(s0 *
// sum_s gate) (* s1 * sum_s up)) for the valid pairs. kDownRows / kFc2Rows:
// out[t] = dtype(out[t] (accumulate) + sum_j w_{t,j} * s0 * sum_s
// part[s][t*k + j]) over the valid pairs of token t in slot order. s0 / s1:
// fp8 column scales of the pair's expert, or 1.
struct DecFinish {
    const float* part;
    const int* meta;
    int ks_lim, P, N, E, T, k_top, act;
    const uint32_t* idx;
    const float* routing_w;   // (down / fc2)
    const float* scale0;      // (fp8) gate / fc1 / down / fc2 column scales, else null
    const float* scale1;      // (fp8) up column scales, else null
    void* out;                // inter [P, N] or out [T, N] (dtype)
    int overwrite;            // (down / fc2) write out instead of adding to it
};
hipError_t launch_dec_finish(int mode, int dtype, const DecFinish& f, hipStream_t stream);


// fp8 weight preparation (fp8.hip): quantize [E][K][N] (kn) or [E][N][K]
// weights of dtype to e4m3 codes [E][N][K] and scales [E][N]; dequantize
// codes and scales to [E][N][K] of dtype.
hipError_t launch_quantize_fp8(const void* w, int dtype, int E, int K, int N, int kn, uint8_t* q, float* scales,
                               hipStream_t stream);
hipError_t launch_dequantize_fp8(const uint8_t* q, const float* scales, int E, int N, int K, void* out, int dtype,
                                 hipStream_t stream);
// 16-bit weights [E][K][N] -> K-contiguous [E][N][K] (the pre-packed format)
hipError_t launch_pack_kn(const void* w, int E, int K, int N, void* out, hipStream_t stream);

// f32 accumulator helpers
hipError_t launch_fill_zero_f32(float* p, long long n, hipStream_t stream);
hipError_t launch_fill_zero_bytes(void* p, long long nbytes, hipStream_t stream);
// out[t] = dtype(out[t] + sum_j rows[t*k + j]), or without out[t] with
// overwrite (rows: [T*k, H] of the output dtype, f32 sums in slot order;
// slots whose expert idx[t*k + j] >= E were dropped and have no row)
hipError_t launch_pair_rows_sum(void* out, int dtype, const void* rows, const uint32_t* idx, int E, int T, int k,
                                int H, bool overwrite, hipStream_t stream);
// out[i] = dtype(out[i] + acc[i]), or dtype(acc[i]) with overwrite
hipError_t launch_finalize(void* out, int dtype, const float* acc, long long n, bool overwrite, hipStream_t stream);

// ------------------------------------------------------------ C-ABI core
// Record the message of a failing call (thread-local) and return `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();
int topk_softmax_impl(const void* g, int gdt, void* w, int wdt, void* idx, void* ei, int E, int T, int k,
                      void* stream);
struct Fp8Weights;
int fused_moe_impl(const void* x, const void* gate, const void* up, const void* down, const void* rw,
                   const void* idx, void* out, int T, int H, int I, int E, int k, int act, uint32_t moe_type,
                   uint32_t dtype, void* ws, size_t ws_bytes, bool own_ws, bool overwrite, void* stream,
                   const Fp8Weights* f8 = nullptr, bool packed = false);

}  // namespace cm
