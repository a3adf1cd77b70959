// C ABI of libcandle_moe_hip.so: the reference's two FFI symbols
// (/root/reference/src/ffi.rs:15-62), their status-returning variants and
// the fused-MoE dispatcher (/root/reference/kernels/moe.cu:453-771).
//
// Dispatcher, per call, all on the caller's stream, no host sync. Two paths:
//  expert-set path (few distinct expert sets next to the token count):
//   pair grouping + token grouping by expert set -> GEMM1 (gate+up or fc1,
//   activation and routing weight fused, rows written in token-set order)
//   -> GEMM2 over K = k*I per expert set, added once into the output.
//  pair path (everything else):
//   pair grouping -> GEMM1 (activation fused) -> GEMM2 with the routing
//   weight fused, then either
//    * pair rows (16-bit prefill kernels): each pair's weighted row stored
//      in the dtype, then a pass that sums a token's k rows in f32 in slot
//      order and adds them to the output (rounded once), or
//    * f32 atomics (32-row decode kernels, f32 kernels, and pair rows that
//      would exceed kRowsMaxBytes): coalesced atomic adds into an f32
//      [T, H] accumulator that the gate/up launch clears, then finalize
//      (output += accumulator, rounded once).
// Workspace (256-byte aligned pieces): offsets[E+2], per-block counts,
// sorted pair ids, row-tile table, intermediate [T*k, I] in the input dtype
// and the pair rows [T*k, H] (dtype) or the f32 accumulator [T, H].
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/candle_moe.h"
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

static int hip_fail(hipError_t e, const char* what) {
    return set_error(CANDLE_MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------- profiling
// Optional per-kernel timing: while enabled, every internal launch is
// bracketed by a pair of HIP events on the caller's stream.
enum ProfSlot { kSlotTopk = 0, kSlotGroup, kSlotGemm1, kSlotZero, kSlotGemm2, kSlotFinal, kNumSlots };
static const char* kSlotNames[kNumSlots] = {"topk_softmax", "grouping", "gemm_gate_up", "acc_clear",
                                            "gemm_down", "finalize"};
struct ProfRec {
    int slot;
    hipEvent_t a, b;
};
static std::mutex g_prof_mu;
static bool g_prof_on = false;
static uint32_t g_prof_mask = ~0u;  // slots bracketed while profiling is on
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_event_pool;  // events of finished sessions, reused (creation costs host time)

static bool pooled_event_locked(hipEvent_t& ev) {
    if (!g_event_pool.empty()) {
        ev = g_event_pool.back();
        g_event_pool.pop_back();
        return true;
    }
    return hipEventCreate(&ev) == hipSuccess;
}

struct ProfScope {
    ProfRec rec;
    hipStream_t s;
    bool on;
    ProfScope(int slot, hipStream_t stream) : s(stream), on(false) {
        std::lock_guard<std::mutex> lk(g_prof_mu);
        if (!g_prof_on || !((g_prof_mask >> slot) & 1u)) return;
        rec.slot = slot;
        if (!pooled_event_locked(rec.a)) return;
        if (!pooled_event_locked(rec.b)) {
            g_event_pool.push_back(rec.a);
            return;
        }
        on = hipEventRecord(rec.a, s) == hipSuccess;
        if (!on) {
            g_event_pool.push_back(rec.a);
            g_event_pool.push_back(rec.b);
        }
    }
    ~ProfScope() {
        if (!on) return;
        (void)hipEventRecord(rec.b, s);
        std::lock_guard<std::mutex> lk(g_prof_mu);
        g_prof.push_back(rec);
    }
};

// ------------------------------------------------------------------ router
int topk_softmax_impl(const void* g, int gdt, void* w, int wdt, void* idx, void* ei, int E, int T, int k,
                      void* stream) {
    clear_error();
    if (T < 0) return set_error(CANDLE_MOE_ERR_INVALID, "topk_softmax: num_tokens must be >= 0 (got %d)", T);
    if (E < 1 || E > 1024)
        return set_error(CANDLE_MOE_ERR_INVALID, "topk_softmax: num_experts must be in [1, 1024] (got %d)", E);
    if (k < 1 || k > E)
        return set_error(CANDLE_MOE_ERR_INVALID, "topk_softmax: topk must be in [1, num_experts=%d] (got %d)", E, k);
    if (T == 0) return CANDLE_MOE_OK;
    if (!g || !w || !idx || !ei) return set_error(CANDLE_MOE_ERR_INVALID, "topk_softmax: null tensor pointer");
    hipError_t e;
    {
        ProfScope ps(kSlotTopk, reinterpret_cast<hipStream_t>(stream));
        e = launch_topk_softmax(g, gdt, w, wdt, reinterpret_cast<uint32_t*>(idx), reinterpret_cast<uint32_t*>(ei), T,
                                E, k, reinterpret_cast<hipStream_t>(stream));
    }
    if (e == hipErrorInvalidValue && !((gdt == wdt) || wdt == kF32))
        return set_error(CANDLE_MOE_ERR_UNSUPPORTED, "topk_softmax: unsupported dtype pair (%d, %d)", gdt, wdt);
    if (e != hipSuccess) return hip_fail(e, "topk_softmax launch");
    return CANDLE_MOE_OK;
}

// ------------------------------------------------------------- fused MoE
struct Problem {
    int T, H, I, E, k, act, moe_type, dtype;
    bool mfma;
    bool packed;  // pre-packed K-contiguous 16-bit weights (candle_moe_fused_moe_packed)
    int cfg;  // TileCfg of both GEMMs
    int BM;
    long long P;
    bool set_path;  // expert-set down projection (no atomics, no f32 accumulator)
    int nkeys;      // (E+1)^k expert-set keys
    int split1;     // K splits of the gate/up GEMM (moe_lds_gemm only; > 1 needs partial + counters)
    int split2;     // K splits of the pair-path down GEMM (atomic combine)
    int n_tiles1, n_tiles2;
    bool lds_family;  // both GEMMs run moe_lds_gemm (fused clears and K splits available)
    bool fused_clear_ok;  // the gate/up kernel can clear the pair path's accumulator
    bool rows_path;   // pair path: each pair's weighted down row stored, then summed per token (no atomics)
    int tail_cus;     // tail balance of the 8-wave 256x256 kernel: CUs per XCD (0 = off)
    int split_target; // K splits: the kernels aim at this many workgroups (live tiles * splits)
    bool narrow1;     // fc1 GEMM on 128-column tiles of the 32-row kernel
    bool narrow2;     // pair-path down / fc2 GEMM on 128-column tiles of the 32-row kernel
    int dec_ks1, dec_ks2;  // decode kernels: most K slices of the gate/up (fc1) and down (fc2) GEMMs
};

// CUs per XCD of the current device (its CUs over the 8 XCDs of MI355X), 0
// when unknown; read once per device.
static int cus_per_xcd() {
    static std::mutex mu;
    static int cached[64];
    static bool known[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    std::lock_guard<std::mutex> lk(mu);
    if (!known[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
        cached[dev] = (n > 0 && n % 8 == 0) ? n / 8 : 0;
        known[dev] = true;
    }
    return cached[dev];
}

// Every workspace starts with a fixed header, the same for every shape, whose
// counters the library-owned workspaces hold at zero between calls: the
// one-launch grouping's (offset 0, 256 bytes). The router's split partials
// go after it.
constexpr size_t kWsHeaderBytes = 256;
struct Layout {
    size_t sync;  // 4 ints of the one-launch grouping (offset 0, 256 bytes)
    size_t offsets, block_counts, sorted_pair, tile_row, tile_exp, num_tiles;
    size_t k_offsets, k_block_counts, tok_sorted, tile_row2, tile_key2, num_tiles2, pair_dest;
    size_t inter, acc, partial, counters, dec_meta, total;
};

// 0: choose per call; 1: always the pair path (pair rows or f32 atomics,
// by kernel); 2: the expert-set path whenever the shape allows it.
// Pair-row bytes (T*k*H 16-bit values) from which the expert-set path is
// preferred over the pair path's row stores and k-row sums.
constexpr double kSetMinRowBytes = 256.0 * 1024 * 1024;
// Largest pair-row buffer (T*k*H 16-bit values) the pair path stores; beyond
// it the down GEMM adds into the f32 [T, H] accumulator with atomics instead
// (k*H*2 bytes per token against H*4), which bounds the workspace of shapes
// whose expert sets are too many for the expert-set path (large k and E).
constexpr double kRowsMaxBytes = 2.0 * 1024 * 1024 * 1024;
// fp8 weights: most pairs for the register-operand decode kernel (kW8Gemv;
// its workgroups re-stream an expert's weights per 32-row tile like the
// 32-row kernel's, without that kernel's LDS stages and split-K fixup).
// Measured against the 32-row kernel (fp8 GEMM µs, gate/up + down):
// Qwen3-30B-A3B T=1 (8 pairs) 29.1 -> 21.4, Qwen3 T=16 (32 pairs) 51.2
// against 50.5, Qwen3 T=64 65.2 against 51.3, Qwen3-30B-A3B T=16 (128 pairs
// over ~30 experts) 51.6 against 40.2. (The host cannot tell how many
// experts a batch touches, so the bound is on the pairs.)
constexpr long long kW8GemvPairs = 16;
constexpr long long kW8DecPairs = 128;
// fp8 weights beyond 32 rows per touched expert: the 32-row kernel streams
// each touched expert's weights once per 32-row chunk, the 8-wave 256x256
// kernel once per 256 rows but with mostly empty tiles and few workgroups
// until the experts hold a few hundred rows each. The 32-row kernel wins
// while that stream stays within this many bytes (fp8 step us, 32-row
// against 256x256): 302 MB: Qwen3 T=256 75.8 / 103.0, Nomic T=1024 65.7 /
// 87.9; 151 MB and less: Nomic T=192 / 256 / 512 37.2 / 44.5 / 50.3 against
// 64.1 / 65.3 / 75.8; 604 MB: Qwen3 T=512 125.6 / 128.1, Nomic T=2048 107.9
// / 97.4; 1.2 GB: Qwen3 T=1024 212.9 / 146.3, Qwen3-30B-A3B T=1024 297.1 /
// 250.8. (Measured up to 256 rows per touched expert; the rule stops there.)
constexpr long long kW8Rows32StreamBytes = 384LL << 20;
static int g_combine_policy = 0;
// 0: choose the GEMM kernel per call; a shipped TileCfg code: force it.
static int g_tile_policy = 0;
// Grouping launches above kGroupSmallMax items: 0 one launch where the
// workspace's counters are known to start at zero (library-owned
// workspaces, each used by one stream), the launch fits the device and the
// pair job has at most kGroupOneMaxBlocks blocks, else two; 1 always two; 2
// one launch whose workgroups all take the recount fallback (tests).
// Beyond that many blocks the one launch's agent-scope fences (a release per
// workgroup, an acquire in each waiter) cost more than the second launch:
// Qwen3 T=32768 (64 blocks per job) 18.6-20.0 us in one launch against 14.1
// us in two, and the gate/up GEMM after it 1370 against 1383 us;
// Qwen3-30B-A3B T=4096 (32 blocks) 13.8 against 13.7 us; Nomic T=4096 (8
// blocks) 11.6 against 12.5 us.
static int g_grouping_mode = 0;
constexpr int kGroupOneMaxBlocks = 32;

static long long set_tiles_max(const Problem& p) {
    return (p.T + p.BM - 1) / p.BM + (p.nkeys < p.T ? p.nkeys : p.T);
}

static size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }
size_t a256_bytes(size_t x) { return a256(x); }

static Layout make_layout(const Problem& p) {
    Layout L;
    const size_t es = p.dtype == kF32 ? 4 : 2;
    const long long nb = grouping_blocks(p.P);
    const long long mt = grouping_max_tiles(p.P, p.E, p.BM);
    size_t o = 0;
    L.sync = o; o += kWsHeaderBytes;
    L.offsets = o; o += a256((size_t)(p.E + 2) * 4);
    L.block_counts = o; o += a256((size_t)(nb > 0 ? nb : 1) * p.E * 4);
    L.sorted_pair = o; o += a256((size_t)(p.P > 0 ? p.P : 1) * 4);
    L.tile_row = o; o += a256((size_t)mt * 4);
    L.tile_exp = o; o += a256((size_t)mt * 4);
    L.num_tiles = o; o += 256;
    if (p.set_path) {
        const long long nbt = grouping_blocks(p.T);
        const long long mt2 = set_tiles_max(p);
        L.k_offsets = o; o += a256((size_t)(p.nkeys + 2) * 4);
        L.k_block_counts = o; o += a256((size_t)(nbt > 0 ? nbt : 1) * p.nkeys * 4);
        L.tok_sorted = o; o += a256((size_t)(p.T > 0 ? p.T : 1) * 4);
        L.tile_row2 = o; o += a256((size_t)mt2 * 4);
        L.tile_key2 = o; o += a256((size_t)mt2 * 4);
        L.num_tiles2 = o; o += 256;
        L.pair_dest = o; o += a256((size_t)(p.P > 0 ? p.P : 1) * 4);
    } else {
        L.k_offsets = L.k_block_counts = L.tok_sorted = L.tile_row2 = L.tile_key2 = L.num_tiles2 = L.pair_dest = 0;
    }
    L.inter = o; o += a256((size_t)p.P * p.I * es);
    L.acc = o;  // pair path: f32 accumulator [T, H], or the pair rows [T*k, H] (dtype)
    if (p.cfg == kDecGemv) {
        // decode kernels: the f32 partials of both GEMMs (one after the other)
        const size_t nc1 = (size_t)(p.moe_type == kQwen3 ? 2 : 1) * p.I;
        const size_t n1 = p.dec_ks1 > 1 ? (size_t)p.dec_ks1 * p.P * nc1 : 0;  // (ks == 1: rows in the dtype)
        const size_t n2 = (size_t)p.dec_ks2 * p.P * p.H;
        o += a256(std::max(n1, n2) * 4);
    } else if (!p.set_path) {
        o += p.rows_path ? a256((size_t)p.P * p.H * es) : a256((size_t)p.T * p.H * 4);
    }
    // split-K partials and arrival counters, shared by the two GEMMs (they run
    // one after the other; the counters are left zero)
    L.dec_meta = o;
    if (p.cfg == kDecGemv) o += 256;  // decode kernels: the slices each GEMM chose
    L.partial = L.counters = o;
    if (p.split1 > 1 || p.split2 > 1) {
        // partial slots: live tiles * splits, at most split_target with the
        // device's choice, else the host's fixed split over the most tiles
        const size_t c1 = p.split1 > 1 ? (size_t)mt * p.n_tiles1 : 0;
        const size_t c2 = p.split2 > 1 ? (size_t)mt * p.n_tiles2 : 0;
        const size_t slots = p.split_target > 0 ? (size_t)p.split_target
                                                : std::max(c1 * p.split1, c2 * p.split2);
        L.partial = o; o += a256(slots * p.BM * tile_cols(p.cfg) * 4);
        L.counters = o; o += a256((c1 > c2 ? c1 : c2) * 4);
    } else if (p.tail_cus > 0) {
        const size_t slots = 8 * (size_t)p.tail_cus;
        L.partial = o; o += a256(slots * p.BM * tile_cols(p.cfg) * 4);
        L.counters = o; o += a256(slots * 4);
    }
    L.total = o;
    return L;
}

// The decode kernels (kDecGemv) group the pairs in LDS (at most
// kDecMaxPairs of them, experts below kDecMaxE), address operands with 32-bit
// buffer offsets and load 16-byte chunks (hidden and intermediate sizes
// multiples of 8, 16-byte aligned operands: p.mfma).
// (Their waves' K ranges are whole rounds of 4 steps of 32, which may run
// up to 512 past K: the weight offsets stay below 2^31 with that margin.)
static bool dec_gemv_fits(const Problem& p) {
    const long long lim = 0x7fffff00LL;
    return p.mfma && p.P <= kDecMaxPairs && p.E <= kDecMaxE && (long long)p.T * p.H * 2 < lim &&
           p.P * p.I * 2 < lim && p.P * p.H * 2 < lim && (long long)(p.H + 1024) * p.I * 2 < lim &&
           (long long)(p.I + 1024) * p.H * 2 < lim;
}

// Most K slices of a decode GEMM over N columns and K (the kernels choose
// the slices from the experts a batch touches, up to this): cold weights
// stream at the rate of the access pattern and of the workgroups reading
// them (a probe over the Qwen3 T=8 gate/up weights, 176 MB: 128-byte runs of
// k-rows on 168 workgroups 4.0 TB/s, 256-byte runs on 500-1000 workgroups
// 5.9 TB/s), so slices let 128-column blocks (256-byte runs) fill the
// device. Bounds: at least kDecMinSteps steps of 32 k per wave (kp waves
// share a slice of one tensor) and f32 partials of at most kDecPartBytes.
// Used where the weight stream is at least kDecSliceBytes (check_problem).
constexpr int kDecMinSteps = 1;
constexpr double kDecPartBytes = 16.0 * 1024 * 1024;
constexpr double kDecSliceBytes = 128.0 * 1024 * 1024;
static int dec_slices(long long P, int N, int K, int kp, int nc_mult) {
    long long ks = cdiv(K, 32) / (kp * kDecMinSteps);
    ks = std::min<long long>(ks, kDecMaxSlices);
    ks = std::min<long long>(ks, (long long)(kDecPartBytes / ((double)std::max<long long>(P, 1) * N * nc_mult * 4)));
    return (int)std::max<long long>(ks, 1);
}
// Workgroups of one round of the decode kernels: two per CU.
static int dec_cap() { return 2 * 8 * std::max(cus_per_xcd(), 32); }
// Most pairs the decode kernels take by default (16-bit weights; up to 32
// per touched expert). Beyond, their items outnumber one round of
// workgroups and the 32-row kernel is faster: Qwen3-30B-A3B steps at T=32 /
// 48 / 64 / 128 (256 / 384 / 512 / 1024 pairs) 108 / 140 / 156 / 213 us on
// the decode kernels against 115 / 126 / 134 / 149 us; Qwen3 T=128 (256
// pairs) 102 against 115 us.
constexpr long long kDecDefaultPairs = 256;

// aligned16: input and weights start on 16-byte boundaries (the MFMA and f32
// tiled kernels read them with 16-byte loads; otherwise the scalar kernel
// runs). out16: so does the output (the expert-set down GEMM stores straight
// into it, 8 bytes at a time; otherwise the pair path, whose last pass
// handles any alignment).
// fp8: fp8 weights (candle_moe_fused_moe_fp8): the 32-row kernel for decode
// batches, the 8-wave 256x256 kernel beyond, on the pair path.
static int check_problem(int T, int H, int I, int E, int k, int act, uint32_t moe_type, uint32_t dtype,
                         Problem& p, bool aligned16 = true, bool out16 = true, bool fp8 = false,
                         bool packed = false) {
    if (T < 0) return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: num_tokens must be >= 0 (got %d)", T);
    if (H < 1 || I < 1)
        return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: hidden_dim and intermediate_dim must be >= 1 (got %d, %d)", H, I);
    if (E < 1 || E > 4096)
        return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: num_experts must be in [1, 4096] (got %d)", E);
    if (k < 1) return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: num_selected_experts must be >= 1 (got %d)", k);
    if (act < 0 || act > 2) return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: activation_type must be 0, 1 or 2 (got %d)", act);
    if (moe_type > 1) return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: moe_type must be one of 0 or 1 (got %u)", moe_type);
    if (dtype > 2) return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: dtype must be 0 (f16), 1 (bf16) or 2 (f32) (got %u)", dtype);
    const long long P = (long long)T * k;
    if (P > 0x7fffffffLL)
        return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: num_tokens * num_selected_experts exceeds 2^31-1");
    p.T = T; p.H = H; p.I = I; p.E = E; p.k = k; p.act = act; p.moe_type = (int)moe_type; p.dtype = (int)dtype;
    p.P = P;
    p.mfma = mfma_supported(p.dtype, H, I) && mfma_supported(p.dtype, I, H) && aligned16;
    p.packed = packed;
    if (packed && !p.mfma)
        return set_error(CANDLE_MOE_ERR_UNSUPPORTED,
                         "fused_moe_packed: needs f16 or bf16, hidden_dim and intermediate_dim multiples of 8 and "
                         "16-byte aligned tensors (got dtype %u, %d, %d)", dtype, H, I);
    // Default MFMA kernel, by rows per touched expert (measured on MI355X
    // over T = 1 .. 32768 of the Qwen3, Qwen3-30B and Nomic shapes):
    //  * at most 32 (decode): the GEMMs stream each touched expert's weights
    //    once; the 32-row tile keeps the padding and the MFMA work small;
    //  * at most 128, where the 256x256 tile would leave fewer than 256
    //    workgroups (few experts): the 128x128 tile, which doubles to
    //    quadruples the workgroups;
    //  * fewer than 1024 with a hidden size of at most 2048 (short K loops of
    //    the gate/up GEMM): the 128x256 tile, two workgroups per CU, so that
    //    one's prologue, barriers and epilogue overlap the other's MFMAs --
    //    if the down GEMM's 128x256 tiles fill both slots of every CU; with
    //    a small hidden size (Nomic, H = 768: 3 column tiles) they do not,
    //    and the 256x256 tile, whose partly filled last round is split along
    //    K, is faster (Nomic T=2048 / 4096 steps 192 / 219 -> 119 / 198 us);
    //  * otherwise the 256x256 tile with 8 waves.
    // Expected live row tiles of a tile height: one per touched expert at
    // least, the rows over the tile height at least.
    const long long touched = P < E ? P : E;
    auto est_tiles = [&](int bm) { return std::max<long long>((P + bm - 1) / bm, touched); };
    // (policy kW8Gemv concerns fp8 weights only: automatic here; pre-packed
    // weights run the LDS-DMA and decode kernels only)
    int policy = g_tile_policy == kW8Gemv ? 0 : g_tile_policy;
    if (packed && policy && !is_lds_cfg(policy) && policy != kDecGemv) policy = 0;
    p.cfg = !p.mfma ? kTileSimt : (policy ? policy : kLds256w8);
    // f32: the tiled vector-FMA kernel (32-row tile with K splits for decode,
    // 128-row tile otherwise) wherever 16-byte loads are possible
    const bool f32_tiled = p.dtype == kF32 && H % 4 == 0 && I % 4 == 0 && aligned16;
    if (f32_tiled) {
        p.cfg = (P <= 32 * touched) ? kF32Rows32 : kF32Tile128;
        if (policy == kF32Rows32 || policy == kF32Tile128) p.cfg = policy;
    } else if (!p.mfma || is_f32_cfg(p.cfg)) {
        p.cfg = kTileSimt;
    }
    if (fp8) {
        if (p.dtype == kF32 || H % 16 || I % 16 || !p.mfma)
            return set_error(CANDLE_MOE_ERR_UNSUPPORTED,
                             "fused_moe_fp8: needs f16 or bf16 activations, hidden_dim and intermediate_dim multiples "
                             "of 16 and 16-byte aligned tensors (got dtype %u, %d, %d)", dtype, H, I);
        // decode batches stream each touched expert's weights once per row
        // tile: up to kW8GemvPairs pairs the register-operand kernel (no LDS
        // staging, no K splits across workgroups), up to 32 rows per touched
        // expert, or up to 256 while its weight stream stays within
        // kW8Rows32StreamBytes, the 32-row tile kernel; beyond, the 8-wave
        // 256x256 kernel.
        // Tile policies 17, 12 and 7 force one of them.
        // Up to kW8DecPairs pairs the decode kernels instead (the pairs
        // grouped inside the GEMM kernels, no grouping launch; GEMM time at
        // Qwen3 T=16 / Qwen3-30B-A3B T=1 / Nomic T=16 48.7 / 19.3 / 22.6
        // against 53.3 / 21.8 / 27.6 us). At 128 pairs (Qwen3 T=64,
        // Qwen3-30B-A3B T=16) their GEMMs take 48.5 / 43.2 us against 48.4 /
        // 39.5 us on the 32-row kernel, whose grouping launch (7.4 us) makes
        // its steps the longer ones: graph-replayed steps 53.2 / 56.2 us
        // against 56.8 / 59.3 us.
        const long long w8_bytes = (p.moe_type == kQwen3 ? 3LL : 2LL) * H * I;  // one expert's codes
        const bool rows32 = P <= 32 * touched ||
                            (P <= 256 * touched && est_tiles(32) * w8_bytes <= kW8Rows32StreamBytes);
        p.cfg = (P <= kW8GemvPairs) ? kW8Gemv : rows32 ? kLdsRows32 : kLds256w8;
        if (P <= kW8DecPairs && dec_gemv_fits(p)) p.cfg = kDecGemv;
        if (g_tile_policy == kW8Gemv || g_tile_policy == kLdsRows32 || g_tile_policy == kLds256w8 ||
            (g_tile_policy == kDecGemv && dec_gemv_fits(p)))
            p.cfg = g_tile_policy;
    } else if (p.mfma && !policy) {
        const long long wgs256 = est_tiles(256) * cdiv(I, gemm_tile_cols(p.moe_type == kQwen3 ? kGateUp : kFc1, kLds256w8));
        if (P <= 32 * touched) p.cfg = P <= kDecDefaultPairs && dec_gemv_fits(p) ? kDecGemv : kLdsRows32;
        // up to 128 rows per touched expert, where the 128x128 tile would
        // leave the down GEMM too few tiles for the CUs (a narrow hidden
        // dimension: Nomic's 768) and its K is long enough to split (I >=
        // 1024), the 32-row kernel with its K splits: Nomic T=192 / 256 / 512
        // steps 64.0 / 66.7 / 88.5 us on the 128x128 tile against 49.8 /
        // 55.9 / 75.1 us. (Its f32 atomics make these sizes' results vary in
        // the last bits from call to call, as on the decode sizes it takes.)
        else if (P <= 128 * touched && I >= 1024 && est_tiles(128) * cdiv(H, 128) < 8LL * std::max(cus_per_xcd(), 32))
            p.cfg = kLdsRows32;
        else if (wgs256 < 256 && P <= 128 * touched) p.cfg = kLds128;
        else if (H <= 2048 && P < 1024 * touched && (long long)cdiv(H, 256) * est_tiles(128) >= 512)
            p.cfg = kLds128x256o2;
    }
    // (a forced decode kernel on sizes it does not take: the 32-row kernel)
    if (p.cfg == kDecGemv && !dec_gemv_fits(p)) p.cfg = kLdsRows32;
    // the LDS-DMA kernels address operands with 32-bit buffer offsets
    if (is_lds_cfg(p.cfg)) {
        const long long es = 2;
        const long long lim = 0x7fffff00LL;
        if ((long long)T * H * es >= lim || P * I * es >= lim || (long long)H * I * es >= lim) {
            if (fp8) return set_error(CANDLE_MOE_ERR_UNSUPPORTED, "fused_moe_fp8: operands beyond 2 GiB");
            p.cfg = kTile128;
        }
    }
    if (packed && !is_lds_cfg(p.cfg) && p.cfg != kDecGemv)
        return set_error(CANDLE_MOE_ERR_UNSUPPORTED, "fused_moe_packed: operands beyond 2 GiB");
    p.BM = tile_rows(p.cfg);
    // Expert-set path: each distinct sorted expert set becomes one GEMM group
    // over K = k*I; worth it when the sets are few next to the tokens: on
    // average at least half a row tile per set where the hidden size is large
    // (the pair path's f32 combine and finalize grow with H; Qwen3, H = 4096,
    // BM = 256: sets from T >= 3584), 1.4 row tiles with a small hidden size
    // (Nomic, H = 768: pairs 267 against 312 us at T=8192, sets 379 against
    // 404 us at T=12288).
    p.set_path = false;
    p.nkeys = 0;
    // (fp8 weights: on the 8-wave prefill kernel, whose expert-set GEMM keeps
    // its accumulators in per-segment column units)
    if (p.mfma && (!fp8 || p.cfg == kLds256w8) && out16 && (I % 64) == 0 && k <= kSetMaxK &&
        g_combine_policy != 1) {
        long long nk = 1;
        for (int j = 0; j < k && nk <= kSetMaxKeys; ++j) nk *= (E + 1);
        if (nk <= kSetMaxKeys) {
            double sets = 1.0;
            for (int j = 0; j < k; ++j) sets = sets * (E - j) / (j + 1);
            if (sets < 1.0) sets = 1.0;
            p.nkeys = (int)nk;
            const double fill = H >= 2048 ? 0.5 : 1.4;
            // Against the pair path's row stores and k-row sums (16-bit
            // LDS-DMA kernels) the expert sets pay off only once those rows
            // are large: Qwen3 T=4096 / 8192 pairs 454 / 792 against sets 484 /
            // 830 us, T=32768 (537 MB of rows) sets 2346 against 2499 us;
            // Nomic T=12288 / 32768 pairs 377 / 859 against 390 / 899 us.
            const bool rows_ok = p.mfma && is_lds_cfg(p.cfg) && p.dtype != kF32;
            const bool big_rows = (double)P * H * 2.0 >= (double)kSetMinRowBytes;
            p.set_path = p.cfg != kDecGemv &&
                         (g_combine_policy == 2 ||
                          (p.cfg != kLdsRows32 && (double)T >= fill * p.BM * sets && (!rows_ok || big_rows)));
        }
    }
    // K splits for the 32-row (decode) GEMMs and the f32 kernels, whose output
    // tiles can leave most CUs idle. Each split writes an f32 partial tile
    // that the last one sums, so splitting only pays where the weight stream
    // would otherwise run on a few CUs.
    //  * 32-row MFMA kernels: the kernel picks the count from the live tiles of
    //    the grouping (adaptive_split): one round of workgroups (one per CU),
    //    at most 8 splits; here only the bound and the target. (A second round
    //    measured slower: Qwen3 T=64 gate/up 52 -> 47 us, Qwen3-30B-A3B T=1
    //    25 -> 20 us against the host's estimate.)
    //  * f32 kernels (two workgroups per CU, one K chunk in flight each): the
    //    host's count from the expected tiles, up to ~512 workgroups and 16
    //    splits (they gain from more than one round: Nomic T=512 f32 fc1
    //    136 us against 150-190 us with the device's one-round choice).
    p.lds_family = p.mfma && is_lds_cfg(p.cfg);
    p.fused_clear_ok = p.lds_family || is_f32_cfg(p.cfg);
    // Pair path on the LDS-DMA kernels (16-bit): the down GEMM stores each
    // pair's weighted row once and a row-contiguous pass sums a token's k
    // rows, instead of f32 atomics into [T, H] and a finalize pass (the
    // atomics were 27-42 % of the down GEMM on Qwen3 T=2048 and the
    // Qwen3-30B-A3B shapes). Deterministic for every k. Not for the 32-row
    // decode kernels, whose few atomics cost less than the k-row pass
    // (Qwen3-30B-A3B T=16: 90 against 94 us).
    p.rows_path = p.cfg == kDecGemv ||
                  (!p.set_path && p.lds_family && p.dtype != kF32 && p.cfg != kLdsRows32 && p.cfg != kW8Gemv &&
                   (double)P * H * 2.0 <= kRowsMaxBytes);
    p.n_tiles1 = cdiv(I, gemm_tile_cols(p.moe_type == kQwen3 ? kGateUp : kFc1, p.cfg));
    // Decode fc1 (Nomic) likewise on 128-column tiles where the 256-column
    // ones would split K: T=16 / 64 16.8 -> 13.4, 15.2 -> 12.9 us. (The
    // gate/up tile cannot narrow the same way: a wave holds matching gate and
    // up columns, so 128 columns leave two waves per workgroup, whose fewer
    // loads in flight lost 2.6-3.5 us at Qwen3 T=16 / 64.) fp8 weights the
    // same: Nomic T=16 fc1 17.6 -> 12.5 us, against 14.5 us with bf16 weights)
    const long long dev_wgs = 8LL * std::max(cus_per_xcd(), 32);
    p.narrow1 = p.cfg == kLdsRows32 && p.moe_type == kNomic && touched * cdiv(I, 256) < dev_wgs;
    if (p.narrow1) p.n_tiles1 = cdiv(I, 128);
    // Decode down / fc2 GEMM (32-row kernel, 16-bit weights): 128-column
    // tiles where the 256-column tiling would leave CUs without a tile (and
    // so split K) and K = I is long. Twice the tiles then fill the device
    // with fewer or no K splits, which saves the split-K fixup: Qwen3 T=8 /
    // 16 / 64 18.5 -> 16.8, 24.0 -> 21.9, 25.0 -> 23.1 us, Nomic T=16 / 64
    // 16.0 -> 13.6, 16.5 -> 14.2 us. With I = 768 (Qwen3-30B-A3B) or live
    // tiles enough for every CU the wide tiles stay ahead (T=1: 13.1 against
    // 13.6 us, T=16: 50.6 against 56.1 us). fp8 weights the same: Qwen3 T=16
    // / 64 20.4 -> 16.2, 20.5 -> 16.6 us.
    const int down_cols = (p.cfg == kLdsRows32 && I >= 1536 && touched * cdiv(H, 256) < dev_wgs)
                              ? 128
                              : gemm_tile_cols(kDown, p.cfg);
    p.narrow2 = down_cols == 128 && gemm_tile_cols(kDown, p.cfg) != 128;
    p.n_tiles2 = cdiv(H, down_cols);
    if (p.cfg == kW8Gemv) {
        // the grid of the split with the most workgroups (the kernel picks
        // the split from the live row tiles)
        p.n_tiles1 = cdiv(I, gv_wg_cols(p.moe_type == kQwen3 ? kGateUp : kFc1, 4));
        p.n_tiles2 = cdiv(H, gv_wg_cols(kDown, 4));
    }
    p.split1 = p.split2 = 1;
    // tail balance for the 8-wave 256x256 kernel (its K splits meet in the
    // split-K fixup): the tiles of each XCD's last, partly filled round are
    // split along K
    p.tail_cus = (p.lds_family && p.cfg == kLds256w8) ? cus_per_xcd() : 0;
    p.split_target = 0;
    if (p.lds_family && p.cfg == kLdsRows32 && P > 0) {
        p.split_target = cus_per_xcd() > 0 ? 8 * cus_per_xcd() : 256;
        const int bk = tile_bk(p.cfg);
        auto bound = [&](int K) { return std::max(1, std::min(8, cdiv(K, bk))); };
        if (!p.set_path) p.split2 = bound(I);
        p.split1 = bound(H);
    } else if (is_f32_cfg(p.cfg) && P > 0) {
        const long long mt = est_tiles(p.BM);
        const int bk = tile_bk(p.cfg);
        const long long target = 512, max_sp = 16;
        auto choose = [&](long long tiles, int K) {
            if (tiles >= target / 2) return 1;
            const int nk = (K + bk - 1) / bk;
            long long sp = (target + tiles - 1) / tiles;
            if (sp > max_sp) sp = max_sp;
            if (sp > nk) sp = nk;
            if (sp < 1) sp = 1;
            const int per = (int)((nk + sp - 1) / sp);
            return (nk + per - 1) / per;
        };
        if (!p.set_path) p.split2 = choose(mt * p.n_tiles2, I);
        p.split1 = choose(mt * p.n_tiles1, H);
    }
    p.dec_ks1 = p.dec_ks2 = 1;
    if (p.cfg == kDecGemv) {
        // K slices for the gate/up (fc1) GEMM only where they paid: few
        // column blocks of 128 and a large weight stream. Measured steps
        // (router + forward, graph-replayed, cold bf16 weights), sliced
        // against not: Qwen3 T=8 / 64 65.1 / 80.1 against 73.3 / 84.1 us;
        // Qwen3-30B-A3B T=1 / 16 29.6 / 83.4 against 29.0 / 78.4 us, Nomic
        // T=16 36.4 against 35.1 us (the finishing launch costs more than
        // the faster stream saves); fp8 weights (half the bytes) slower
        // sliced too. The down / fc2 GEMM, whose finishing launch sums the
        // pairs anyway, ran 1-3 us faster unsliced on every shape.
        const bool q3 = p.moe_type == kQwen3;
        const long long groups = std::min<long long>(P, E);
        const double wbytes = (double)groups * (q3 ? 2 : 1) * H * I * (fp8 ? 1 : 2);
        if (groups * cdiv(I, 128) < 256 && wbytes >= kDecSliceBytes)
            p.dec_ks1 = dec_slices(P, I, H, q3 ? 2 : 4, q3 ? 2 : 1);
    }
    return CANDLE_MOE_OK;
}

// fp8 expert weights of candle_moe_fused_moe_fp8 (codes [E][N][K], scales [E][N])
struct Fp8Weights {
    const float* gate_scale;
    const float* up_scale;
    const float* down_scale;
};

// Decode path (kDecGemv): the gate/up (fc1) GEMM into inter [P, I] by pair
// (with K slices: f32 partials, then a finishing launch that sums them and
// applies the activation), the down (fc2) GEMM into f32 partials [ks][P][H],
// then a finishing launch that sums each token's pairs (slices in order,
// slots in order, one rounding). The GEMM kernels group the pairs themselves
// (no grouping launch) and choose the slices from the touched experts.
// Columns per lane: 8 with K slices (256-byte runs of [K,N] rows); without,
// the block whose items (touched experts x column blocks, estimated from
// min(P, E)) fall into the fewest per CU for their number: items / ceil(items
// / CUs) largest (a CU with two items takes twice as long as one with one),
// the wider block on ties. [K,N] weights (trans): 8 or 4 columns (16 or
// 8-byte loads; 4-byte loads ran the Qwen3 T=8 gate/up at 78 against 46 us).
// [N,K] weights (16-byte loads of 16 columns whatever the block): 8, 6, 4, 3
// or 2 (blocks of 48 and 96 columns put Qwen3's 1536 and Nomic's 3072
// columns of 8 experts into 256 items).
static int dec_cpl(long long groups, int N, bool trans, int ks_lim) {
    if (ks_lim > 1) return 8;
    const double cus = 8.0 * std::max(cus_per_xcd(), 32);
    static const int kTrans[] = {8, 4}, kNK[] = {8, 6, 4, 3, 2};
    const int* cand = trans ? kTrans : kNK;
    const int ncand = trans ? 2 : 5;
    int best = cand[0];
    double best_b = -1.0;
    for (int i = 0; i < ncand; ++i) {
        const double items = (double)groups * cdiv(N, 16 * cand[i]);
        const double b = items / std::ceil(items / cus);
        if (b > best_b + 1e-9) {
            best_b = b;
            best = cand[i];
        }
    }
    return best;
}
static int run_moe_dec(const Problem& p, const void* x, const void* gate, const void* up, const void* down,
                       const float* rw, const uint32_t* idx, void* out, bool overwrite, char* ws, const Layout& L,
                       hipStream_t s, const Fp8Weights* f8) {
    const bool qwen3 = p.moe_type == kQwen3;
    void* inter = ws + L.inter;
    float* part = reinterpret_cast<float*>(ws + L.acc);
    int* meta = reinterpret_cast<int*>(ws + L.dec_meta);
    DecArgs d = {};
    d.A = x;
    d.B0 = gate;
    d.B1 = up;
    d.C = inter;
    d.part = part;
    d.meta = meta;
    d.idx = idx;
    d.P = (int)p.P;
    d.E = p.E;
    d.K = p.H;
    d.N = p.I;
    d.k_top = p.k;
    d.act = p.act;
    d.strideB = (long long)p.H * p.I;
    d.ldb = (p.packed || f8) ? p.H : p.I;  // gate / up [E][H][I], or packed / fp8 codes [E][I][H]
    d.packed = p.packed ? 1 : 0;
    if (f8) {
        d.w8 = 1;
        d.scale0 = f8->gate_scale;
        d.scale1 = f8->up_scale;
    }
    d.a_bytes = (long long)p.T * p.H * 2;
    d.max_groups = (int)std::min<long long>(p.P, p.E);
    d.rows_max = (int)std::min<long long>(p.P, p.T);
    d.cap = dec_cap();
    d.ks_lim = p.dec_ks1;
    d.cpl = dec_cpl(d.max_groups, p.I, !p.packed && !f8, d.ks_lim);
    d.nblk = cdiv(p.I, 16 * d.cpl);
    const int mode1 = qwen3 ? kGateUp : kFc1;
    hipError_t e;
    {
        ProfScope ps(kSlotGemm1, s);
        e = launch_dec_gemv(mode1, p.dtype, d, s);
        if (e == hipSuccess && d.ks_lim > 1) {
            DecFinish f = {};
            f.part = part;
            f.meta = meta;
            f.ks_lim = d.ks_lim;
            f.P = (int)p.P;
            f.N = p.I;
            f.E = p.E;
            f.T = p.T;
            f.k_top = p.k;
            f.act = p.act;
            f.idx = idx;
            f.scale0 = f8 ? f8->gate_scale : nullptr;
            f.scale1 = f8 ? f8->up_scale : nullptr;
            f.out = inter;
            e = launch_dec_finish(mode1, p.dtype, f, s);
        }
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe decode gate/up GEMM");
    DecArgs d2 = d;
    d2.A = inter;
    d2.B0 = qwen3 ? down : up;
    d2.B1 = nullptr;
    d2.C = nullptr;
    d2.K = p.I;
    d2.N = p.H;
    d2.ldb = (qwen3 && !p.packed && !f8) ? p.H : p.I;  // down [E][I][H] (packed / fp8 [E][H][I]); fc2 [E][H][I]
    d2.a_bytes = p.P * p.I * 2;
    d2.ks_lim = p.dec_ks2;
    // fp8 column scales: multiplied in by the GEMM when it is not K-sliced
    // (its partials are then whole sums), else by the finishing launch
    const float* s2 = f8 ? (qwen3 ? f8->down_scale : f8->up_scale) : nullptr;
    d2.scale0 = d2.ks_lim == 1 ? s2 : nullptr;
    d2.scale1 = nullptr;
    d2.cpl = dec_cpl(d.max_groups, p.H, qwen3 && !p.packed && !f8, d2.ks_lim);
    d2.nblk = cdiv(p.H, 16 * d2.cpl);
    {
        ProfScope ps(kSlotGemm2, s);
        e = launch_dec_gemv(qwen3 ? kDownRows : kFc2Rows, p.dtype, d2, s);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe decode down GEMM");
    {
        ProfScope ps(kSlotFinal, s);
        DecFinish f = {};
        f.part = part;
        f.meta = meta;
        f.ks_lim = d2.ks_lim;
        f.P = (int)p.P;
        f.N = p.H;
        f.E = p.E;
        f.T = p.T;
        f.k_top = p.k;
        f.idx = idx;
        f.routing_w = rw;
        f.scale0 = d2.ks_lim == 1 ? nullptr : s2;
        f.out = out;
        f.overwrite = overwrite ? 1 : 0;
        e = launch_dec_finish(qwen3 ? kDownRows : kFc2Rows, p.dtype, f, s);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe decode row sums");
    return CANDLE_MOE_OK;
}

// sync_zero: the workspace's grouping counters (Layout::sync) are zero
// (library-owned workspaces: cleared at allocation, left zero by every
// launch), which allows the one-launch grouping.
static int run_moe(const Problem& p, const void* x, const void* gate, const void* up, const void* down,
                   const float* rw, const uint32_t* idx, void* out, bool overwrite, char* ws, hipStream_t s,
                   const Fp8Weights* f8 = nullptr, bool sync_zero = false) {
    auto gemm = [&](int mode, const GemmArgs& g) {
        return f8 ? launch_moe_gemm_w8(mode, p.dtype, p.cfg, g, s) : launch_moe_gemm(mode, p.dtype, p.cfg, g, s);
    };
    const Layout L = make_layout(p);
    GroupingBufs gb = {};
    gb.offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
    gb.block_counts = reinterpret_cast<int32_t*>(ws + L.block_counts);
    gb.sorted_pair = reinterpret_cast<int32_t*>(ws + L.sorted_pair);
    gb.tile_row = reinterpret_cast<int32_t*>(ws + L.tile_row);
    gb.tile_exp = reinterpret_cast<int32_t*>(ws + L.tile_exp);
    gb.num_tiles = reinterpret_cast<int32_t*>(ws + L.num_tiles);
    int32_t* counters = reinterpret_cast<int32_t*>(ws + L.counters);
    if (p.split1 > 1 || p.split2 > 1) {
        const long long mt = grouping_max_tiles(p.P, p.E, p.BM);
        gb.zero_ptr = counters;
        gb.zero_n = (int)(mt * (p.n_tiles1 > p.n_tiles2 ? p.n_tiles1 : p.n_tiles2));
    } else if (p.tail_cus > 0) {
        gb.zero_ptr = counters;
        gb.zero_n = 8 * p.tail_cus;
    }
    hipError_t e;

    const bool qwen3 = p.moe_type == kQwen3;
    const int m_tiles_max = (int)grouping_max_tiles(p.P, p.E, p.BM);
    void* inter = ws + L.inter;
    float* acc = reinterpret_cast<float*>(ws + L.acc);
    GroupingBufs tb = {};
    int32_t* pair_dest = nullptr;
    if (p.set_path) {
        tb.offsets = reinterpret_cast<int32_t*>(ws + L.k_offsets);
        tb.block_counts = reinterpret_cast<int32_t*>(ws + L.k_block_counts);
        tb.sorted_pair = reinterpret_cast<int32_t*>(ws + L.tok_sorted);
        tb.tile_row = reinterpret_cast<int32_t*>(ws + L.tile_row2);
        tb.tile_exp = reinterpret_cast<int32_t*>(ws + L.tile_key2);
        tb.num_tiles = reinterpret_cast<int32_t*>(ws + L.num_tiles2);
        pair_dest = reinterpret_cast<int32_t*>(ws + L.pair_dest);
    }
    if (p.cfg == kDecGemv) return run_moe_dec(p, x, gate, up, down, rw, idx, out, overwrite, ws, L, s, f8);
    {
        // pairs by expert and, on the expert-set path, tokens by expert set
        const GroupJob pj = pair_grouping_job(idx, p.P, p.E, p.BM, gb);
        GroupJob tj = {};
        if (p.set_path) tj = set_grouping_job(idx, p.T, p.k, p.E, p.nkeys, p.BM, tb, pair_dest);
        ProfScope ps(kSlotGroup, s);
        const bool one = sync_zero && g_grouping_mode != 1 &&
                         (g_grouping_mode == 2 || grouping_blocks(p.P) <= kGroupOneMaxBlocks);
        const int cus = cus_per_xcd() > 0 ? 8 * cus_per_xcd() : 0;
        e = launch_groupings(pj, p.set_path ? &tj : nullptr, s,
                             one ? reinterpret_cast<int32_t*>(ws + L.sync) : nullptr, cus,
                             g_grouping_mode == 2 ? -1 : kGroupSpin);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe grouping");

    GemmArgs g1 = {};
    g1.A = x;
    g1.B0 = gate;
    g1.B1 = up;
    g1.C = inter;
    g1.routing_w = rw;
    g1.sorted_pair = gb.sorted_pair;
    g1.sorted_n = (int)p.P;
    g1.tile_row = gb.tile_row;
    g1.tile_exp = gb.tile_exp;
    g1.num_tiles = gb.num_tiles;
    g1.offsets = gb.offsets;
    g1.strideB = (long long)p.H * p.I;
    g1.ldb = p.packed ? p.H : p.I;  // gate / up / fc1: [E][H][I], or packed [E][I][H]
    g1.packed = p.packed ? 1 : 0;
    g1.K = p.H;
    g1.N = p.I;
    g1.k_top = p.k;
    g1.act = p.act;
    const int mode1 = qwen3 ? kGateUp : kFc1;
    g1.n_tiles = p.n_tiles1;
    g1.narrow = p.narrow1 ? 1 : 0;
    g1.m_tiles_max = m_tiles_max;
    g1.ksplit = p.split1;
    g1.split_target = p.split_target;
    g1.partial = reinterpret_cast<float*>(ws + L.partial);
    g1.counters = counters;
    g1.tail_cus = p.tail_cus;
    // the gate/up workgroups clear the pair path's accumulator
    const bool fused_clear = !p.set_path && !p.rows_path && p.fused_clear_ok;
    if (fused_clear) {
        g1.zero_f32 = acc;
        g1.zero_n = (long long)p.T * p.H;
    }
    g1.a_bytes = (long long)p.T * p.H * (p.dtype == kF32 ? 4 : 2);
    g1.pair_dest = pair_dest;
    g1.fold_w = p.set_path ? 1 : 0;
    g1.n_experts = p.E;
    g1.seg_len = p.I;
    if (f8) {  // codes [E][I][H]: n-rows of H bytes
        g1.ldb = p.H;
        g1.scale0 = f8->gate_scale;
        g1.scale1 = f8->up_scale;
    }
    {
        ProfScope ps(kSlotGemm1, s);
        e = gemm(mode1, g1);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe gate/up GEMM");

    if (p.set_path) {
        // down / fc2 over the expert sets, straight into the caller's output
        GemmArgs g2 = g1;
        g2.A = inter;
        g2.B0 = qwen3 ? down : up;
        g2.B1 = nullptr;
        g2.C = out;
        g2.strideB = (long long)p.I * p.H;
        g2.ldb = (qwen3 && !p.packed) ? p.H : p.I;  // down [E][I][H] (packed [E][H][I]); fc2 [E][H][I]
        g2.K = p.k * p.I;
        g2.N = p.H;
        g2.a_bytes = p.P * p.I * 2;
        g2.offsets = tb.offsets;
        g2.tile_row = tb.tile_row;
        g2.tile_exp = tb.tile_exp;
        g2.num_tiles = tb.num_tiles;
        g2.tok_sorted = tb.sorted_pair;
        g2.pair_dest = nullptr;
        g2.fold_w = 0;
        g2.ksplit = 1;
        g2.narrow = 0;
        g2.zero_f32 = nullptr;
        g2.zero_n = 0;
        g2.overwrite = overwrite ? 1 : 0;
        if (f8) {  // codes [E][H][I] (down, or Nomic's fc2 in up): n-rows of I bytes, scales per expert
            g2.ldb = p.I;
            g2.scale0 = qwen3 ? f8->down_scale : f8->up_scale;
            g2.scale1 = nullptr;
        }
        const int mode2 = qwen3 ? kDownSet : kFc2Set;
        g2.n_tiles = cdiv(p.H, gemm_tile_cols(mode2, p.cfg));
        g2.m_tiles_max = (int)set_tiles_max(p);
        {
            ProfScope ps(kSlotGemm2, s);
            e = gemm(mode2, g2);
        }
        if (e != hipSuccess) return hip_fail(e, "fused_moe down GEMM (expert sets)");
        return CANDLE_MOE_OK;
    }

    if (!fused_clear && !p.rows_path) {
        ProfScope ps(kSlotZero, s);
        e = launch_fill_zero_f32(acc, (long long)p.T * p.H, s);
        if (e != hipSuccess) return hip_fail(e, "fused_moe accumulator clear");
    }

    GemmArgs g2 = g1;
    g2.A = inter;
    g2.B0 = qwen3 ? down : up;
    g2.B1 = nullptr;
    g2.C = p.rows_path ? static_cast<void*>(ws + L.acc) : static_cast<void*>(acc);
    g2.strideB = (long long)p.I * p.H;
    g2.ldb = (qwen3 && !p.packed) ? p.H : p.I;  // down [E][I][H] (packed [E][H][I]); fc2 [E][H][I]
    g2.K = p.I;
    g2.N = p.H;
    g2.a_bytes = p.P * p.I * (p.dtype == kF32 ? 4 : 2);
    const int mode2 = p.rows_path ? (qwen3 ? kDownRows : kFc2Rows) : (qwen3 ? kDown : kFc2);
    g2.n_tiles = p.n_tiles2;
    g2.narrow = p.narrow2 ? 1 : 0;
    g2.ksplit = p.split2;
    g2.split_target = p.split_target;
    g2.partial = reinterpret_cast<float*>(ws + L.partial);
    g2.counters = counters;
    g2.zero_f32 = nullptr;
    g2.zero_n = 0;
    if (f8) {  // codes [E][H][I] (down, or Nomic's fc2 in up): n-rows of I bytes
        g2.ldb = p.I;
        g2.scale0 = qwen3 ? f8->down_scale : f8->up_scale;
        g2.scale1 = nullptr;
    }
    {
        ProfScope ps(kSlotGemm2, s);
        e = gemm(mode2, g2);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe down GEMM");

    {
        ProfScope ps(kSlotFinal, s);
        e = p.rows_path ? launch_pair_rows_sum(out, p.dtype, ws + L.acc, static_cast<const uint32_t*>(idx), p.E,
                                               p.T, p.k, p.H, overwrite, s)
                        : launch_finalize(out, p.dtype, acc, (long long)p.T * p.H, overwrite, s);
    }
    if (e != hipSuccess) return hip_fail(e, "fused_moe finalize");
    return CANDLE_MOE_OK;
}

static int check_ptrs(const Problem& p, const void* x, const void* gate, const void* up, const void* down,
                      const void* rw, const void* idx, const void* out) {
    if (p.T == 0) return CANDLE_MOE_OK;
    if (!x || !gate || !up || !rw || !idx || !out)
        return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: null tensor pointer");
    if (p.moe_type == kQwen3 && !down)
        return set_error(CANDLE_MOE_ERR_INVALID, "fused_moe: down_weights is required for moe_type 0 (Qwen3)");
    return CANDLE_MOE_OK;
}

// Stream-ordered pool allocation; the pool keeps freed memory (release
// threshold raised once per device) so repeated calls do not go to the driver.
// Library-owned workspaces, one per (device, stream), kept between calls and
// grown when a call needs more: allocating and freeing a stream-ordered
// workspace on every call costs ~50 us of host time, more than a whole
// decode step's kernels. Reuse is safe because every call on a stream is
// ordered after the previous one on that stream; the lock is held while a
// call enqueues its kernels, so two host threads on one stream never
// interleave their launches over the shared buffer. A grown buffer's old
// allocation is released with hipFreeAsync on its own stream.
struct OwnedWs {
    int device;
    hipStream_t stream;
    void* ptr;
    size_t bytes;
};
static std::mutex g_ws_mu;
static std::vector<OwnedWs> g_ws;

// A stream being captured into a graph gets no new or larger workspace
// (err = hipErrorStreamCaptureUnsupported): hipMallocAsync there would add an
// allocation node to the caller's graph, memory the graph owns and releases
// when it is destroyed, while this table would keep handing it out.
static OwnedWs* owned_ws_locked(int dev, hipStream_t s, size_t need, hipError_t& err) {
    err = hipSuccess;
    OwnedWs* w = nullptr;
    for (auto& e : g_ws)
        if (e.device == dev && e.stream == s) w = &e;
    if (w && w->bytes >= need) return w;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        err = hipErrorStreamCaptureUnsupported;
        return nullptr;
    }
    // grow by at least 1.5x and to whole MiB, so that a slowly growing T
    // does not reallocate on every call
    size_t want = need + need / 2;
    want = (want + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    void* mem = nullptr;
    err = hipMallocAsync(&mem, want, s);
    if (err != hipSuccess) return nullptr;
    // the header's counters start at zero (a kernel, not a memset node,
    // should the call be captured into a graph)
    err = launch_fill_zero_f32(reinterpret_cast<float*>(mem), (long long)(kWsHeaderBytes / 4), s);
    if (err != hipSuccess) {
        (void)hipFreeAsync(mem, s);
        return nullptr;
    }
    if (w) {
        if (w->ptr) (void)hipFreeAsync(w->ptr, s);
        w->ptr = mem;
        w->bytes = want;
        return w;
    }
    g_ws.push_back(OwnedWs{dev, s, mem, want});
    return &g_ws.back();
}

static int ws_fail(const char* who, size_t need, hipError_t e) {
    if (e == hipErrorStreamCaptureUnsupported)
        return set_error(CANDLE_MOE_ERR_WORKSPACE,
                         "%s: the stream is being captured and its library workspace is missing or smaller than "
                         "the %zu bytes this call needs: make one call of this size on the stream before capturing",
                         who, need);
    return set_error(CANDLE_MOE_ERR_WORKSPACE, "%s: hipMallocAsync(%zu) failed: %s", who, need, hipGetErrorString(e));
}

int trim_owned_workspaces() {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) cur = -1;
    hipError_t first = hipSuccess;
    // hipFree, not hipFreeAsync on the stream of each workspace: that stream
    // may have been destroyed since its last call (hipFree waits for the
    // device instead)
    for (auto& e : g_ws) {
        if (!e.ptr) continue;
        if (e.device != cur) (void)hipSetDevice(e.device);
        const hipError_t r = hipFree(e.ptr);
        if (first == hipSuccess) first = r;
        if (e.device != cur && cur >= 0) (void)hipSetDevice(cur);
    }
    g_ws.clear();
    return first == hipSuccess ? CANDLE_MOE_OK : hip_fail(first, "trim workspaces: hipFree");
}

int fused_moe_impl(const void* x, const void* gate, const void* up, const void* down, const void* rw,
                   const void* idx, void* out, int T, int H, int I, int E, int k, int act, uint32_t moe_type,
                   uint32_t dtype, void* ws, size_t ws_bytes, bool own_ws, bool overwrite, void* stream,
                   const Fp8Weights* f8, bool packed) {
    clear_error();
    Problem p;
    auto a16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    const bool aligned16 = a16(x) && a16(gate) && a16(up) && a16(down);
    int rc = check_problem(T, H, I, E, k, act, moe_type, dtype, p, aligned16, a16(out), f8 != nullptr, packed);
    if (rc) return rc;
    rc = check_ptrs(p, x, gate, up, down, rw, idx, out);
    if (rc) return rc;
    if (T == 0) return CANDLE_MOE_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Layout L = make_layout(p);
    if (!own_ws) {
        if (!ws || ws_bytes < L.total)
            return set_error(CANDLE_MOE_ERR_WORKSPACE, "fused_moe: workspace of %zu bytes is smaller than the %zu required",
                             ws_bytes, L.total);
        if ((uintptr_t)ws % 256)
            return set_error(CANDLE_MOE_ERR_WORKSPACE, "fused_moe: workspace must be 256-byte aligned");
        return run_moe(p, x, gate, up, down, reinterpret_cast<const float*>(rw),
                       reinterpret_cast<const uint32_t*>(idx), out, overwrite, reinterpret_cast<char*>(ws), s, f8);
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "fused_moe: hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    OwnedWs* w = owned_ws_locked(dev, s, L.total, e);
    if (!w) return ws_fail("fused_moe", L.total, e);
    return run_moe(p, x, gate, up, down, reinterpret_cast<const float*>(rw), reinterpret_cast<const uint32_t*>(idx),
                   out, overwrite, reinterpret_cast<char*>(w->ptr), s, f8, true);
}

// ----------------------------------------------- fused MoE without allocation
// Scratch of candle_moe_fused_moe_noalloc: a file-scope device array, one per
// GPU the library is loaded on, held until the process ends. In host code
// `scratch` names a host-side stand-in, not a device address: the device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and only that address is ever handed to kernels.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_of_current_device(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "fused_moe_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(CANDLE_MOE_ERR_UNSUPPORTED, "fused_moe_noalloc: device ordinal %d beyond %d", dev,
                         kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                   "fused_moe_noalloc: hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return CANDLE_MOE_OK;
}

int fused_moe_noalloc_impl(const void* x, const void* gate, const void* up, const void* down, const void* rw,
                           const void* idx, void* out, int T, int H, int I, int E, int k, int act, uint32_t moe_type,
                           uint32_t dtype, void* stream) {
    clear_error();
    Problem p;
    auto a16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    const bool aligned16 = a16(x) && a16(gate) && a16(up) && a16(down);
    int rc = check_problem(T, H, I, E, k, act, moe_type, dtype, p, aligned16, a16(out));
    if (rc) return rc;
    rc = check_ptrs(p, x, gate, up, down, rw, idx, out);
    if (rc) return rc;
    if (T == 0) return CANDLE_MOE_OK;
    const Layout L = make_layout(p);
    if (L.total > kNoAllocScratchBytes)
        return set_error(CANDLE_MOE_ERR_WORKSPACE,
                         "fused_moe_noalloc: this call needs %zu bytes of scratch; the library holds %zu per device "
                         "(use fused_moe or candle_moe_fused_moe_ws for larger calls)",
                         L.total, kNoAllocScratchBytes);
    void* ws = nullptr;
    rc = scratch_of_current_device(&ws);
    if (rc) return rc;
    // every piece of the layout that must start at zero (split-K arrival
    // counters, the f32 accumulator) is cleared by this call's own kernels.
    // The grouping takes its two-launch form (sync_zero false): the one-launch
    // form counts workgroups in and out on counters that the previous launch
    // leaves at zero, and on this array shared by every call on the GPU an
    // overlapping call could leave them nonzero for the calls after it.
    // Batches of up to kGroupSmallMax pairs (decode) take the one-workgroup
    // grouping either way.
    return run_moe(p, x, gate, up, down, reinterpret_cast<const float*>(rw), reinterpret_cast<const uint32_t*>(idx),
                   out, false, reinterpret_cast<char*>(ws), reinterpret_cast<hipStream_t>(stream), nullptr, false);
}

size_t fused_moe_ws_size(int T, int H, int I, int E, int k, uint32_t dtype) {
    // the kernel choice may depend on the operands' alignment and on the
    // moe_type (the gate/up and fc1 tiles differ in width): enough for each
    size_t most = 0;
    for (uint32_t mt = 0; mt < 2; ++mt)
        for (int al = 0; al < 2; ++al) {
            Problem p;
            if (check_problem(T, H, I, E, k, 0, mt, dtype, p, al != 0)) return 0;
            most = std::max(most, make_layout(p).total);
        }
    return most;
}

}  // namespace cm

// ----------------------------------------------------------------- C ABI
extern "C" {

void topk_softmax(const void* gating_output, void* topk_weight, void* topk_indices, void* token_expert_indices,
                  int num_experts, int num_tokens, int topk, void* stream) {
    (void)cm::topk_softmax_impl(gating_output, cm::kF32, topk_weight, cm::kF32, topk_indices, token_expert_indices,
                                num_experts, num_tokens, topk, stream);
}

int candle_moe_topk_softmax_status(const void* gating_output, void* topk_weight, void* topk_indices,
                                   void* token_expert_indices, int num_experts, int num_tokens, int topk,
                                   void* stream) {
    return cm::topk_softmax_impl(gating_output, cm::kF32, topk_weight, cm::kF32, topk_indices, token_expert_indices,
                                 num_experts, num_tokens, topk, stream);
}

int candle_moe_topk_softmax_ex(const void* gating_output, int gating_dtype, void* topk_weight, int weight_dtype,
                               void* topk_indices, void* token_expert_indices, int num_experts, int num_tokens,
                               int topk, void* stream) {
    if (gating_dtype < 0 || gating_dtype > 2 || weight_dtype < 0 || weight_dtype > 2)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "topk_softmax: dtype codes must be 0, 1 or 2");
    return cm::topk_softmax_impl(gating_output, gating_dtype, topk_weight, weight_dtype, topk_indices,
                                 token_expert_indices, num_experts, num_tokens, topk, stream);
}

void fused_moe(const void* input, const void* gate_weights, const void* up_weights, const void* down_weights,
               const void* routing_weights, const void* expert_indices, void* output, int num_tokens, int hidden_dim,
               int intermediate_dim, int num_experts, int num_selected_experts, int activation_type,
               uint32_t moe_type, uint32_t dtype, void* stream) {
    (void)cm::fused_moe_impl(input, gate_weights, up_weights, down_weights, routing_weights, expert_indices, output,
                             num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts,
                             activation_type, moe_type, dtype, nullptr, 0, true, false, stream);
}

int candle_moe_fused_moe_status(const void* input, const void* gate_weights, const void* up_weights,
                                const void* down_weights, const void* routing_weights, const void* expert_indices,
                                void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
                                void* stream) {
    return cm::fused_moe_impl(input, gate_weights, up_weights, down_weights, routing_weights, expert_indices, output,
                              num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts,
                              activation_type, moe_type, dtype, nullptr, 0, true, false, stream);
}

int candle_moe_fused_moe_noalloc(const void* input, const void* gate_weights, const void* up_weights,
                                 const void* down_weights, const void* routing_weights, const void* expert_indices,
                                 void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                 int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
                                 void* stream) {
    return cm::fused_moe_noalloc_impl(input, gate_weights, up_weights, down_weights, routing_weights, expert_indices,
                                      output, num_tokens, hidden_dim, intermediate_dim, num_experts,
                                      num_selected_experts, activation_type, moe_type, dtype, stream);
}

size_t candle_moe_fused_moe_noalloc_scratch_bytes(void) { return cm::kNoAllocScratchBytes; }

size_t candle_moe_fused_moe_workspace_size(int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                           int num_selected_experts, uint32_t dtype) {
    return cm::fused_moe_ws_size(num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts, dtype);
}

int candle_moe_fused_moe_ws(const void* input, const void* gate_weights, const void* up_weights,
                            const void* down_weights, const void* routing_weights, const void* expert_indices,
                            void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                            int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
                            void* workspace, size_t workspace_bytes, void* stream) {
    return cm::fused_moe_impl(input, gate_weights, up_weights, down_weights, routing_weights, expert_indices, output,
                              num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts,
                              activation_type, moe_type, dtype, workspace, workspace_bytes, false, false, stream);
}

int candle_moe_fused_moe_fp8(const void* input, const void* gate_q, const void* up_q, const void* down_q,
                             const float* gate_scale, const float* up_scale, const float* down_scale,
                             const void* routing_weights, const void* expert_indices, void* output, int num_tokens,
                             int hidden_dim, int intermediate_dim, int num_experts, int num_selected_experts,
                             int activation_type, uint32_t moe_type, uint32_t dtype, void* stream) {
    cm::clear_error();
    if (num_tokens > 0) {
        if (!gate_scale || (moe_type == 0 && (!up_scale || !down_scale)) || (moe_type == 1 && !up_scale))
            return cm::set_error(CANDLE_MOE_ERR_INVALID, "fused_moe_fp8: null scale pointer");
        if (!up_q) return cm::set_error(CANDLE_MOE_ERR_INVALID, "fused_moe_fp8: null tensor pointer");
    }
    const cm::Fp8Weights f8 = {gate_scale, up_scale, down_scale};
    return cm::fused_moe_impl(input, gate_q, up_q, down_q, routing_weights, expert_indices, output, num_tokens,
                              hidden_dim, intermediate_dim, num_experts, num_selected_experts, activation_type,
                              moe_type, dtype, nullptr, 0, true, false, stream, &f8);
}

int candle_moe_quantize_fp8(const void* weights, uint32_t dtype, int num_experts, int k_dim, int n_dim, int input_kn,
                            void* codes, float* scales, void* stream) {
    cm::clear_error();
    if (dtype > 2) return cm::set_error(CANDLE_MOE_ERR_INVALID, "quantize_fp8: dtype must be 0, 1 or 2 (got %u)", dtype);
    if (num_experts < 0 || k_dim < 0 || n_dim < 0)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "quantize_fp8: sizes must be >= 0");
    if ((long long)num_experts * k_dim * n_dim == 0) return CANDLE_MOE_OK;
    if (!weights || !codes || !scales) return cm::set_error(CANDLE_MOE_ERR_INVALID, "quantize_fp8: null pointer");
    const hipError_t e = cm::launch_quantize_fp8(weights, (int)dtype, num_experts, k_dim, n_dim, input_kn ? 1 : 0,
                                                 reinterpret_cast<uint8_t*>(codes), scales,
                                                 reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "quantize_fp8 launch");
}

int candle_moe_dequantize_fp8(const void* codes, const float* scales, int num_experts, int n_dim, int k_dim, void* out,
                              uint32_t dtype, void* stream) {
    cm::clear_error();
    if (dtype > 2) return cm::set_error(CANDLE_MOE_ERR_INVALID, "dequantize_fp8: dtype must be 0, 1 or 2 (got %u)", dtype);
    if (num_experts < 0 || k_dim < 0 || n_dim < 0)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "dequantize_fp8: sizes must be >= 0");
    if ((long long)num_experts * k_dim * n_dim == 0) return CANDLE_MOE_OK;
    if (!codes || !scales || !out) return cm::set_error(CANDLE_MOE_ERR_INVALID, "dequantize_fp8: null pointer");
    const hipError_t e = cm::launch_dequantize_fp8(reinterpret_cast<const uint8_t*>(codes), scales, num_experts, n_dim,
                                                   k_dim, out, (int)dtype, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "dequantize_fp8 launch");
}

// Scratch of candle_moe_group_pairs: per-block counts and the row-tile table
// (256-row tiles) of the grouping.
static size_t group_pairs_ws(long long P, int E) {
    const long long nb = cm::grouping_blocks(P);
    const long long mt = cm::grouping_max_tiles(P, E, 256);
    return cm::a256_bytes((size_t)(nb > 0 ? nb : 1) * E * 4) + 2 * cm::a256_bytes((size_t)(mt > 0 ? mt : 1) * 4) + 256;
}

size_t candle_moe_grouping_workspace_size(int num_pairs, int num_experts) {
    if (num_pairs < 0 || num_experts < 1 || num_experts > 4096) return 0;
    return group_pairs_ws(num_pairs, num_experts);
}

int candle_moe_group_pairs(const void* expert_indices, int num_pairs, int num_experts, void* offsets,
                           void* sorted_pairs, void* workspace, size_t workspace_bytes, void* stream) {
    cm::clear_error();
    const int P = num_pairs, E = num_experts;
    if (P < 0) return cm::set_error(CANDLE_MOE_ERR_INVALID, "group_pairs: num_pairs must be >= 0 (got %d)", P);
    if (E < 1 || E > 4096)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "group_pairs: num_experts must be in [1, 4096] (got %d)", E);
    if (!offsets || (P > 0 && (!expert_indices || !sorted_pairs)))
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "group_pairs: null pointer");
    const size_t need = group_pairs_ws(P, E);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 256))
        return cm::set_error(CANDLE_MOE_ERR_WORKSPACE,
                             "group_pairs: workspace must be 256-byte aligned and hold %zu bytes (got %zu)", need,
                             workspace_bytes);
    char* ws = reinterpret_cast<char*>(workspace);
    const long long nb = cm::grouping_blocks(P);
    const long long mt = cm::grouping_max_tiles(P, E, 256);
    cm::GroupingBufs gb = {};
    gb.offsets = reinterpret_cast<int32_t*>(offsets);
    gb.sorted_pair = reinterpret_cast<int32_t*>(sorted_pairs);
    gb.block_counts = reinterpret_cast<int32_t*>(ws);
    ws += cm::a256_bytes((size_t)(nb > 0 ? nb : 1) * E * 4);
    gb.tile_row = reinterpret_cast<int32_t*>(ws);
    ws += cm::a256_bytes((size_t)(mt > 0 ? mt : 1) * 4);
    gb.tile_exp = reinterpret_cast<int32_t*>(ws);
    ws += cm::a256_bytes((size_t)(mt > 0 ? mt : 1) * 4);
    gb.num_tiles = reinterpret_cast<int32_t*>(ws);
    const cm::GroupJob pj =
        cm::pair_grouping_job(reinterpret_cast<const uint32_t*>(expert_indices), P, E, 256, gb);
    const hipError_t e = cm::launch_groupings(pj, nullptr, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "group_pairs launch");
}

int candle_moe_router_topk(const void* hidden, const void* router_weight, void* topk_weight, void* topk_indices,
                           void* token_expert_indices, int num_tokens, int hidden_dim, int num_experts, int topk,
                           uint32_t dtype, void* stream) {
    cm::clear_error();
    const int T = num_tokens, H = hidden_dim, E = num_experts, k = topk;
    if (T < 0) return cm::set_error(CANDLE_MOE_ERR_INVALID, "router_topk: num_tokens must be >= 0 (got %d)", T);
    if (E < 1 || E > 128)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "router_topk: num_experts must be in [1, 128] (got %d)", E);
    if (k < 1 || k > E)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "router_topk: topk must be in [1, num_experts=%d] (got %d)", E, k);
    if (dtype > 2) return cm::set_error(CANDLE_MOE_ERR_INVALID, "router_topk: dtype code must be 0, 1 or 2");
    const int epv = dtype == cm::kF32 ? 4 : 8;
    if (H < 1 || H % epv)
        return cm::set_error(CANDLE_MOE_ERR_UNSUPPORTED,
                             "router_topk: hidden_dim must be a positive multiple of %d for this dtype (got %d)", epv, H);
    // the matrix-core kernel addresses 32 rows of hidden and the whole weight
    // with 31-bit byte offsets
    if (H > (1 << 22))
        return cm::set_error(CANDLE_MOE_ERR_UNSUPPORTED, "router_topk: hidden_dim must be <= 4194304 (got %d)", H);
    if (T == 0) return CANDLE_MOE_OK;
    if (!hidden || !router_weight || !topk_weight || !topk_indices || !token_expert_indices)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "router_topk: null tensor pointer");
    if (((uintptr_t)hidden | (uintptr_t)router_weight) & 15)
        return cm::set_error(CANDLE_MOE_ERR_UNSUPPORTED, "router_topk: hidden and router_weight must be 16-byte aligned");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // small batches split K over workgroups, with f32 partials in the
    // library-owned workspace of this (device, stream) (held while enqueuing,
    // as fused_moe does)
    // (after the workspace header, whose counters stay zero)
    const size_t rneed = cm::router_ws_bytes(T, H, E, (int)dtype);
    const size_t need = rneed > 0 ? cm::kWsHeaderBytes + rneed : 0;
    hipError_t e = hipSuccess;
    if (need > 0) {
        int dev = 0;
        e = hipGetDevice(&dev);
        if (e != hipSuccess) return cm::hip_fail(e, "router_topk: hipGetDevice");
        std::lock_guard<std::mutex> lk(cm::g_ws_mu);
        cm::OwnedWs* w = cm::owned_ws_locked(dev, s, need, e);
        if (!w) return cm::ws_fail("router_topk", need, e);
        e = cm::launch_router_topk(hidden, router_weight, (int)dtype, reinterpret_cast<float*>(topk_weight),
                                   reinterpret_cast<uint32_t*>(topk_indices),
                                   reinterpret_cast<uint32_t*>(token_expert_indices), T, H, E, k, s,
                                   reinterpret_cast<float*>(static_cast<char*>(w->ptr) + cm::kWsHeaderBytes),
                                   w->bytes - cm::kWsHeaderBytes);
    } else {
        e = cm::launch_router_topk(hidden, router_weight, (int)dtype, reinterpret_cast<float*>(topk_weight),
                                   reinterpret_cast<uint32_t*>(topk_indices),
                                   reinterpret_cast<uint32_t*>(token_expert_indices), T, H, E, k, s);
    }
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "router_topk launch");
}

int candle_moe_pack_weights(const void* weights, uint32_t dtype, int num_experts, int k_dim, int n_dim,
                            void* packed, void* stream) {
    cm::clear_error();
    if (dtype > 1)
        return cm::set_error(CANDLE_MOE_ERR_UNSUPPORTED, "pack_weights: dtype must be 0 (f16) or 1 (bf16) (got %u)",
                             dtype);
    if (num_experts < 0 || k_dim < 0 || n_dim < 0)
        return cm::set_error(CANDLE_MOE_ERR_INVALID, "pack_weights: sizes must be >= 0");
    if ((long long)num_experts * k_dim * n_dim == 0) return CANDLE_MOE_OK;
    if (!weights || !packed) return cm::set_error(CANDLE_MOE_ERR_INVALID, "pack_weights: null tensor pointer");
    if (k_dim > 64 * 65535 || num_experts > 65535)
        return cm::set_error(CANDLE_MOE_ERR_UNSUPPORTED, "pack_weights: k_dim <= 4194240 and num_experts <= 65535");
    const hipError_t e = cm::launch_pack_kn(weights, num_experts, k_dim, n_dim, packed,
                                            reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "pack_weights launch");
}

int candle_moe_fused_moe_packed(const void* input, const void* gate_packed, const void* up_packed,
                                const void* down_packed, const void* routing_weights, const void* expert_indices,
                                void* output, int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                int num_selected_experts, int activation_type, uint32_t moe_type, uint32_t dtype,
                                void* stream) {
    return cm::fused_moe_impl(input, gate_packed, up_packed, down_packed, routing_weights, expert_indices, output,
                              num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts,
                              activation_type, moe_type, dtype, nullptr, 0, true, false, stream, nullptr, true);
}

int candle_moe_test_router_exp(uint32_t first_bits, uint32_t count, uint32_t* stats, void* stream) {
    cm::clear_error();
    if (!stats) return cm::set_error(CANDLE_MOE_ERR_INVALID, "test_router_exp: null stats pointer");
    const hipError_t e = cm::launch_router_exp_check(first_bits, count, stats, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CANDLE_MOE_OK : cm::hip_fail(e, "test_router_exp launch");
}

int candle_moe_trim_workspaces(void) {
    cm::clear_error();
    return cm::trim_owned_workspaces();
}

const char* candle_moe_last_error(void) { return cm::g_last_error.c_str(); }

int candle_moe_set_combine_policy(int policy) {
    if (policy < 0 || policy > 2) return cm::set_error(CANDLE_MOE_ERR_INVALID, "combine policy must be 0, 1 or 2");
    cm::g_combine_policy = policy;
    return CANDLE_MOE_OK;
}

int candle_moe_set_grouping_mode(int mode) {
    if (mode < 0 || mode > 2) return cm::set_error(CANDLE_MOE_ERR_INVALID, "grouping mode must be 0, 1 or 2");
    cm::g_grouping_mode = mode;
    return CANDLE_MOE_OK;
}

int candle_moe_set_tile_policy(int policy) {
    if (policy < 0 || policy >= cm::kNumTileCfgs || !cm::is_shipped_cfg(policy))
        return cm::set_error(CANDLE_MOE_ERR_INVALID,
                             "tile policy must be one of 0 (auto), 1, 5, 7, 12, 14, 15, 16, 17, 18 (got %d)", policy);
    cm::g_tile_policy = policy;
    return CANDLE_MOE_OK;
}

int candle_moe_fused_moe_path_ex(int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                                 int num_selected_experts, uint32_t dtype, uint32_t moe_type) {
    cm::Problem p;
    if (cm::check_problem(num_tokens, hidden_dim, intermediate_dim, num_experts, num_selected_experts, 0, moe_type,
                          dtype, p))
        return -1;
    return (p.set_path ? 2 : (p.mfma ? 1 : 0)) | (p.cfg << 2) | (p.rows_path ? (1 << 8) : 0);
}

int candle_moe_fused_moe_path(int num_tokens, int hidden_dim, int intermediate_dim, int num_experts,
                              int num_selected_experts, uint32_t dtype) {
    const int c = candle_moe_fused_moe_path_ex(num_tokens, hidden_dim, intermediate_dim, num_experts,
                                               num_selected_experts, dtype, 0);
    return c < 0 ? c : (c & 0xff);
}

int candle_moe_profile_begin(void) {
    std::lock_guard<std::mutex> lk(cm::g_prof_mu);
    cm::g_prof_on = true;
    cm::g_prof_mask = ~0u;
    return cm::kNumSlots;
}

int candle_moe_profile_begin_slots(uint32_t slot_mask) {
    std::lock_guard<std::mutex> lk(cm::g_prof_mu);
    cm::g_prof_on = true;
    cm::g_prof_mask = slot_mask;
    return cm::kNumSlots;
}

int candle_moe_profile_end(double* total_ms, int* counts, int nslots) {
    std::vector<cm::ProfRec> recs;
    {
        std::lock_guard<std::mutex> lk(cm::g_prof_mu);
        cm::g_prof_on = false;
        recs.swap(cm::g_prof);
    }
    for (int i = 0; i < nslots; ++i) {
        if (total_ms) total_ms[i] = 0.0;
        if (counts) counts[i] = 0;
    }
    int rc = CANDLE_MOE_OK;
    for (auto& r : recs) {
        float ms = 0.0f;
        if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
            rc = CANDLE_MOE_ERR_HIP;
        else if (r.slot < nslots) {
            if (total_ms) total_ms[r.slot] += ms;
            if (counts) counts[r.slot] += 1;
        }
    }
    std::lock_guard<std::mutex> lk(cm::g_prof_mu);
    for (auto& r : recs) {
        cm::g_event_pool.push_back(r.a);
        cm::g_event_pool.push_back(r.b);
    }
    return rc;
}

const char* candle_moe_profile_slot_name(int slot) {
    return (slot >= 0 && slot < cm::kNumSlots) ? cm::kSlotNames[slot] : "";
}

const char* candle_moe_version(void) { return "candle-moe-hip 0.1.0 (gfx950)"; }

}  // extern "C"
