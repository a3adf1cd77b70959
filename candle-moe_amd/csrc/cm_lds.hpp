// Device helpers of the LDS-DMA grouped GEMMs (moe_gemm_lds.hip): buffer
// resources, global->LDS DMA, explicit waits,
// LDS swizzles, XCD-aware tile order and the per-tile epilogues.
#pragma once

#include <type_traits>

#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {
namespace lds {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
#define CM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

constexpr uint32_t kOob = 0x80000000u;  // buffer offset past every resource (operands are < 2 GiB)

// Buffer resource (V#) of a raw byte range: base, stride 0, num_records =
// bytes, dword3 0x00020000 (gfx9 data format); loads past num_records
// return zeros. Made wave-uniform so it lives in SGPRs.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, long long bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)b);
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((b >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane((int32_t)bytes);
    r[3] = 0x00020000;
    return r;
}

// One wave instruction: 64 lanes x 16 bytes from the buffer into LDS at
// lds_off + 16*lane. Issued as inline asm so that the compiler neither waits
// for it before unrelated LDS reads nor tracks it: stage hand-over is done
// with the explicit s_waitcnt / s_barrier below.
__device__ __forceinline__ void dma16(const i32x4& r, uint32_t lds_off, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_off), "v"(voff), "s"(r)
                 : "memory");
}
// Same with a wave-uniform byte offset in an SGPR (address = base + voff +
// soff). Used only where base + voff + soff stays inside the operand for
// every lane whose voff is in range.
__device__ __forceinline__ void dma16s(const i32x4& r, uint32_t lds_off, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_off), "v"(voff), "s"(r), "s"(soff)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
// Wait for the DMA of the stage that has `newer` stages (of LOADS
// instructions each) issued after it; at most MAXN of them can be.
template <int LOADS, int MAXN>
__device__ __forceinline__ void wait_stage(int newer) {
    if constexpr (MAXN <= 0) {
        wait_vm<0>();
    } else {
        if (newer >= MAXN) wait_vm<MAXN * LOADS>();
        else wait_stage<LOADS, MAXN - 1>(newer);
    }
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" : : : "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)(p));
}

// Rows of K-contiguous tiles (A, [N,K] weights) hold ACH 16-byte chunks
// (ACH = BK / 8); chunk c of row r is stored at a_swz(r, c). 16 lanes of a
// ds_read_b128 read 16 consecutive rows at one logical chunk and land in 16
// distinct bank groups.
template <int ACH>
__device__ __forceinline__ int a_swz(int r, int c) {
    if constexpr (ACH == 8) return (c ^ r ^ (r >> 3)) & 7;
    else return (c ^ (r >> 2)) & 3;
}

// [K,N] sub-tile rows of BCH 16-byte chunks: chunk c of k-row r is stored at
// kn_swz(r, c). A transposed read touches 4 consecutive rows x 4 consecutive
// chunks (c multiple of 4 first) per 32 lanes; the xor sends them to 16
// distinct bank groups (rows are 256 B apart for BCH >= 16, 128 B for 8).
template <int BCH>
__device__ __forceinline__ int kn_swz(int r, int c) {
    if constexpr (BCH >= 16) return c ^ ((r & 3) << 2);
    else return c ^ (((r >> 1) & 1) << 2);
}


// Clear this workgroup's share of n floats at p (16-byte stores where p is
// 16-byte aligned, which the workspace guarantees).
__device__ __forceinline__ void clear_share(float* p, long long n) {
    if (!p || n <= 0) return;
    const long long per = ((n + gridDim.x - 1) / gridDim.x + 3) & ~3LL;
    const long long lo = (long long)blockIdx.x * per;
    const long long hi = lo + per < n ? lo + per : n;
    for (long long i = lo + 4LL * threadIdx.x; i < hi; i += 4LL * blockDim.x) {
        if (i + 4 <= hi) {
            *reinterpret_cast<f32x4*>(p + i) = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            for (long long j = i; j < hi; ++j) p[j] = 0.f;
        }
    }
}

// Two ds_read_b64_tr_b16 results (k rows kr..kr+3 and kr+4..kr+7 of one
// column) as the 8-value MFMA operand.
__device__ __forceinline__ u32x4 tr_pair(const char* p_lo, const char* p_hi) {
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(CM_LDS(p_lo)));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(CM_LDS(p_hi)));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
    const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
    u32x4 v;
    v[0] = l2[0];
    v[1] = l2[1];
    v[2] = h2[0];
    v[3] = h2[1];
    return v;
}

// Eight OCP fp8 e4m3 values (bytes of v, lowest first) as the MFMA operand of
// the activation dtype, exactly (every e4m3 value is a bf16 and an f16): the
// gfx950 scaled conversion with scale 1 turns the two bytes of one 16-bit
// word into a DT pair, low byte in the low half (one instruction per pair
// instead of an f32 decode and a packing conversion).
template <int DT>
__device__ __forceinline__ u32x4 fp8x8_to(const u32x2& v) {
    u32x4 r;
    if constexpr (DT == kBF16) {
        r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.0f, false));
        r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.0f, true));
        r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.0f, false));
        r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.0f, true));
    } else {
        r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[0], 1.0f, false));
        r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[0], 1.0f, true));
        r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[1], 1.0f, false));
        r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v[1], 1.0f, true));
    }
    return r;
}

// Split-K fixup. Every split writes its f32 partial tile to partial slot
// slot0 + ks (per wave, per 32x32 block, 4 registers of a lane as one 16-byte
// chunk, lanes contiguous), then counts itself in a.counters[ctr]; the split
// that arrives last sums all partials in split order (so the result does not
// depend on which split finished last), resets the counter and returns true
// (it runs the epilogue, once per tile), the others return false. The splits
// may run on different XCDs, whose L2s are not coherent with each other. The
// ordering is the memory model's: every thread's partial stores precede the
// workgroup barrier, which precedes thread 0's release increment at agent
// scope; the last split's increment reads every earlier one (one release
// sequence), and its acquire fence (the last split only: an acquire
// invalidates the XCD's L2 under every other workgroup there) precedes its
// partial loads, which follow after a second barrier.
// The partials are also written and read with device-coherent buffer
// accesses (cache policy sc1: written through to, and read from, the level
// shared by all XCDs). The accesses are compiler builtins, not inline asm:
// the stores read MFMA results, whose read-after-write hazards only the
// compiler knows to pad.
constexpr int kCachePolicyDevice = 16;  // CPol::SC1

// PAIRED: the partials of two splits are loaded per round (the 32-row
// kernels, whose fixup is a chain of round trips at decode sizes).
template <int MB, int NB, int NW, int BATCH, bool PAIRED = false>
__device__ __forceinline__ bool splitk_fixup(const GemmArgs& a, f32x16 (&acc)[MB][NB], int slot0, int ctr, int ks,
                                             int nsplit, int wave, int lane) {
    __shared__ int s_last;
    constexpr int PER_WAVE = MB * NB * 16 * 64;
    constexpr int PER = NW * PER_WAVE;  // floats per workgroup partial (BM * BN)
    constexpr int NQ = MB * NB * 4;     // 16-byte chunks per lane
    static_assert(NQ % BATCH == 0, "fixup batch");
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, 0x7ffffff0, 0x00020000);
    const uint32_t lane_off = (uint32_t)(wave * PER_WAVE) * 4u + (uint32_t)lane * 16u;
    const uint32_t mine = (uint32_t)(slot0 + ks) * (uint32_t)PER * 4u + lane_off;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const f32x16& r = acc[(q >> 2) / NB][(q >> 2) % NB];
        const int i = 4 * (q & 3);
        const u32x4 v = {__float_as_uint(r[i]), __float_as_uint(r[i + 1]), __float_as_uint(r[i + 2]),
                         __float_as_uint(r[i + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(v, pr, mine + q * 1024, 0, kCachePolicyDevice);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        s_last = __hip_atomic_fetch_add(a.counters + ctr, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
        if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!s_last) return false;
    // split 0 replaces the registers, the others add in split order
    auto gather = [&](int s2, auto first) {
        const uint32_t src = (uint32_t)(slot0 + s2) * (uint32_t)PER * 4u + lane_off;
#pragma unroll
        for (int q0 = 0; q0 < NQ; q0 += BATCH) {
            u32x4 v[BATCH];
#pragma unroll
            for (int b = 0; b < BATCH; ++b)
                v[b] = __builtin_amdgcn_raw_buffer_load_b128(pr, src + (q0 + b) * 1024, 0, kCachePolicyDevice);
#pragma unroll
            for (int b = 0; b < BATCH; ++b) {
                const int q = q0 + b;
                f32x16& r = acc[(q >> 2) / NB][(q >> 2) % NB];
                const int i = 4 * (q & 3);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float x = __uint_as_float(v[b][j]);
                    if constexpr (decltype(first)::value) r[i + j] = x;
                    else r[i + j] += x;
                }
            }
        }
    };
    if constexpr (PAIRED) {
        // splits s2 and s2 + 1 in flight together, summed in split order
        auto gather2 = [&](int s2, auto first) {
            const uint32_t src0 = (uint32_t)(slot0 + s2) * (uint32_t)PER * 4u + lane_off;
            const uint32_t src1 = src0 + (uint32_t)PER * 4u;
            const bool two = s2 + 1 < nsplit;
            u32x4 v0[NQ], v1[NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q) v0[q] = __builtin_amdgcn_raw_buffer_load_b128(pr, src0 + q * 1024, 0, kCachePolicyDevice);
            if (two) {
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    v1[q] = __builtin_amdgcn_raw_buffer_load_b128(pr, src1 + q * 1024, 0, kCachePolicyDevice);
            }
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                f32x16& r = acc[(q >> 2) / NB][(q >> 2) % NB];
                const int i = 4 * (q & 3);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float x = __uint_as_float(v0[q][j]);
                    if constexpr (decltype(first)::value) r[i + j] = x;
                    else r[i + j] += x;
                    if (two) r[i + j] += __uint_as_float(v1[q][j]);
                }
            }
        };
        gather2(0, std::true_type{});
        for (int s2 = 2; s2 < nsplit; s2 += 2) gather2(s2, std::false_type{});
    } else {
        gather(0, std::true_type{});
        for (int s2 = 1; s2 < nsplit; ++s2) gather(s2, std::false_type{});
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.counters + ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Work item of this workgroup under tail balance (GemmArgs::tail_cus = C > 0).
// XCD x takes a contiguous range of nx of the `live` tiles, as xcd_logical;
// its first nx - R (R = nx mod C) tiles run whole, in nx / C full rounds over
// the XCD's C CUs. The R tiles of the last round are split along K into
// S = min(C / R, 8, K tiles / 8) parts when R <= C / 2, so that R * S workgroups
// share that round instead of R. Split j of tail tile t of XCD x uses partial
// slot x*C + t*S + j and counter x*C + t. Returns false for a workgroup
// without work.
__device__ __forceinline__ bool tail_item(int live, int C, int nk_all, int& tile, int& ks, int& nsplit, int& slot0,
                                          int& ctr) {
    live = min(live, (int)gridDim.x);
    const int w = blockIdx.x, xcd = w & 7, idx = w >> 3;
    const int per = live >> 3, rem = live & 7;
    const int nx = per + (xcd < rem ? 1 : 0);
    const int base = xcd * per + (xcd < rem ? xcd : rem);
    const int R = nx % C, full = nx - R;
    int S = 1;
    if (R > 0 && 2 * R <= C) S = min(min(C / R, kTailMaxSplit), nk_all / kTailMinKTiles);
    ks = 0;
    nsplit = 1;
    slot0 = ctr = 0;
    if (S <= 1) {
        if (idx >= nx) return false;
        tile = base + idx;
        return true;
    }
    if (idx < full) {
        tile = base + idx;
        return true;
    }
    const int j = idx - full;
    if (j >= R * S) return false;
    const int t = j / S;
    tile = base + full + t;
    ks = j - t * S;
    nsplit = S;
    ctr = xcd * C + t;
    slot0 = xcd * C + t * S;
    return true;
}

// Expert ids of the k slots of an expert-set key (base n_experts+1 digits,
// most significant first) and the number of valid ones.
__device__ __forceinline__ int decode_set(int key, int k_top, int n_experts, int (&seg_exp)[kSetMaxK]) {
    const int base = n_experts + 1;
    for (int s = k_top - 1; s >= 0; --s) {
        seg_exp[s] = key % base;
        key /= base;
    }
    int n = 0;
    for (int s = 0; s < k_top; ++s) n += seg_exp[s] < n_experts;
    return n;
}

// ------------------------------------------------------------------ epilogues
// One wave's MB x NB blocks of 32x32 accumulators, the wave's sub-tile at
// rows wm*WM, columns wn*WN of a BM x BN block tile (row tile r0, column
// tile nt). Non-atomic modes were computed with swapped MFMA operands, so
// lane l holds row l%32 and, in register group g = i/4, the 4 consecutive
// columns 8g + 4(l/32) .. +3 of each 32-column block. Atomic modes were not
// swapped: register i of lane l is row 8(i/4) + 4(l/32) + i%4, column l%32
// (32 consecutive columns per atomic instruction).
//  kGateUp / kFc1 : inter[dst] = dtype(w? * act(gate) (* up)), dst = pair_dest[p] or the sorted row
//  kDownSet/kFc2Set: out[tok] = dtype(out[tok] + acc), or dtype(acc) with overwrite
//                   (each output row is owned by one tile)
//  kDown / kFc2   : acc_f32[tok] += w * acc            (f32 atomics)
//  kDownRows / kFc2Rows: rows[p] = dtype(w * acc)      (the pair's own row)
// sc0 / sc1 (fp8 weights, else null): per-output-column scales of the
// tile's expert (gate / up for kGateUp), indexed from the tile's first column
// (nt * BN, or nt * BN/2 for kGateUp), applied to the f32 sums first.
template <int DT, int MODE, int BN, int WM, int WN, int MB, int NB>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, f32x16 (&acc)[MB][NB], int r0, int m_valid, int nt,
                                              int wm, int wn, int lane, const int32_t* s_tok, const float* s_w,
                                              const int* pre_dst = nullptr, const float* pre_w = nullptr,
                                              const float* sc0 = nullptr, const float* sc1 = nullptr) {
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool ATOMIC = (MODE == kDown || MODE == kFc2);
    const int N = a.N;
    const int lr = lane & 31, lh = lane >> 5;
    if constexpr (ATOMIC) {
        float* C = reinterpret_cast<float*>(a.C);
        float cs[NB];  // this lane's column scale per block
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int col = nt * BN + wn * WN + nb * 32 + lr;
            cs[nb] = sc0 ? sc0[col - nt * BN] : 1.0f;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ml = wm * WM + mb * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
                if (ml >= m_valid) continue;
                const long long rowoff = (long long)s_tok[ml] * N;
                const float w = s_w[ml];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int col = nt * BN + wn * WN + nb * 32 + lr;
                    if (col < N) unsafeAtomicAdd(C + rowoff + col, w * (cs[nb] * acc[mb][nb][i]));
                }
            }
        }
    } else {
        const int nsub = 4 * lh;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = wm * WM + mb * 32 + lr;
            if (ml >= m_valid) continue;
            const int r = r0 + ml;
            if constexpr (MODE == kGateUp || MODE == kFc1) {
                int dst;
                float wscale;
                if (pre_dst) {
                    dst = pre_dst[mb];
                    wscale = pre_w[mb];
                } else {
                    const int p = a.sorted_pair[r];
                    dst = a.pair_dest ? a.pair_dest[p] : r;
                    wscale = a.fold_w ? a.routing_w[p] : 1.0f;
                }
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
                                // (fp8 weights: the column scales first)
                                const int cj = col + j - (DUAL ? nt * (BN / 2) : nt * BN);
                                const float s0 = sc0 ? sc0[cj] : 1.0f;
                                if constexpr (DUAL) {
                                    const float s1 = sc1 ? sc1[cj] : 1.0f;
                                    h[j] = act_t<ACT>(s0 * acc[mb][2 * q][4 * g + j]) * (s1 * acc[mb][2 * q + 1][4 * g + j]);
                                } else {
                                    h[j] = act_t<ACT>(s0 * acc[mb][q][4 * g + j]);
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
            } else if constexpr (MODE == kDownRows || MODE == kFc2Rows) {
                // the pair's own row: rows[p] = dtype(w_p * acc)
                const int p = pre_dst ? pre_dst[mb] : a.sorted_pair[r];
                const float wscale = pre_w ? pre_w[mb] : a.routing_w[p];
                uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + (long long)p * N;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int colbase = nt * BN + wn * WN + nb * 32;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = colbase + 8 * g + nsub;
                        if (col >= N) continue;
                        u32x2 v;
                        v[0] = pack2<DT>(wscale * acc[mb][nb][4 * g + 0], wscale * acc[mb][nb][4 * g + 1]);
                        v[1] = pack2<DT>(wscale * acc[mb][nb][4 * g + 2], wscale * acc[mb][nb][4 * g + 3]);
                        *reinterpret_cast<u32x2*>(C + col) = v;
                    }
                }
            } else {
                // (moe_lds_gemm stages the tile's tokens in s_tok)
                const int tok = pre_dst ? pre_dst[mb] : (s_tok ? s_tok[ml] : a.tok_sorted[r]);
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

// Epilogue through LDS for the large-tile kernels (gate/up, fc1, expert-set
// down / fc2 with overwrite, pair-row down / fc2). In the swapped MFMA layout
// a lane holds 4-column pieces of one tile row, so direct stores put 16
// bytes into each of 32 rows per instruction. Instead: (1) every wave writes
// its finished values, converted to DT, into a [BM][W] tile in the stage
// buffers (row-major, 16-byte chunk c of row r at c ^ (r % CPR), so that the
// 32 rows of a write and the chunks of a row read land in distinct banks);
// (2) the waves store whole rows, 16 bytes per lane, CPR lanes per row.
// dst_rows[r]: output row of tile row r; rows >= m_valid are not stored.
// SC (fp8 weights): the f32 sums are first scaled by the tile's column
// scales sc0 (gate/up: gate's, sc1 up's), indexed by the output column in
// the tile.
template <int DT, int MODE, int BM, int BN, int WM, int WN, int MB, int NB, int NW, bool SC = false>
__device__ __forceinline__ void staged_epilogue(const GemmArgs& a, f32x16 (&acc)[MB][NB], char* tile_lds,
                                                const int32_t* dst_rows, int m_valid, int nt, int wm, int wn,
                                                int lane, const float* pre_w, const float* sc0 = nullptr,
                                                const float* sc1 = nullptr) {
    constexpr bool DUAL = (MODE == kGateUp);
    constexpr bool GATHER = (MODE == kGateUp || MODE == kFc1);
    constexpr bool ROWS = (MODE == kDownRows || MODE == kFc2Rows);
    constexpr int W = DUAL ? BN / 2 : BN;  // output columns of the tile
    constexpr int CPR = W / 8;             // 16-byte chunks per row
    constexpr int RB = W * 2;              // bytes per row
    static_assert(CPR == 8 || CPR == 16 || CPR == 32, "row chunks");
    const int N = a.N;
    const int lr = lane & 31, nsub = 4 * (lane >> 5);
    auto put = [&](int ml, int lc, float h0, float h1, float h2, float h3) {
        u32x2 v;
        v[0] = pack2<DT>(h0, h1);
        v[1] = pack2<DT>(h2, h3);
        const int c = lc >> 3;
        *reinterpret_cast<u32x2*>(tile_lds + ml * RB + ((c ^ (ml % CPR)) << 4) + (lc & 7) * 2) = v;
    };
    // (1) values into LDS
    if constexpr (GATHER) {
        with_act(a.act, [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int ml = wm * WM + mb * 32 + lr;
                const float ws = pre_w[mb];
                constexpr int PAIRS = DUAL ? NB / 2 : NB;
#pragma unroll
                for (int q = 0; q < PAIRS; ++q) {
                    const int lbase = DUAL ? ((wn * WN) / 64 + q) * 32 : wn * WN + q * 32;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        float h[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            float gv = DUAL ? acc[mb][2 * q][4 * g + j] : acc[mb][q][4 * g + j];
                            float uv = DUAL ? acc[mb][2 * q + 1][4 * g + j] : 1.0f;
                            if constexpr (SC) {
                                const int lc = lbase + 8 * g + nsub + j;  // output column in the tile
                                gv *= sc0[lc];
                                if constexpr (DUAL) uv *= sc1[lc];
                            }
                            if constexpr (DUAL)
                                h[j] = act_t<ACT>(gv) * uv;
                            else
                                h[j] = act_t<ACT>(gv);
                            h[j] *= ws;
                        }
                        put(ml, lbase + 8 * g + nsub, h[0], h[1], h[2], h[3]);
                    }
                }
            }
        });
    } else {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int ml = wm * WM + mb * 32 + lr;
            const float ws = ROWS ? pre_w[mb] : 1.0f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int i = 4 * g;
                    const int lc = wn * WN + nb * 32 + 8 * g + nsub;
                    float c0 = ws, c1 = ws, c2 = ws, c3 = ws;
                    if constexpr (SC) {
                        c0 *= sc0[lc];
                        c1 *= sc0[lc + 1];
                        c2 *= sc0[lc + 2];
                        c3 *= sc0[lc + 3];
                    }
                    put(ml, lc, c0 * acc[mb][nb][i], c1 * acc[mb][nb][i + 1], c2 * acc[mb][nb][i + 2],
                        c3 * acc[mb][nb][i + 3]);
                }
            }
        }
    }
    __syncthreads();
    // (2) whole rows out
    constexpr int RPI = 64 / CPR;  // rows per wave instruction
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane % CPR;
    const int col = nt * W + c * 8;
    uint16_t* C = reinterpret_cast<uint16_t*>(a.C);
    if (col < N) {
        for (int r = wave * RPI + lane / CPR; r < m_valid; r += NW * RPI) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(tile_lds + r * RB + ((c ^ (r % CPR)) << 4));
            *reinterpret_cast<u32x4*>(C + (long long)dst_rows[r] * N + col) = v;
        }
    }
}

// Expert-set down / fc2 in accumulate mode (out = dtype(out + acc), one
// rounding from f32): as staged_epilogue, but the tile goes through LDS in
// f32, half of its columns at a time (BM x BN/2 x 4 bytes fit the stages),
// and each row store first reads the row's old values (16 bytes per lane).
template <int DT, int BM, int BN, int WM, int WN, int MB, int NB, int NW>
__device__ __forceinline__ void staged_epilogue_acc(const GemmArgs& a, f32x16 (&acc)[MB][NB], char* tile_lds,
                                                    const int32_t* dst_rows, int m_valid, int nt, int wm, int wn,
                                                    int lane) {
    constexpr int HW = BN / 2;     // columns per half
    constexpr int CPR = HW / 4;    // 16-byte (4 x f32) chunks per LDS row
    constexpr int RB = HW * 4;     // bytes per LDS row
    static_assert(CPR == 32, "half-tile rows");
    static_assert(WN <= HW && HW % WN == 0, "a wave's columns lie in one half");
    const int N = a.N;
    const int lr = lane & 31, nsub = 4 * (lane >> 5);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint16_t* C = reinterpret_cast<uint16_t*>(a.C);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (h) __syncthreads();  // the first half's rows are stored
        // (1) the waves whose columns lie in this half write them, f32
        if ((wn * WN) / HW == h) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int ml = wm * WM + mb * 32 + lr;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int lc = wn * WN - h * HW + nb * 32 + 8 * g + nsub;  // column in the half
                        const int c = lc >> 2;
                        u32x4 v;
#pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] = __float_as_uint(acc[mb][nb][4 * g + j]);
                        *reinterpret_cast<u32x4*>(tile_lds + ml * RB + ((c ^ (ml % CPR)) << 4)) = v;
                    }
                }
            }
        }
        __syncthreads();
        // (2) rows: 16 lanes per row, 8 columns (two LDS chunks) per lane
        const int c8 = lane & 15;
        const int col = nt * BN + h * HW + c8 * 8;
        if (col < N) {
            for (int r = wave * 4 + (lane >> 4); r < m_valid; r += NW * 4) {
                const u32x4 lo = *reinterpret_cast<const u32x4*>(tile_lds + r * RB + (((2 * c8) ^ (r % CPR)) << 4));
                const u32x4 hi = *reinterpret_cast<const u32x4*>(tile_lds + r * RB + (((2 * c8 + 1) ^ (r % CPR)) << 4));
                uint16_t* dst = C + (long long)dst_rows[r] * N + col;
                const u32x4 old = *reinterpret_cast<const u32x4*>(dst);
                u32x4 v;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t o = old[q];
                    const float x0 = Elem<DT>::to_f32((uint16_t)(o & 0xffffu)) + __uint_as_float(q < 2 ? lo[2 * q] : hi[2 * q - 4]);
                    const float x1 = Elem<DT>::to_f32((uint16_t)(o >> 16)) + __uint_as_float(q < 2 ? lo[2 * q + 1] : hi[2 * q - 3]);
                    v[q] = pack2<DT>(x0, x1);
                }
                *reinterpret_cast<u32x4*>(dst) = v;
            }
        }
    }
}

}  // namespace lds
}  // namespace cm
