// Shared device helpers for the gfx950 fused-MoE kernels: storage types,
// conversions, activations, wave64 cross-lane reductions and MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace cm {

// dtype codes of the C ABI (/root/reference/src/lib.rs:174-182)
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };
// activation codes (/root/reference/src/lib.rs:164-171)
enum Act : int { kSilu = 0, kGelu = 1, kRelu = 2 };
// moe_type codes (/root/reference/src/ffi.rs:42)
enum MoeType : int { kQwen3 = 0, kNomic = 1 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-bit storage element tags. Global memory holds raw bits (uint16_t).
struct bf16_t { uint16_t v; };
struct f16_t { uint16_t v; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)x;
}
// Round to nearest even (gfx950 lowers the bf16 truncation to v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    __bf16 b = (__bf16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
// Two f32 values rounded to nearest even and packed, a in the low half: one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 for the pair.
template <int DT> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {a, b};
    if constexpr (DT == kBF16) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    } else {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
}

template <int DT> struct Elem;
template <> struct Elem<kBF16> {
    typedef uint16_t storage;
    static __device__ __forceinline__ float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
    static __device__ __forceinline__ uint16_t from_f32(float f) { return (uint16_t)f32_to_bf16_bits(f); }
};
template <> struct Elem<kF16> {
    typedef uint16_t storage;
    static __device__ __forceinline__ float to_f32(uint16_t v) { return f16_bits_to_f32(v); }
    static __device__ __forceinline__ uint16_t from_f32(float f) { return (uint16_t)f32_to_f16_bits(f); }
};
template <> struct Elem<kF32> {
    typedef float storage;
    static __device__ __forceinline__ float to_f32(float v) { return v; }
    static __device__ __forceinline__ float from_f32(float f) { return f; }
};

// Activations (/root/reference/kernels/common.cuh:116-138): SiLU x/(1+e^-x),
// tanh-approximation GELU, ReLU. Evaluated in f32 with the accurate
// library expf / tanhf (the reference build used approximate __expf).
__device__ __forceinline__ float act_f32(float x, int act) {
    if (act == kGelu) {
        const float c = 0.7978845608028654f;  // sqrt(2/pi)
        return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
    }
    if (act == kRelu) return fmaxf(x, 0.0f);
    return x / (1.0f + expf(-x));
}

// The same activations from the hardware base-2 exponential (v_exp_f32) and
// reciprocal (v_rcp_f32), a few f32 ulp from act_f32: used by the 16-bit
// MFMA epilogues, whose results are rounded to bf16 / f16 right after.
//   silu(x) = x * 1 / (1 + 2^(-x log2 e))
//   gelu(x) = x * 1 / (1 + 2^(-2 log2 e * sqrt(2/pi) (x + 0.044715 x^3)))
//             (0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)))
// For x -> -inf, 2^z overflows to +inf and v_rcp_f32(+inf) = 0, so the
// result goes to (-)0 as x / (1 + e^-x) does; x = -inf gives NaN in both.
template <int ACT> __device__ __forceinline__ float act_t(float x) {
    if constexpr (ACT == kRelu) {
        return fmaxf(x, 0.0f);
    } else {
        float z;
        if constexpr (ACT == kGelu) {
            const float k = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
            z = k * (x + 0.044715f * x * x * x);
        } else {
            z = -1.4426950408889634f * x;
        }
        return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
    }
}
__device__ __forceinline__ float act_fast(float x, int act) {
    if (act == kRelu) return act_t<kRelu>(x);
    if (act == kGelu) return act_t<kGelu>(x);
    return act_t<kSilu>(x);
}
// f(std::integral_constant<int, ACT>{}) for the runtime activation code, so
// that a loop over elements inside f is compiled once per activation with no
// per-element branch.
template <class F> __device__ __forceinline__ void with_act(int act, F&& f) {
    if (act == kGelu) {
        f(std::integral_constant<int, kGelu>{});
    } else if (act == kRelu) {
        f(std::integral_constant<int, kRelu>{});
    } else {
        f(std::integral_constant<int, kSilu>{});
    }
}

// ---------------------------------------------------------------------
// wave64 cross-lane exchange: lane L receives the value of lane L ^ m.
// m = 1, 2 : DPP quad_perm; m = 4, 8, 16 : ds_swizzle bitmask mode
// (and 0x1f, xor m; no LDS memory traffic); m = 32 : ds_bpermute.
// ---------------------------------------------------------------------
template <int M>
__device__ __forceinline__ int xor_lane_i32(int v) {
    if constexpr (M == 1) {
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4 || M == 8 || M == 16) {
        return __builtin_amdgcn_ds_swizzle(v, 0x1F | (M << 10));
    } else {
        const int lane = __lane_id();
        return __builtin_amdgcn_ds_bpermute((lane ^ M) << 2, v);
    }
}
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
    return __int_as_float(xor_lane_i32<M>(__float_as_int(v)));
}
template <int M>
__device__ __forceinline__ double xor_lane(double v) {
    const uint64_t u = __double_as_longlong(v);
    const int lo = xor_lane_i32<M>((int)(uint32_t)u);
    const int hi = xor_lane_i32<M>((int)(uint32_t)(u >> 32));
    return __longlong_as_double(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// ---------------------------------------------------------------------
// MFMA 32x32x16 (gfx950) for bf16 / f16 operands, f32 accumulate.
// Operand layout used throughout: lane l supplies 8 consecutive K values
// of row/column (l % 32), K-half (l / 32). Result lane l, register i holds
// element (row 8*(i/4) + 4*(l/32) + i%4, col l%32) of the 32x32 block.
// ---------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    if constexpr (DT == kBF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// Workgroup -> logical work item. The hardware hands workgroup w to XCD w % 8;
// this gives each XCD a contiguous range of the `live` items (neighbouring
// tiles then share that XCD's L2) and spreads the live items evenly over the
// 8 XCDs, however many spare workgroups a grid sized for the worst case holds.
// Returns -1 for a workgroup with no item.
__device__ __forceinline__ int xcd_logical(int live) {
    live = min(live, (int)gridDim.x);
    const int w = blockIdx.x, xcd = w & 7, idx = w >> 3;
    const int per = live >> 3, rem = live & 7;
    if (idx >= per + (xcd < rem ? 1 : 0)) return -1;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// K splits of a launch with `live` output tiles (known on the device only,
// from the grouping): target / live, target = workgroups that fill the
// device once, so live * splits <= target (one round of workgroups: the
// weight-streaming 32-row kernels gain nothing from a second); at most
// max_split, no empty split among nk K tiles. target <= 0: max_split as
// given (fixed by the host).
__device__ __forceinline__ int adaptive_split(int max_split, int target, int live, int nk) {
    if (max_split <= 1) return 1;
    if (target <= 0) return max_split;
    int sp = live > 0 ? target / live : max_split;
    sp = sp < 1 ? 1 : (sp > max_split ? max_split : sp);
    sp = sp < nk ? sp : (nk > 0 ? nk : 1);
    const int per = (nk + sp - 1) / sp;
    return per > 0 ? (nk + per - 1) / per : 1;
}

// Output tile (row tile mt, column tile nt) of this workgroup, or false when
// it has none: the row-tile count m_live comes from the grouping on the device.
__device__ __forceinline__ bool tile_coords(int n_tiles, int m_live, int& mt, int& nt) {
    const int logical = xcd_logical(m_live * n_tiles);
    if (logical < 0) return false;
    mt = logical / n_tiles;
    nt = logical - mt * n_tiles;
    return true;
}
__host__ __device__ __forceinline__ long long cdivll(long long a, long long b) { return (a + b - 1) / b; }

}  // namespace cm
