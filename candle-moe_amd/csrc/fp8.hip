// FP8 expert weights: OCP e4m3 (E4M3FN: bias 7, 3 mantissa bits, no
// infinities, 0x7F / 0xFF NaN, largest finite 448) with one f32 scale per
// output channel, stored K-contiguous, [E][N][K] bytes and [E][N] scales,
// for the fp8-weight decode GEMMs (launch_moe_gemm_w8).
//
//   scale[e][n] = max_k |w[e][k][n]| / 448    (1 when the channel is all zeros)
//   q[e][n][k]  = e4m3(w[e][k][n] / scale[e][n])   (round to nearest, ties to even)
//   w ~ decode(q) * scale
//
// The rounding is written out in exact f32 steps (no conversion instruction
// whose saturation or NaN rules would need pinning): the CPU oracle restates
// it operation for operation. Decoding uses v_cvt_pk_f32_fp8, checked against
// the format's definition for all 256 codes by the tests.
#include "cm_common.hpp"
#include "cm_internal.hpp"

namespace cm {

// e4m3 code of a finite f32 (|x| >= 448 saturates to +-448; NaN -> 0x7F).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t sign = (bits >> 24) & 0x80u;
    const float a = __uint_as_float(bits & 0x7fffffffu);
    if (!(a == a)) return 0x7fu;
    if (a >= 448.0f) return sign | 0x7eu;
    if (a < 0.015625f) {  // below 2^-6: subnormal codes m * 2^-9 (m = 8 is 2^-6, code 0x08)
        return sign | (uint32_t)__builtin_rintf(a * 512.0f);
    }
    int e = (int)((__float_as_uint(a) >> 23) & 0xffu) - 127;          // 2^e <= a < 2^(e+1), e in [-6, 8]
    const float m = __uint_as_float((__float_as_uint(a) & 0x7fffffu) | 0x3f800000u);  // a / 2^e, exact
    uint32_t q = (uint32_t)__builtin_rintf((m - 1.0f) * 8.0f);        // exact steps, one rounding
    if (q == 8u) {
        q = 0u;
        ++e;
    }
    return sign | ((uint32_t)(e + 7) << 3) | q;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)(code & 0xffu), false);
    return v[0];
}

// One workgroup per (expert, 64 output channels): the channels' largest
// magnitudes over K (4 K ranges per channel, combined in LDS), then the codes.
// kn: the input is [E][K][N] (else [E][N][K]); the output is always [E][N][K].
template <int DT>
__global__ __launch_bounds__(256) void quantize_fp8_kernel(const void* __restrict__ w, int K, int N, int kn,
                                                           uint8_t* __restrict__ q, float* __restrict__ scales) {
    typedef typename Elem<DT>::storage S;
    __shared__ float s_amax[4][64];
    const int e = blockIdx.y;
    const int nl = threadIdx.x & 63, part = threadIdx.x >> 6;
    const int n = blockIdx.x * 64 + nl;
    const S* W = reinterpret_cast<const S*>(w) + (long long)e * K * N;
    auto at = [&](int k) -> float {
        return Elem<DT>::to_f32(kn ? W[(long long)k * N + n] : W[(long long)n * K + k]);
    };
    float amax = 0.0f;
    if (n < N)
        for (int k = part; k < K; k += 4) amax = fmaxf(amax, fabsf(at(k)));
    s_amax[part][nl] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_amax[0][nl], s_amax[1][nl]), fmaxf(s_amax[2][nl], s_amax[3][nl]));
    if (n >= N) return;
    const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (part == 0) scales[(long long)e * N + n] = sc;
    uint8_t* Q = q + ((long long)e * N + n) * K;
    for (int k = part; k < K; k += 4) Q[k] = (uint8_t)f32_to_e4m3(at(k) / sc);
}

// out[e][n][k] = dtype(decode(q[e][n][k]) * scale[e][n])
template <int DT>
__global__ __launch_bounds__(256) void dequantize_fp8_kernel(const uint8_t* __restrict__ q,
                                                             const float* __restrict__ scales, long long total, int K,
                                                             typename Elem<DT>::storage* __restrict__ out) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const float v = e4m3_to_f32(q[i]) * scales[i / K];
        out[i] = Elem<DT>::from_f32(v);
    }
}

hipError_t launch_quantize_fp8(const void* w, int dtype, int E, int K, int N, int kn, uint8_t* q, float* scales,
                               hipStream_t stream) {
    if (E <= 0 || K <= 0 || N <= 0) return hipSuccess;
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)E), block(256);
    if (dtype == kBF16) hipLaunchKernelGGL(quantize_fp8_kernel<kBF16>, grid, block, 0, stream, w, K, N, kn, q, scales);
    else if (dtype == kF16) hipLaunchKernelGGL(quantize_fp8_kernel<kF16>, grid, block, 0, stream, w, K, N, kn, q, scales);
    else if (dtype == kF32) hipLaunchKernelGGL(quantize_fp8_kernel<kF32>, grid, block, 0, stream, w, K, N, kn, q, scales);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_dequantize_fp8(const uint8_t* q, const float* scales, int E, int N, int K, void* out, int dtype,
                                 hipStream_t stream) {
    const long long total = (long long)E * N * K;
    if (total <= 0) return hipSuccess;
    long long g = (total + 255) / 256;
    if (g > 65536) g = 65536;
    const dim3 grid((unsigned)g), block(256);
    if (dtype == kBF16)
        hipLaunchKernelGGL(dequantize_fp8_kernel<kBF16>, grid, block, 0, stream, q, scales, total, K,
                           reinterpret_cast<uint16_t*>(out));
    else if (dtype == kF16)
        hipLaunchKernelGGL(dequantize_fp8_kernel<kF16>, grid, block, 0, stream, q, scales, total, K,
                           reinterpret_cast<uint16_t*>(out));
    else if (dtype == kF32)
        hipLaunchKernelGGL(dequantize_fp8_kernel<kF32>, grid, block, 0, stream, q, scales, total, K,
                           reinterpret_cast<float*>(out));
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// 16-bit weights [E][K][N] -> [E][N][K]: 64 x 64 tiles through LDS, read
// along N, written along K (rows of the padded tile 66 values apart, so the
// column reads of the write pass spread over the banks).
__global__ __launch_bounds__(256) void pack_kn_k(const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int K,
                                                 int N) {
    __shared__ uint16_t t[64][66];
    const long long e = blockIdx.z;
    const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const uint16_t* src = w + e * K * (long long)N;
    uint16_t* dst = out + e * N * (long long)K;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int r = i >> 6, c = i & 63;
        const int k = k0 + r, n = n0 + c;
        t[r][c] = (k < K && n < N) ? src[(long long)k * N + n] : (uint16_t)0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int r = i >> 6, c = i & 63;
        const int n = n0 + r, k = k0 + c;
        if (n < N && k < K) dst[(long long)n * K + k] = t[c][r];
    }
}

hipError_t launch_pack_kn(const void* w, int E, int K, int N, void* out, hipStream_t stream) {
    if (E <= 0 || K <= 0 || N <= 0) return hipSuccess;
    const long long gy = (K + 63) / 64;
    if (gy > 65535 || E > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pack_kn_k, dim3((N + 63) / 64, (unsigned)gy, E), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t*>(w), reinterpret_cast<uint16_t*>(out), K, N);
    return hipGetLastError();
}

}  // namespace cm
