// Shared device/host helpers for the gfx950 camera-path library.
//
// Numeric contract: activations and weights enter the matrix cores as bf16,
// products accumulate in fp32 (v_mfma_f32_16x16x32_bf16); LayerNorm, softmax,
// GELU, BN-folded bias and residual adds stay fp32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

namespace bfhip {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- host errors
inline int fail(char *error, size_t cap, const char *fmt, ...) {
    if (error && cap) {
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(error, cap, fmt, ap);
        va_end(ap);
    }
    return 0;
}

inline int hip_ok(hipError_t s, char *error, size_t cap, const char *what) {
    return s == hipSuccess ? 1 : fail(error, cap, "%s: %s", what, hipGetErrorString(s));
}

inline int launch_ok(char *error, size_t cap, const char *what) {
    return hip_ok(hipGetLastError(), error, cap, what);
}

// ------------------------------------------------------------- device numeric
__device__ __forceinline__ bf16 to_bf16(float v) { return static_cast<bf16>(v); }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }

// One 16x16x32 bf16 MFMA: acc[16x16] += A[16x32] * B[32x16].
// Lane l holds A row (l & 15), k = 8*(l >> 4) .. +7; B column (l & 15), same
// k; C column (l & 15), rows 4*(l >> 4) .. +3.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

// Exact-erf GELU 0.5*x*(1 + erf(x/sqrt(2))) with erf from Abramowitz & Stegun,
// Handbook of Mathematical Functions, formula 7.1.26 (|error| <= 1.5e-7 for
// all x; odd symmetry for x < 0): one reciprocal, one exp2 and five FMAs
// instead of a full-precision erff, well inside the bf16 rounding of the
// output it feeds.
__device__ __forceinline__ float gelu_erf(float x) {
    const float z = fabsf(x) * 0.7071067811865475244f;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));  // v_rcp_f32, 1 ulp
    float poly = fmaf(1.061405429f, t, -1.453152027f);
    poly = fmaf(poly, t, 1.421413741f);
    poly = fmaf(poly, t, -0.284496736f);
    poly = fmaf(poly, t, 0.254829592f);
    poly *= t;
    // v_exp_f32 directly: an argument below -126 flushes to 0, where erf is 1.
    const float e = __builtin_amdgcn_exp2f(-z * z * 1.4426950408889634f);
    const float erf_abs = fmaf(-poly, e, 1.0f);
    const float erf_x = x < 0.0f ? -erf_abs : erf_abs;
    return 0.5f * x * (1.0f + erf_x);
}

// Rows of the same LayerNorm live in a power-of-two group of lanes.
template <int Lanes>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = Lanes / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, Lanes);
    return v;
}

template <int Lanes>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = Lanes / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, Lanes));
    return v;
}

// Map a linear workgroup id so that consecutive logical tiles stay on one XCD
// (workgroups are dealt round-robin over the 8 XCDs; each XCD owns an L2).
__device__ __forceinline__ int xcd_swizzle(int pid, int count) {
    constexpr int kXcd = 8;
    if (count < kXcd * 2) return pid;
    const int per = count / kXcd, extra = count % kXcd;
    const int xcd = pid % kXcd, local = pid / kXcd;
    // The first `extra` XCDs receive per+1 tiles.
    const int base = xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per;
    return base + local;
}

}  // namespace bfhip
