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

// 16-bit operands travel through the loaders, LDS and registers as raw
// 16-bit words typed bf16; a context that needs more mantissa than bf16's 8
// bits (a deep conv stack) stores fp16 words instead, and its tiles select
// the fp16 MFMA (same lane layout, same rate).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma16_f16(bf16x8 a, bf16x8 b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x4 mfma16_as(bf16x8 a, bf16x8 b, f32x4 acc) {
    if constexpr (F16) return mfma16_f16(a, b, acc);
    else return mfma16(a, b, acc);
}
// fp16 words (IEEE binary16, round to nearest even) in the bf16 container,
// rounded once from the fp32 value.  The empty asm keeps the compiler from
// folding the multiply or add that produced v into the conversion
// (v_fma_mix*_f16 rounds a*b+c straight to fp16): the folded and unfolded
// forms can differ by one fp16 ulp, and the compiler chooses per unrolled
// copy, so a row's result would depend on the tile slot it was computed in
// (the GEMM epilogues unroll over rows).
__device__ __forceinline__ bf16 to_half(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(bf16, static_cast<_Float16>(v));
}
__device__ __forceinline__ float half_to_f32(bf16 v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}
// A float stored as the 16-bit word of the chosen format.
__device__ __forceinline__ bf16 to_word(float v, bool f16) {
    return f16 ? to_half(v) : static_cast<bf16>(v);
}

// GELU 0.5*x*(1 + erf(x/sqrt(2))) (the reference's exact-erf form,
// kernels_ref.c:448-452) evaluated as x * sigmoid(x * p(x^2)), p a quartic in
// x^2 fitted (Lawson's iteratively reweighted least squares, i.e. minimax) to
// the exact-erf GELU over [-10, 10]: relative error where |GELU(x)| > 0.01,
// absolute error below that.  p < 0 for every x (its x^8 term dominates past
// the fitted range), so u = x*p(x^2) has the sign of -x and |u| grows without
// bound: 2^u saturates to 0 (GELU = x) or to +inf (GELU = x * 0 = -0) with no
// clamp; |u| >= 39 once |x| >= 6.  Evaluated in fp32 as below the absolute
// error is <= 9.1e-6 for every x, and the relative error <= 5.7e-5 wherever
// |GELU(x)| > 0.01: under a quarter of the half-ulp (2^-12) of the fp16 value
// it feeds.  Cost: 8 VALU + v_exp_f32 + v_rcp_f32 (vs 16 + 2 for a rational
// erf).  The constants carry the -log2(e) of sigmoid(u) = 1/(1 + 2^(-u log2 e)).
__device__ __forceinline__ float gelu(float x) {
    const float t = x * x;
    float p = fmaf(t, -2.720398243e-06f, 7.499327330e-05f);
    p = fmaf(t, p, 4.688421031e-04f);
    p = fmaf(t, p, -1.055332273e-01f);
    p = fmaf(t, p, -2.301823854e+00f);
    const float e = __builtin_amdgcn_exp2f(x * p);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
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
__host__ __device__ __forceinline__ int xcd_swizzle(int pid, int count) {
    constexpr int kXcd = 8;
    if (count < kXcd * 2) return pid;
    const int per = count / kXcd, extra = count % kXcd;
    const int xcd = pid % kXcd, local = pid / kXcd;
    // The first `extra` XCDs receive per+1 tiles.
    const int base = xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per;
    return base + local;
}

// Row-major tile index of workgroup `bid` when a tiles_m x tiles_n grid is
// dealt to the 8 XCDs as rectangular blocks: XCD x (the one that runs the
// workgroups with bid % 8 == x) owns the tiles of row group x / (8 / gm) and
// column group x % (8 / gm), so it fetches 1/gm of A's rows and gm/8 of B's
// columns instead of, for a grid of whole row panels, all of B.  The blocks
// hold floor/ceil shares of the rows and columns and an XCD's workgroup count
// is fixed by the round-robin deal, so a block can hold more tiles than its
// XCD has workgroups: those tiles go, in XCD order, to the workgroups that
// XCDs with smaller blocks have left over.  Every bid in [0, tiles_m * tiles_n)
// maps to a distinct tile (tests/tile_order_check.hip checks this on the
// host).  Uniform per workgroup (scalar arithmetic).
__host__ __device__ __forceinline__ int xcd_block_tile(int bid, int tiles_m, int tiles_n, int gm) {
    constexpr int kXcd = 8;
    const int gn = kXcd / gm, count = tiles_m * tiles_n;
    if (count < kXcd * 2 || tiles_m < gm || tiles_n < gn) return xcd_swizzle(bid, count);
    struct Block { int r0, c0, cols, tiles, slots; };
    auto block = [&](int x) {
        const int yr = x / gn, yc = x % gn;
        const int r0 = yr * tiles_m / gm, r1 = (yr + 1) * tiles_m / gm;
        const int c0 = yc * tiles_n / gn, c1 = (yc + 1) * tiles_n / gn;
        return Block{r0, c0, c1 - c0, (r1 - r0) * (c1 - c0), count / kXcd + (x < count % kXcd)};
    };
    const int x = bid % kXcd, l = bid / kXcd;
    Block b = block(x);
    if (l < b.tiles) return (b.r0 + l / b.cols) * tiles_n + b.c0 + l % b.cols;
    // A workgroup this XCD has left over: the j-th tile, in XCD order, of the
    // blocks larger than their XCD's share.
    int j = l - b.tiles;
    for (int y = 0; y < x; ++y) {
        const Block o = block(y);
        if (o.slots > o.tiles) j += o.slots - o.tiles;
    }
    for (int y = 0; y < kXcd; ++y) {
        b = block(y);
        const int extra = b.tiles - b.slots;
        if (extra <= 0) continue;
        if (j < extra) {
            const int t = b.slots + j;
            return (b.r0 + t / b.cols) * tiles_n + b.c0 + t % b.cols;
        }
        j -= extra;
    }
    return 0;  // not reached: the left-over workgroups and tiles are equal in number
}

}  // namespace bfhip
