// Tiled bf16 MFMA GEMM core for gfx950: C[M,N] = A[M,K] * B[N,K]^T.
//
// One workgroup computes a BM x BN tile with WM x WN wave64s; each wave owns a
// (BM/WM) x (BN/WN) sub-tile built from 16x16x32 MFMA fragments with fp32
// accumulators.  A and B stream through double-buffered LDS tiles of BK
// reduction columns: while the matrix cores consume buffer k, the next tile is
// fetched into registers and written to buffer k^1, one barrier per step.
// LDS rows are padded by 8 bf16 (16 B) so the per-lane 16-byte fragment reads
// of 16 consecutive rows hit distinct banks.
//
// Operand producers ("loaders") and the output consumer ("epilogue") are
// template policies, so the same main loop serves plain linear layers,
// LayerNorm-fed linears, implicit-GEMM convolutions with arbitrary gathers,
// and fused bias / GELU / ReLU / residual / NCHW / split / transpose stores.
#pragma once

#include "hip_common.h"

namespace bfhip {

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int kThreads = WM * WN * kWave;
    static constexpr int kWaveRows = BM / WM, kWaveCols = BN / WN;
    static constexpr int kFragM = kWaveRows / 16, kFragN = kWaveCols / 16;
    static constexpr int kStride = BK + 8;  // bf16 elements per LDS row
    static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA depth");
    static_assert(kWaveRows % 16 == 0 && kWaveCols % 16 == 0, "wave tile must be 16-aligned");
};

// ------------------------------------------------------------------ loaders
// Row-major bf16 operand X[R, K] (leading dimension ld, K % 8 == 0, rows
// 16-byte aligned).  Fills LDS rows [0, ROWS) of the tile.
template <int ROWS, int BK, int THREADS>
struct LoadRowsBf16 {
    static constexpr int kPerRow = BK / 8;
    static constexpr int kChunks = ROWS * kPerRow;
    static constexpr int kPer = (kChunks + THREADS - 1) / THREADS;
    const bf16 *base;
    int ld, rows, K;
    int r0, tid;
    bf16x8 st[kPer];

    __device__ void setup(int origin, int t) { r0 = origin; tid = t; }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int c = tid + p * THREADS;
            const int r = c / kPerRow, gk = k0 + (c % kPerRow) * 8, gr = r0 + r;
            bf16x8 v = {};
            if (c < kChunks && gr < rows && gk < K)
                v = *reinterpret_cast<const bf16x8 *>(base + (size_t)gr * ld + gk);
            st[p] = v;
        }
    }
    __device__ void store(bf16 *lds) const {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int c = tid + p * THREADS;
            if (c < kChunks)
                *reinterpret_cast<bf16x8 *>(lds + (c / kPerRow) * (BK + 8) + (c % kPerRow) * 8) = st[p];
        }
    }
};

// Row-major fp32 operand converted to bf16 on the way into LDS.  VEC requires
// K % 4 == 0, ld % 4 == 0 and a 16-byte aligned base; otherwise elementwise.
template <int ROWS, int BK, int THREADS, bool VEC>
struct LoadRowsF32 {
    static constexpr int kPerRow = BK / 8;
    static constexpr int kChunks = ROWS * kPerRow;
    static constexpr int kPer = (kChunks + THREADS - 1) / THREADS;
    const float *base;
    int ld, rows, K;
    int r0, tid;
    bf16x8 st[kPer];

    __device__ void setup(int origin, int t) { r0 = origin; tid = t; }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int c = tid + p * THREADS;
            const int gr = r0 + c / kPerRow, gk = k0 + (c % kPerRow) * 8;
            bf16x8 v = {};
            if (c < kChunks && gr < rows) {
                const float *src = base + (size_t)gr * ld + gk;
                if (VEC) {
                    if (gk < K) {  // K % 8 == 0 is not required: K % 4 == 0 is
                        const float4 lo = *reinterpret_cast<const float4 *>(src);
                        v[0] = to_bf16(lo.x); v[1] = to_bf16(lo.y);
                        v[2] = to_bf16(lo.z); v[3] = to_bf16(lo.w);
                        if (gk + 4 < K) {
                            const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
                            v[4] = to_bf16(hi.x); v[5] = to_bf16(hi.y);
                            v[6] = to_bf16(hi.z); v[7] = to_bf16(hi.w);
                        }
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gk + e < K) v[e] = to_bf16(src[e]);
                }
            }
            st[p] = v;
        }
    }
    __device__ void store(bf16 *lds) const {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int c = tid + p * THREADS;
            if (c < kChunks)
                *reinterpret_cast<bf16x8 *>(lds + (c / kPerRow) * (BK + 8) + (c % kPerRow) * 8) = st[p];
        }
    }
};

// ------------------------------------------------------------------ main loop
template <class T, class ALoad, class BLoad, class Epi>
__global__ __launch_bounds__(T::kThreads) void gemm_kernel(ALoad al, BLoad bl, Epi epi,
                                                           int M, int N, int K, int tiles_n) {
    // One LDS arena: double-buffered A/B tiles in the main loop, then (for
    // row-vector epilogues) the fp32 output tile.
    constexpr int kCStride = T::BN + 4;  // floats; staggers rows across banks
    constexpr size_t kABBytes = (size_t)2 * (T::BM + T::BN) * T::kStride * sizeof(bf16);
    constexpr size_t kCBytes = Epi::kRowVector ? (size_t)T::BM * kCStride * sizeof(float) : 0;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kABBytes > kCBytes ? kABBytes : kCBytes];
    bf16(*sA)[T::BM * T::kStride] = reinterpret_cast<bf16(*)[T::BM * T::kStride]>(smem);
    bf16(*sB)[T::BN * T::kStride] =
        reinterpret_cast<bf16(*)[T::BN * T::kStride]>(smem + (size_t)2 * T::BM * T::kStride * sizeof(bf16));

    const int pid = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);
    const int m0 = (pid / tiles_n) * T::BM, n0 = (pid % tiles_n) * T::BN;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;

    al.setup(m0, tid);
    bl.setup(n0, tid);

    f32x4 acc[T::kFragM][T::kFragN];
#pragma unroll
    for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
        for (int j = 0; j < T::kFragN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (K + T::BK - 1) / T::BK;
    al.load(0);
    bl.load(0);
    al.store(sA[0]);
    bl.store(sB[0]);
    __syncthreads();

    const int a_off = (wm * T::kWaveRows + (lane & 15)) * T::kStride + 8 * (lane >> 4);
    const int b_off = (wn * T::kWaveCols + (lane & 15)) * T::kStride + 8 * (lane >> 4);

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            al.load((kt + 1) * T::BK);
            bl.load((kt + 1) * T::BK);
        }
        const bf16 *a = sA[cur] + a_off;
        const bf16 *b = sB[cur] + b_off;
#pragma unroll
        for (int kk = 0; kk < T::BK; kk += 32) {
            bf16x8 af[T::kFragM], bfr[T::kFragN];
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(a + i * 16 * T::kStride + kk);
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(b + j * 16 * T::kStride + kk);
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
                for (int j = 0; j < T::kFragN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
        }
        if (more) {
            al.store(sA[cur ^ 1]);
            bl.store(sB[cur ^ 1]);
        }
        __syncthreads();
    }

    if constexpr (Epi::kRowVector) {
        // Stage the tile through LDS (the loop's final barrier freed it) so
        // the epilogue writes whole rows with 16-byte vectors instead of one
        // scalar per lane per row.
        float *sC = reinterpret_cast<float *>(smem);
        const int r0 = wm * T::kWaveRows + 4 * (lane >> 4), c0 = wn * T::kWaveCols + (lane & 15);
#pragma unroll
        for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sC[(r0 + i * 16 + r) * kCStride + c0 + j * 16] = acc[i][j][r];
        __syncthreads();
        constexpr int kQuads = T::BN / 4;
        for (int c = tid; c < T::BM * kQuads; c += T::kThreads) {
            const int r = c / kQuads, q = c - r * kQuads;
            epi.row4(m0 + r, n0 + 4 * q, *reinterpret_cast<const float4 *>(sC + r * kCStride + 4 * q));
        }
    } else {
        const int row_base = m0 + wm * T::kWaveRows + 4 * (lane >> 4);
        const int col_base = n0 + wn * T::kWaveCols + (lane & 15);
#pragma unroll
        for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j) epi(row_base + i * 16, col_base + j * 16, acc[i][j]);
    }
}

// Host launcher: one workgroup per output tile.
template <class T, class ALoad, class BLoad, class Epi>
inline void launch_gemm(const ALoad &al, const BLoad &bl, const Epi &epi, int M, int N, int K,
                        hipStream_t stream) {
    const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    hipLaunchKernelGGL((gemm_kernel<T, ALoad, BLoad, Epi>), dim3(tiles_m * tiles_n),
                       dim3(T::kThreads), 0, stream, al, bl, epi, M, N, K, tiles_n);
}

// ---------------------------------------------------------------- epilogues
// Each is called with the fragment origin (row, col) of four consecutive rows
// row..row+3 in one column; bounds are the epilogue's responsibility.

// Row-vector epilogues (kRowVector) receive four consecutive columns of one
// row through row4(); vector stores need ld % 4 == 0 and an aligned base,
// otherwise they fall back to scalars.
struct EpiRowsF32 {  // out[row*ld + col] = v (+bias) (ReLU)
    static constexpr bool kRowVector = true;
    float *out;
    const float *bias;
    int ld, M, N, relu;
    __device__ void row4(int row, int col, float4 v) const {
        if (row >= M || col >= N) return;
        float y[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (bias && col + e < N) y[e] += bias[col + e];
            if (relu && y[e] < 0.0f) y[e] = 0.0f;
        }
        float *p = out + (size_t)row * ld + col;
        if (col + 3 < N && (ld & 3) == 0 && ((uintptr_t)out & 15) == 0) {
            *reinterpret_cast<float4 *>(p) = make_float4(y[0], y[1], y[2], y[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < N) p[e] = y[e];
        }
    }
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= N) return;
        const float b = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (row + r < M) {
                float y = v[r] + b;
                if (relu && y < 0.0f) y = 0.0f;
                out[(size_t)(row + r) * ld + col] = y;
            }
    }
};

template <bool GELU>
struct EpiRowsBf16 {  // out[row*ld + col] = bf16(act(v + bias)); ld % 4 == 0
    static constexpr bool kRowVector = true;
    bf16 *out;
    const float *bias;
    int ld, M, N;
    __device__ void row4(int row, int col, float4 v) const {
        if (row >= M || col >= N) return;
        float y[4] = {v.x, v.y, v.z, v.w};
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = y[e] + (bias && col + e < N ? bias[col + e] : 0.0f);
            if (GELU) t = gelu_erf(t);
            o[e] = to_bf16(t);
        }
        bf16 *p = out + (size_t)row * ld + col;
        if (col + 3 < N) {
            *reinterpret_cast<bf16x4 *>(p) = o;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < N) p[e] = o[e];
        }
    }
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= N) return;
        const float b = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (row + r < M) {
                float y = v[r] + b;
                if (GELU) y = gelu_erf(y);
                out[(size_t)(row + r) * ld + col] = to_bf16(y);
            }
    }
};

struct EpiResidualF32 {  // x[row*ld + col] += v + bias; ld % 4 == 0
    static constexpr bool kRowVector = true;
    float *x;
    const float *bias;
    int ld, M, N;
    __device__ void row4(int row, int col, float4 v) const {
        if (row >= M || col >= N) return;
        float *p = x + (size_t)row * ld + col;
        if (col + 3 < N) {
            float4 a = *reinterpret_cast<const float4 *>(p);
            const float4 b = bias ? *reinterpret_cast<const float4 *>(bias + col) : make_float4(0, 0, 0, 0);
            a.x += v.x + b.x; a.y += v.y + b.y; a.z += v.z + b.z; a.w += v.w + b.w;
            *reinterpret_cast<float4 *>(p) = a;
        } else {
            const float y[4] = {v.x, v.y, v.z, v.w};
            for (int e = 0; e < 4 && col + e < N; ++e) p[e] = p[e] + (y[e] + (bias ? bias[col + e] : 0.0f));
        }
    }
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= N) return;
        const float b = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (row + r < M) {
                float *p = x + (size_t)(row + r) * ld + col;
                *p = *p + (v[r] + b);
            }
    }
};

// Implicit-GEMM convolution output: row = n*OHW + p, col = output channel,
// stored NCHW.  Four consecutive rows of one image are one float4 when aligned.
struct EpiNCHW {
    static constexpr bool kRowVector = false;
    float *out;
    const float *bias;
    int M, Co, ohw, relu;
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= Co) return;
        const float b = bias ? bias[col] : 0.0f;
        f32x4 y;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            y[r] = v[r] + b;
            if (relu && y[r] < 0.0f) y[r] = 0.0f;
        }
        const int n = row / ohw, p = row - n * ohw;
        if ((ohw & 3) == 0 && row + 3 < M) {  // rows 4-aligned => same image
            *reinterpret_cast<f32x4 *>(out + ((size_t)n * Co + col) * ohw + p) = y;
            return;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = row + r;
            if (rr >= M) break;
            const int nn = rr / ohw, pp = rr - nn * ohw;
            out[((size_t)nn * Co + col) * ohw + pp] = y[r];
        }
    }
};

}  // namespace bfhip
