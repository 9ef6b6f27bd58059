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

#include <type_traits>

namespace bfhip {

// F16_: operands are fp16 words (fp16 MFMA) instead of bf16.
template <int BM_, int BN_, int BK_, int WM_, int WN_, bool F16_ = false>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr bool kF16 = F16_;
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

// Workgroup barrier for LDS traffic: waits for this wave's own LDS accesses
// (lgkmcnt), then s_barrier; unlike __syncthreads it leaves global loads and
// LDS-DMA in flight (vmcnt), so a prefetch survives it.  The lgkmcnt wait is
// what makes a stage buffer free after the barrier: the compiler may sink the
// MFMAs that consume a wave's last fragment reads below the barrier, leaving
// those reads outstanding, and another wave's next DMA into that buffer could
// overtake them.  The empty asm statements keep the compiler from moving LDS
// accesses across it.  s_waitcnt encoding (gfx9): vmcnt 63, expcnt 7,
// lgkmcnt 0.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ epilogue
// Optional epilogue traits: kRowStat epilogues need one Stat per output row
// (e.g. LayerNorm statistics): thread t < BM fetches row m0 + t's inputs at
// kernel start (Pre stat_load(row), so the loads overlap the main loop),
// reduces them after it (Stat stat_finish(pre)) into LDS, and rows() gets
// them; kFullRow epilogues take the whole staged fp32 tile
// (tile<T>(sC, stride, m0, n0, tid)) to reduce across full rows or to store it
// in another order.
template <class E, class = void>
struct EpiRowStat : std::false_type {};
template <class E>
struct EpiRowStat<E, std::void_t<decltype(E::kRowStat)>> : std::bool_constant<E::kRowStat> {};
struct NoRowStat {};
template <class E, bool = EpiRowStat<E>::value>
struct EpiPre { using type = NoRowStat; using stat = float2; };
template <class E>
struct EpiPre<E, true> { using type = typename E::Pre; using stat = typename E::Stat; };

// kCorrSteps > 0 (row-statistics epilogues only): before staging, every
// accumulator gets a rank-limited correction added on the matrix cores,
// acc[row][col] += sum over kCorrSteps 32-deep k-steps of A[row][k] B[col][k].
// A carries per-row values split into two fp16 words each: k-slots 2t and
// 2t + 1 hold hi = fp16(u_t) and lo = fp16(u_t - hi), u_4q..u_4q+3 coming
// from the row's Stat as epi.corr_u4(stat, q); B is the epilogue's fp16
// table (epi.corr_col(col, k0) -> 8 words at k0..k0+7), fetched at kernel
// start.  The LayerNorm-folded linears use it for their centring correction
// (ln_fold.h).
template <class E, class = void>
struct EpiCorr { static constexpr int value = 0; };
template <class E>
struct EpiCorr<E, std::void_t<decltype(E::kCorrSteps)>> { static constexpr int value = E::kCorrSteps; };

template <class T, class Epi, int KC = EpiCorr<Epi>::value>
struct EpiPrefetch {
    typename EpiPre<Epi>::type pre;
    bf16x8 cb[T::kFragN][KC];  // correction B fragments of the wave's columns
};
template <class T, class Epi>
struct EpiPrefetch<T, Epi, 0> {
    typename EpiPre<Epi>::type pre;
};

template <class T, class Epi>
__device__ __forceinline__ EpiPrefetch<T, Epi> epi_prefetch(const Epi &epi, int m0, int n0, int tid) {
    static_assert(!EpiRowStat<Epi>::value || T::BM <= T::kThreads, "one thread per tile row");
    static_assert(EpiCorr<Epi>::value == 0 || (EpiRowStat<Epi>::value && Epi::kRowVector),
                  "the correction reads the staged row statistics");
    EpiPrefetch<T, Epi> pf{};
    if constexpr (EpiRowStat<Epi>::value)
        if (tid < T::BM) pf.pre = epi.stat_load(m0 + tid);
    if constexpr (EpiCorr<Epi>::value > 0) {
        const int lane = tid & 63, wn = (tid >> 6) % T::WN;
#pragma unroll
        for (int j = 0; j < T::kFragN; ++j)
#pragma unroll
            for (int c = 0; c < EpiCorr<Epi>::value; ++c)
                pf.cb[j][c] = epi.corr_col(n0 + wn * T::kWaveCols + j * 16 + (lane & 15),
                                           32 * c + 8 * (lane >> 4));
    }
    return pf;
}
// kQuadRows epilogues reduce across the 16 lanes that hold one 64-column
// group (row16_sum): they need the whole-quad path below, in which every
// thread owns one column quad for the whole tile and control flow is uniform
// over each row of 16 lanes.
template <class E, class = void>
struct EpiQuadRows : std::false_type {};
template <class E>
struct EpiQuadRows<E, std::void_t<decltype(E::kQuadRows)>> : std::bool_constant<E::kQuadRows> {};
template <class E, class = void>
struct EpiFullRow : std::false_type {};
template <class E>
struct EpiFullRow<E, std::void_t<decltype(E::kFullRow)>> : std::bool_constant<E::kFullRow> {};

// Hands the accumulators of one BM x BN tile to the epilogue policy.  Row-vector
// epilogues get the tile staged through LDS (the caller has synchronised the
// arena) so that whole rows leave as 16-byte vectors; column-fragment
// epilogues take the four rows of each MFMA fragment directly.
template <class T, class Epi>
__device__ __forceinline__ void store_tile(f32x4 (&acc)[T::kFragM][T::kFragN], const Epi &epi,
                                           unsigned char *smem, int m0, int n0, int tid,
                                           const EpiPrefetch<T, Epi> &pf) {
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;
    if constexpr (Epi::kRowVector) {
        constexpr int kCStride = T::BN + 4;  // floats; staggers rows across banks
        float *sC = reinterpret_cast<float *>(smem);
        using Stat = typename EpiPre<Epi>::stat;
        Stat *sStat = reinterpret_cast<Stat *>(smem + (size_t)T::BM * kCStride * sizeof(float));
        const int r0 = wm * T::kWaveRows + 4 * (lane >> 4), c0 = wn * T::kWaveCols + (lane & 15);
        if constexpr (EpiCorr<Epi>::value > 0) {
            // Row statistics first (the correction's A operand), then the
            // correction on the matrix cores, then the staging below.
            if (tid < T::BM) sStat[tid] = epi.stat_finish(pf.pre);
            lds_barrier();
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i) {
                const Stat &st = sStat[wm * T::kWaveRows + i * 16 + (lane & 15)];
#pragma unroll
                for (int c = 0; c < EpiCorr<Epi>::value; ++c) {
                    const float4 u4 = epi.corr_u4(st, 4 * c + (lane >> 4));
                    const float u[4] = {u4.x, u4.y, u4.z, u4.w};
                    bf16x8 a;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        a[2 * t] = to_half(u[t]);
                        a[2 * t + 1] = to_half(u[t] - half_to_f32(a[2 * t]));
                    }
#pragma unroll
                    for (int j = 0; j < T::kFragN; ++j) acc[i][j] = mfma16_as<T::kF16>(a, pf.cb[j][c], acc[i][j]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sC[(r0 + i * 16 + r) * kCStride + c0 + j * 16] = acc[i][j][r];
        if constexpr (EpiRowStat<Epi>::value && EpiCorr<Epi>::value == 0)
            if (tid < T::BM) sStat[tid] = epi.stat_finish(pf.pre);
        lds_barrier();  // LDS only: prefetches in flight stay in flight
        constexpr int kQuads = T::BN / 4;
        static_assert(!(EpiRowStat<Epi>::value || EpiQuadRows<Epi>::value) ||
                          (T::kThreads % kQuads == 0 && T::BM % (T::kThreads / kQuads) == 0),
                      "row-statistics and 64-column-group epilogues need whole column quads per thread");
        if constexpr (EpiFullRow<Epi>::value) {
            epi.template tile<T>(sC, kCStride, m0, n0, tid);
        } else if constexpr (T::kThreads % kQuads == 0 && T::BM % (T::kThreads / kQuads) == 0) {
            // Each thread owns one column quad for the whole tile: the
            // epilogue's per-column state (bias) is fetched once, and all of
            // the thread's rows are handed over together so that their
            // global reads (residual) can be in flight at once.
            constexpr int kStep = T::kThreads / kQuads, kRows = T::BM / kStep;
            const int q = tid % kQuads, r = tid / kQuads;
            float4 v[kRows];
#pragma unroll
            for (int i = 0; i < kRows; ++i)
                v[i] = *reinterpret_cast<const float4 *>(sC + (r + i * kStep) * kCStride + 4 * q);
            if constexpr (EpiRowStat<Epi>::value)
                epi.template rows<kRows>(m0 + r, kStep, epi.column(n0 + 4 * q), v, sStat + r);
            else
                epi.template rows<kRows>(m0 + r, kStep, epi.column(n0 + 4 * q), v);
        } else {
            for (int c = tid; c < T::BM * kQuads; c += T::kThreads) {
                const int r = c / kQuads, q = c - r * kQuads;
                const float4 v[1] = {*reinterpret_cast<const float4 *>(sC + r * kCStride + 4 * q)};
                epi.template rows<1>(m0 + r, 0, epi.column(n0 + 4 * q), v);
            }
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

// Barriers inside a kFullRow epilogue's tile() (E::kTileBarriers, default 0).
template <class E, class = void>
struct EpiTileBarriers { static constexpr int value = 0; };
template <class E>
struct EpiTileBarriers<E, std::void_t<decltype(E::kTileBarriers)>> {
    static constexpr int value = E::kTileBarriers;
};

// Barriers store_tile executes, tile() included (the spec kernel's loader
// waves pass as many).
template <class Epi>
constexpr int store_tile_barriers() {
    if constexpr (!Epi::kRowVector) return 0;
    else
        return 1 + (EpiCorr<Epi>::value > 0 ? 1 : 0) +
               (EpiFullRow<Epi>::value ? EpiTileBarriers<Epi>::value : 0);
}

template <class T, class Epi>
constexpr size_t epilogue_bytes() {
    return Epi::kRowVector ? (size_t)T::BM * (T::BN + 4) * sizeof(float) +
                                 (EpiRowStat<Epi>::value ? (size_t)T::BM * sizeof(typename EpiPre<Epi>::stat) : 0)
                           : 0;
}

// ------------------------------------------------------------------ main loop
// One LDS arena: double-buffered A/B tiles in the main loop, then (for
// row-vector epilogues) the fp32 output tile.
template <class T, class Epi>
constexpr size_t reg_smem_bytes() {
    constexpr size_t kABBytes = (size_t)2 * (T::BM + T::BN) * T::kStride * sizeof(bf16);
    constexpr size_t kCBytes = epilogue_bytes<T, Epi>();
    return kABBytes > kCBytes ? kABBytes : kCBytes;
}
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_reg_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                               int K, int tiles_n, int pid, unsigned char *smem);

template <class T, class ALoad, class BLoad, class Epi>
__global__ __launch_bounds__(T::kThreads) void gemm_kernel(ALoad al, BLoad bl, Epi epi,
                                                           int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[reg_smem_bytes<T, Epi>()];
    gemm_reg_block<T>(al, bl, epi, M, N, K, tiles_n, xcd_swizzle((int)blockIdx.x, (int)gridDim.x), smem);
}

// Tile `pid` of the register-fed core on the workgroup's `smem`
// (reg_smem_bytes); gemm_kernel is one such tile per workgroup.
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_reg_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                               int K, int tiles_n, int pid, unsigned char *smem) {
    bf16(*sA)[T::BM * T::kStride] = reinterpret_cast<bf16(*)[T::BM * T::kStride]>(smem);
    bf16(*sB)[T::BN * T::kStride] =
        reinterpret_cast<bf16(*)[T::BN * T::kStride]>(smem + (size_t)2 * T::BM * T::kStride * sizeof(bf16));

    const int m0 = (pid / tiles_n) * T::BM, n0 = (pid % tiles_n) * T::BN;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;

    al.setup(m0, tid);
    bl.setup(n0, tid);
    const auto pre = epi_prefetch<T>(epi, m0, n0, tid);

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
                for (int j = 0; j < T::kFragN; ++j) acc[i][j] = mfma16_as<T::kF16>(af[i], bfr[j], acc[i][j]);
        }
        if (more) {
            al.store(sA[cur ^ 1]);
            bl.store(sB[cur ^ 1]);
        }
        __syncthreads();
    }

    store_tile<T>(acc, epi, smem, m0, n0, tid, pre);
}

// Host launcher: one workgroup per output tile.
template <class T, class ALoad, class BLoad, class Epi>
inline void launch_gemm(const ALoad &al, const BLoad &bl, const Epi &epi, int M, int N, int K,
                        hipStream_t stream) {
    const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    hipLaunchKernelGGL((gemm_kernel<T, ALoad, BLoad, Epi>), dim3(tiles_m * tiles_n),
                       dim3(T::kThreads), 0, stream, al, bl, epi, M, N, K, tiles_n);
}

// ====================================================== LDS-DMA pipelined core
// Operands that are plain bf16 rows (or 16-byte gathers of them) skip the
// register round trip: buffer_load_dwordx4 ... lds writes each lane's 16 bytes
// straight into LDS at M0 + 16 * lane, so a wave instruction fills 1 KiB of
// the tile.  With registers out of the way, STAGES-1 k-tiles are in flight
// while the matrix cores work on the current one, which is what the short
// reductions of this path (K = 96 ... 3072, a handful of k-tiles per output
// tile) need: one k-tile of look-ahead leaves the loop bound by memory latency.
//
// LDS rows hold BK bf16 with no padding.  To keep the 16-byte fragment reads
// of 8 consecutive rows on distinct banks, chunk c of row r is stored in slot
// c ^ swz(r); the DMA side applies the same permutation to the global chunk
// each lane fetches, so the stored image is already swizzled.
template <int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_, bool F16_ = false>
struct DmaTile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, kStages = STAGES_;
    static constexpr bool kF16 = F16_;
    static constexpr int kThreads = WM * WN * kWave;
    static constexpr int kWaveRows = BM / WM, kWaveCols = BN / WN;
    static constexpr int kFragM = kWaveRows / 16, kFragN = kWaveCols / 16;
    static_assert(BK == 32 || BK == 64 || BK == 128, "swizzle covers BK of 32, 64 or 128");
    static_assert(kWaveRows % 16 == 0 && kWaveCols % 16 == 0, "wave tile must be 16-aligned");
    static_assert(kStages >= 2 && kStages <= 8, "2 to 8 stages");
};

// Tile order of the DMA and wave-specialised kernels.  By default
// xcd_swizzle keeps consecutive row-major tiles on one XCD, so each XCD sweeps
// whole row panels and fetches all of B: right when A is the larger operand.
// A tile type derived as XcdBlocks<T, GM> deals the grid as GM row groups x
// 8 / GM column groups instead (xcd_block_tile), for layers whose B (the
// weights) is as large as A or larger; the choice is compile-time, so other
// layers' kernels carry no decode.
template <class T, class = void>
struct TileXcdRowGroups { static constexpr int value = 0; };
template <class T>
struct TileXcdRowGroups<T, std::void_t<decltype(T::kXcdRowGroups)>> {
    static constexpr int value = T::kXcdRowGroups;
};
template <class T, int GM>
struct XcdBlocks : T {
    static_assert(GM == 1 || GM == 2 || GM == 4 || GM == 8, "row groups must divide the 8 XCDs");
    static constexpr int kXcdRowGroups = GM;
};

template <class T>
__device__ __forceinline__ int tile_pid(int tiles_n) {
    const int bid = (int)blockIdx.x, count = (int)gridDim.x;
    if constexpr (TileXcdRowGroups<T>::value == 0)
        return xcd_swizzle(bid, count);
    else
        return xcd_block_tile(bid, count / tiles_n, tiles_n, TileXcdRowGroups<T>::value);
}

template <int BK>
__device__ __forceinline__ int dma_swizzle(int r) {
    return BK == 32 ? (r >> 1) & 3 : r & 7;
}

// s_waitcnt vmcnt(n) leaving lgkmcnt/expcnt alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}


__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    // Raw buffer, 32-bit data format: offsets at or past `bytes` read as zero.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

constexpr uint32_t kDmaOutOfRange = 0x80000000u;  // >= any num_records used here

// One 16-byte LDS-DMA per lane: LDS[M0 + 16 * lane] = buffer[voffset + soffset].
// soffset is wave-uniform (an SGPR), so per-step address arithmetic that is
// the same for every lane (the k offset) costs no vector instructions.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, bf16 *lds, uint32_t voffset,
                                      uint32_t soffset = 0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void *)(lds), 16, voffset, (int)soffset, 0, 0);
}

// Row-major bf16 operand X[R, K] (leading dimension ld elements, K % 8 == 0,
// 16-byte aligned rows, R * ld * 2 < 2^31 bytes).  Rows past R and k past K
// read as zero.  The lane's row and chunk offset are fixed per tile (vector
// registers); the k-tile offset rides in soffset, so a full k-tile issues
// with no vector arithmetic.  A partial last k-tile (K % BK != 0) checks k
// per lane.
template <int ROWS, int BK, int THREADS>
struct DmaRowsBf16 {
    static constexpr int kCpr = BK / 8, kWaves = THREADS / kWave;
    static constexpr int kChunks = ROWS * kCpr;
    static_assert(kChunks % (kWave * kWaves) == 0, "tile must split evenly over the waves");
    static constexpr int kIssue = kChunks / (kWave * kWaves);  // DMA instructions per wave per stage
    const bf16 *base;
    int ld, rows, K;
    int wave;                  // wave-uniform (SGPR)
    uint32_t voff[kIssue];     // byte offset of the lane's row + chunk, or kDmaOutOfRange
    int kcol[kIssue];          // first k of the lane's chunk within the tile

    __device__ void setup(int r0, int tid) {
        wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        const int lane = tid % kWave;
#pragma unroll
        for (int j = 0; j < kIssue; ++j) {
            const int q = (j * kWaves + wave) * kWave + lane;
            const int r = q / kCpr, slot = q % kCpr;
            kcol[j] = 8 * (slot ^ dma_swizzle<BK>(r));
            voff[j] = r0 + r < rows ? ((uint32_t)(r0 + r) * (uint32_t)ld + (uint32_t)kcol[j]) * 2u
                                    : kDmaOutOfRange;
        }
    }
    __device__ void issue(bf16 *lds, int k0) const {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(base, (uint32_t)rows * (uint32_t)ld * 2u);
        if (k0 + BK <= K) {
#pragma unroll
            for (int j = 0; j < kIssue; ++j)
                dma16(rsrc, lds + (j * kWaves + wave) * kWave * 8, voff[j], 2u * (uint32_t)k0);
        } else {
#pragma unroll
            for (int j = 0; j < kIssue; ++j) {
                const bool in = voff[j] != kDmaOutOfRange && k0 + kcol[j] < K;
                dma16(rsrc, lds + (j * kWaves + wave) * kWave * 8, in ? voff[j] + 2u * k0 : kDmaOutOfRange);
            }
        }
    }
};

// Wait until at most n stages of P instructions are outstanding.  The counter
// holds 63 at most: a larger bound is clamped, which waits for more stages
// than needed (always safe).
template <int N>
struct DmaWait {
    template <int P>
    __device__ static void stages(int n) {
        if constexpr (N > 0) {
            if (n >= N) { wait_vmcnt<(N * P > 63 ? 63 : N * P)>(); return; }
            DmaWait<N - 1>::template stages<P>(n);
        } else {
            wait_vmcnt<0>();
        }
    }
};

// LDS of one LDS-DMA / wave-specialised workgroup: stages, or the epilogue's
// staging tile if larger.
template <class T, class Epi>
constexpr size_t dma_smem_bytes() {
    constexpr size_t kAB = (size_t)T::kStages * (T::BM + T::BN) * T::BK * sizeof(bf16);
    constexpr size_t kC = epilogue_bytes<T, Epi>();
    return kAB > kC ? kAB : kC;
}
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_dma_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                               int K, int tiles_n, int pid, unsigned char *smem);
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_spec_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                                int K, int tiles_n, int pid, unsigned char *smem);

template <class T, class ALoad, class BLoad, class Epi>
__global__ __launch_bounds__(T::kThreads) void gemm_dma_kernel(ALoad al, BLoad bl, Epi epi,
                                                               int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[dma_smem_bytes<T, Epi>()];
    gemm_dma_block<T>(al, bl, epi, M, N, K, tiles_n, tile_pid<T>(tiles_n), smem);
}

// Tile `pid` of the LDS-DMA core on the workgroup's `smem` (dma_smem_bytes);
// gemm_dma_kernel is one such tile per workgroup, and a kernel that fuses
// other work into the same launch can call it for part of its grid.
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_dma_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                               int K, int tiles_n, int pid, unsigned char *smem) {
    constexpr int S = T::kStages;
    constexpr int kA = T::BM * T::BK, kB = T::BN * T::BK;  // elements per stage
    bf16 *sA = reinterpret_cast<bf16 *>(smem);
    bf16 *sB = sA + S * kA;

    const int m0 = (pid / tiles_n) * T::BM, n0 = (pid % tiles_n) * T::BN;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;

    al.setup(m0, tid);
    bl.setup(n0, tid);
    const auto pre = epi_prefetch<T>(epi, m0, n0, tid);

    f32x4 acc[T::kFragM][T::kFragN];
#pragma unroll
    for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
        for (int j = 0; j < T::kFragN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (K + T::BK - 1) / T::BK;
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
        if (st < nk) {
            al.issue(sA + st * kA, st * T::BK);
            bl.issue(sB + st * kB, st * T::BK);
        }

    // Fragment origins: row (lane & 15) of the wave's sub-tile; the 16-byte
    // chunk for MFMA step kk is (kk / 8 + lane / 16) ^ swz(row), and swz only
    // depends on row % 16, i.e. on the lane.
    const int swz = dma_swizzle<T::BK>(lane & 15);
    const int a_row = (wm * T::kWaveRows + (lane & 15)) * T::BK;
    const int b_row = (wn * T::kWaveCols + (lane & 15)) * T::BK;
    constexpr int kSteps = T::BK / 32;
    int koff[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) koff[s] = 8 * ((4 * s + (lane >> 4)) ^ swz);

    constexpr int P = ALoad::kIssue + BLoad::kIssue;
    for (int kt = 0; kt < nk; ++kt) {
        const int ahead = nk - 1 - kt;  // stages issued after this one
        DmaWait<S - 2>::template stages<P>(ahead < S - 2 ? ahead : S - 2);
        lds_barrier();
        const int nxt = kt + S - 1;
        if (nxt < nk) {
            al.issue(sA + (nxt % S) * kA, nxt * T::BK);
            bl.issue(sB + (nxt % S) * kB, nxt * T::BK);
        }
        const bf16 *a = sA + (kt % S) * kA + a_row;
        const bf16 *b = sB + (kt % S) * kB + b_row;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            bf16x8 af[T::kFragM], bfr[T::kFragN];
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(a + i * 16 * T::BK + koff[s]);
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(b + j * 16 * T::BK + koff[s]);
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
                for (int j = 0; j < T::kFragN; ++j) acc[i][j] = mfma16_as<T::kF16>(af[i], bfr[j], acc[i][j]);
        }
    }
    __syncthreads();  // every wave is done with the stage buffers
    store_tile<T>(acc, epi, smem, m0, n0, tid, pre);
}

template <class T, class ALoad, class BLoad, class Epi>
inline void launch_gemm_dma(const ALoad &al, const BLoad &bl, const Epi &epi, int M, int N, int K,
                            hipStream_t stream) {
    const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    hipLaunchKernelGGL((gemm_dma_kernel<T, ALoad, BLoad, Epi>), dim3(tiles_m * tiles_n),
                       dim3(T::kThreads), 0, stream, al, bl, epi, M, N, K, tiles_n);
}

// ======================================== wave-specialised LDS-DMA pipeline
// Same tile, LDS image, loaders and epilogues as gemm_dma_kernel, plus LW
// loader waves that issue every DMA; the WM x WN compute waves never issue a
// vector-memory instruction in the main loop.  In gemm_dma_kernel each wave
// issues its share of the next stage and then runs its MFMAs: when the fetch
// path is the bottleneck the issue itself stalls until the texture unit takes
// the request, and the SIMD's matrix core idles meanwhile, so fetch and math
// add up instead of overlapping (measured on MI355X with a 128 x 64 tile, K =
// 1536: 5.8 us of DMA alone, 11.8 us with the MFMAs).  With the issue moved
// to its own wave, the stall holds that wave only.  A wave keeps at most 63
// vector-memory instructions (63 KiB of LDS-DMA) in flight, which caps one
// loader wave near 70 GB/s per CU at L2 latency: the 80 x 256 conv stripes
// (43 KiB per stage) take two loader waves (their DMA alone 28.8 -> 20.7 us).
//
// Per k-step kt both sides meet at one barrier: the loader has waited for
// stage kt to land, the compute waves have finished reading stage kt - 1, so
// after it the loader refills that buffer with stage kt + S - 1 while the
// compute waves multiply stage kt.  The loader then takes part in the
// epilogue's barriers (it has no rows of its own) and exits.
// ALoad / BLoad are instantiated for THREADS = LW * kWave and set up with the
// thread's index within the loader waves.
template <class T, class ALoad, class BLoad, class Epi>
__global__ __launch_bounds__(T::kThreads + ALoad::kWaves * kWave) void gemm_spec_kernel(
    ALoad al, BLoad bl, Epi epi, int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[dma_smem_bytes<T, Epi>()];
    gemm_spec_block<T>(al, bl, epi, M, N, K, tiles_n, tile_pid<T>(tiles_n), smem);
}

// Tile `pid` of the wave-specialised pipeline on the workgroup's `smem`
// (dma_smem_bytes), as gemm_dma_block.
template <class T, class ALoad, class BLoad, class Epi>
__device__ __forceinline__ void gemm_spec_block(ALoad &al, BLoad &bl, const Epi &epi, int M, int N,
                                                int K, int tiles_n, int pid, unsigned char *smem) {
    constexpr int S = T::kStages;
    constexpr int kA = T::BM * T::BK, kB = T::BN * T::BK;  // elements per stage
    bf16 *sA = reinterpret_cast<bf16 *>(smem);
    bf16 *sB = sA + S * kA;

    const int m0 = (pid / tiles_n) * T::BM, n0 = (pid % tiles_n) * T::BN;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nk = (K + T::BK - 1) / T::BK;

    if (wave >= T::WM * T::WN) {  // loader (wave-uniform branch)
        al.setup(m0, tid - T::kThreads);
        bl.setup(n0, tid - T::kThreads);
        constexpr int P = ALoad::kIssue + BLoad::kIssue;
#pragma unroll
        for (int st = 0; st < S - 1; ++st)
            if (st < nk) {
                al.issue(sA + st * kA, st * T::BK);
                bl.issue(sB + st * kB, st * T::BK);
            }
        for (int kt = 0; kt < nk; ++kt) {
            const int ahead = nk - 1 - kt;  // stages issued after this one
            DmaWait<S - 2>::template stages<P>(ahead < S - 2 ? ahead : S - 2);
            lds_barrier();
            const int nxt = kt + S - 1;
            if (nxt < nk) {
                al.issue(sA + (nxt % S) * kA, nxt * T::BK);
                bl.issue(sB + (nxt % S) * kB, nxt * T::BK);
            }
        }
        __syncthreads();  // the compute waves' end-of-loop barrier
#pragma unroll
        for (int k = 0; k < store_tile_barriers<Epi>(); ++k) __syncthreads();  // store_tile's
        return;
    }

    const int wm = wave / T::WN, wn = wave % T::WN;
    const auto pre = epi_prefetch<T>(epi, m0, n0, tid);
    f32x4 acc[T::kFragM][T::kFragN];
#pragma unroll
    for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
        for (int j = 0; j < T::kFragN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int swz = dma_swizzle<T::BK>(lane & 15);
    const int a_row = (wm * T::kWaveRows + (lane & 15)) * T::BK;
    const int b_row = (wn * T::kWaveCols + (lane & 15)) * T::BK;
    constexpr int kSteps = T::BK / 32;
    int koff[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) koff[s] = 8 * ((4 * s + (lane >> 4)) ^ swz);

    for (int kt = 0; kt < nk; ++kt) {
        lds_barrier();
        const bf16 *a = sA + (kt % S) * kA + a_row;
        const bf16 *b = sB + (kt % S) * kB + b_row;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            bf16x8 af[T::kFragM], bfr[T::kFragN];
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(a + i * 16 * T::BK + koff[s]);
#pragma unroll
            for (int j = 0; j < T::kFragN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(b + j * 16 * T::BK + koff[s]);
#pragma unroll
            for (int i = 0; i < T::kFragM; ++i)
#pragma unroll
                for (int j = 0; j < T::kFragN; ++j) acc[i][j] = mfma16_as<T::kF16>(af[i], bfr[j], acc[i][j]);
        }
    }
    __syncthreads();  // every wave is done with the stage buffers
    store_tile<T>(acc, epi, smem, m0, n0, tid, pre);
}

// Loaders for the spec kernel are built with THREADS = LW * kWave, the same LW
// for both.
template <class T, class ALoad, class BLoad, class Epi>
inline void launch_gemm_spec(const ALoad &al, const BLoad &bl, const Epi &epi, int M, int N, int K,
                             hipStream_t stream) {
    static_assert(ALoad::kWaves == BLoad::kWaves, "both loaders span the same loader waves");
    const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    hipLaunchKernelGGL((gemm_spec_kernel<T, ALoad, BLoad, Epi>), dim3(tiles_m * tiles_n),
                       dim3(T::kThreads + ALoad::kWaves * kWave), 0, stream, al, bl, epi, M, N,
                       K, tiles_n);
}

// ============================================ two independent GEMMs, one launch
// A GEMM (or implicit-GEMM conv) as a job of gemm_pair_kernel: the tile
// instance, its loaders and epilogue, on one of the three cores.
enum class GemmCore { kReg, kDma, kSpec };
template <GemmCore C, class T, class Epi>
constexpr size_t job_smem_bytes() {
    if constexpr (C == GemmCore::kReg) return reg_smem_bytes<T, Epi>();
    else return dma_smem_bytes<T, Epi>();
}
template <GemmCore C, class T, class ALoad>
constexpr int job_threads() {
    if constexpr (C == GemmCore::kSpec) return T::kThreads + ALoad::kWaves * kWave;
    else return T::kThreads;
}
template <GemmCore C, class T, class ALoad, class BLoad, class Epi>
struct GemmJob {
    static_assert(TileXcdRowGroups<T>::value == 0, "jobs use the default tile order");
    static constexpr size_t kSmem = job_smem_bytes<C, T, Epi>();
    static constexpr int kThreads = job_threads<C, T, ALoad>();
    ALoad al;
    BLoad bl;
    Epi epi;
    int M, N, K, tiles_n, tiles;
    // Tile `local` of this job (0 <= local < tiles), XCD-swizzled within it.
    __device__ void run(int local, unsigned char *smem) {
        const int pid = xcd_swizzle(local, tiles);
        if constexpr (C == GemmCore::kReg)
            gemm_reg_block<T>(al, bl, epi, M, N, K, tiles_n, pid, smem);
        else if constexpr (C == GemmCore::kDma)
            gemm_dma_block<T>(al, bl, epi, M, N, K, tiles_n, pid, smem);
        else
            gemm_spec_block<T>(al, bl, epi, M, N, K, tiles_n, pid, smem);
    }
};
template <GemmCore C, class T, class ALoad, class BLoad, class Epi>
GemmJob<C, T, ALoad, BLoad, Epi> gemm_job(const ALoad &al, const BLoad &bl, const Epi &epi, int M,
                                          int N, int K) {
    if constexpr (C == GemmCore::kSpec)
        static_assert(ALoad::kWaves == BLoad::kWaves, "both loaders span the same loader waves");
    const int tiles_n = (N + T::BN - 1) / T::BN;
    return GemmJob<C, T, ALoad, BLoad, Epi>{al, bl, epi, M, N, K, tiles_n,
                                            (M + T::BM - 1) / T::BM * tiles_n};
}

// Two GEMMs with no data dependence between them in one launch: workgroups
// [0, slots_a) run job A's tiles (slots_a is A's tile count rounded up to the
// 8 XCDs, so that B's tiles keep their XCD swizzle), the rest job B's.  Layers
// whose grids each leave most CUs idle for most of their time (a few hundred
// latency-bound tiles) then share the machine instead of running one after the
// other, and one launch boundary goes.  Both jobs run the same workgroup size;
// the branch is uniform per workgroup, and each job's barriers are its own.
template <class JA, class JB>
__global__ __launch_bounds__(JA::kThreads) void gemm_pair_kernel(JA a, JB b, int slots_a) {
    static_assert(JA::kThreads == JB::kThreads, "paired jobs run the same workgroup size");
    constexpr size_t kSmem = JA::kSmem > JB::kSmem ? JA::kSmem : JB::kSmem;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kSmem];
    const int bid = (int)blockIdx.x;
    if (bid < slots_a) {
        if (bid < a.tiles) a.run(bid, smem);
        return;
    }
    b.run(bid - slots_a, smem);
}

// One job alone, on its core's own kernel.
template <GemmCore C, class T, class ALoad, class BLoad, class Epi>
inline void launch_gemm_job(const GemmJob<C, T, ALoad, BLoad, Epi> &j, hipStream_t stream) {
    if constexpr (C == GemmCore::kReg)
        launch_gemm<T>(j.al, j.bl, j.epi, j.M, j.N, j.K, stream);
    else if constexpr (C == GemmCore::kDma)
        launch_gemm_dma<T>(j.al, j.bl, j.epi, j.M, j.N, j.K, stream);
    else
        launch_gemm_spec<T>(j.al, j.bl, j.epi, j.M, j.N, j.K, stream);
}

template <class JA, class JB>
inline void launch_gemm_pair(const JA &a, const JB &b, hipStream_t stream) {
    const int slots_a = (a.tiles + 7) / 8 * 8;
    hipLaunchKernelGGL((gemm_pair_kernel<JA, JB>), dim3(slots_a + b.tiles), dim3(JA::kThreads), 0,
                       stream, a, b, slots_a);
}

// ---------------------------------------------------------------- epilogues
// Each is called with the fragment origin (row, col) of four consecutive rows
// row..row+3 in one column; bounds are the epilogue's responsibility.

// Row-vector epilogues (kRowVector) work on quads of four consecutive columns:
// column(col) gathers the per-column state once, rows<R>(row0, step, c, v)
// then receives R rows row0 + i * step of that quad (rows ascending; bounds
// are the epilogue's responsibility).  Vector accesses need ld % 4 == 0 and
// 16-byte aligned bases, otherwise they fall back to scalars.
struct ColQuad {
    int col;
    float4 b;
};

__device__ __forceinline__ float4 load_quad(const float *p, int col, int n) {
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!p || col >= n) return r;
    if (col + 3 < n && ((uintptr_t)(p + col) & 15) == 0) return *reinterpret_cast<const float4 *>(p + col);
    r.x = p[col];
    if (col + 1 < n) r.y = p[col + 1];
    if (col + 2 < n) r.z = p[col + 2];
    if (col + 3 < n) r.w = p[col + 3];
    return r;
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

struct EpiRowsF32 {  // out[row*ld + col] = v (+bias) (ReLU)
    static constexpr bool kRowVector = true;
    float *out;
    const float *bias;
    int ld, M, N, relu;
    __device__ ColQuad column(int col) const { return ColQuad{col, load_quad(bias, col, N)}; }
    template <int R>
    __device__ void rows(int row0, int step, const ColQuad &c, const float4 (&v)[R]) const {
        if (c.col >= N) return;
        const bool vec = c.col + 3 < N && (ld & 3) == 0 && ((uintptr_t)out & 15) == 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            if (row >= M) break;
            float4 y = add4(v[i], c.b);
            if (relu) {  // NaN passes through, as in the reference's ReLU
                y.x = y.x < 0.f ? 0.f : y.x; y.y = y.y < 0.f ? 0.f : y.y;
                y.z = y.z < 0.f ? 0.f : y.z; y.w = y.w < 0.f ? 0.f : y.w;
            }
            float *p = out + (size_t)row * ld + c.col;
            if (vec) {
                *reinterpret_cast<float4 *>(p) = y;
            } else {
                const float t[4] = {y.x, y.y, y.z, y.w};
                for (int e = 0; e < 4 && c.col + e < N; ++e) p[e] = t[e];
            }
        }
    }
};

template <bool GELU>
struct EpiRowsF16 {  // out[row*ld + col] = fp16(act(v + bias)); ld % 4 == 0
    static constexpr bool kRowVector = true;
    bf16 *out;
    const float *bias;
    int ld, M, N;
    __device__ ColQuad column(int col) const { return ColQuad{col, load_quad(bias, col, N)}; }
    template <int R>
    __device__ void rows(int row0, int step, const ColQuad &c, const float4 (&v)[R]) const {
        if (c.col >= N) return;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            if (row >= M) break;
            const float4 y = add4(v[i], c.b);
            const float t[4] = {y.x, y.y, y.z, y.w};
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = to_half(GELU ? gelu(t[e]) : t[e]);
            bf16 *p = out + (size_t)row * ld + c.col;
            if (c.col + 3 < N) {
                *reinterpret_cast<bf16x4 *>(p) = o;
            } else {
                for (int e = 0; e < 4 && c.col + e < N; ++e) p[e] = o[e];
            }
        }
    }
};

struct EpiResidualF32 {  // x[row*ld + col] += v + bias; ld % 4 == 0, x 16-byte aligned
    static constexpr bool kRowVector = true;
    float *x;
    const float *bias;
    int ld, M, N;
    __device__ ColQuad column(int col) const { return ColQuad{col, load_quad(bias, col, N)}; }
    template <int R>
    __device__ void rows(int row0, int step, const ColQuad &c, const float4 (&v)[R]) const {
        if (c.col >= N) return;
        if (c.col + 3 < N) {
            float4 a[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int row = row0 + i * step;
                a[i] = row < M ? *reinterpret_cast<const float4 *>(x + (size_t)row * ld + c.col)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int row = row0 + i * step;
                if (row < M) *reinterpret_cast<float4 *>(x + (size_t)row * ld + c.col) = add4(a[i], add4(v[i], c.b));
            }
        } else {
            const float b[4] = {c.b.x, c.b.y, c.b.z, c.b.w};
            for (int i = 0; i < R; ++i) {
                const int row = row0 + i * step;
                if (row >= M) break;
                const float t[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
                float *p = x + (size_t)row * ld + c.col;
                for (int e = 0; e < 4 && c.col + e < N; ++e) p[e] = p[e] + (t[e] + b[e]);
            }
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
