// LayerNorm folded into the Swin linears (stages 1-3 and the patch merges).
//
// A linear that consumes LN(x) computes
//   y_j = sum_k ((x_k - mu) r g_k + beta_k) W_jk + b_j
//       = r (sum_k x_k W'_jk - mu c_j) + d_j,
//   W'_jk = g_k W_jk,  c_j = sum_k W'_jk,  d_j = b_j + sum_k beta_k W_jk,
// with mu and r = 1/sqrt(var + 1e-5) the row's statistics.  W' (fp16) and d
// are built once at create.  The GEMM runs on the residual stream itself,
// held as an fp16 copy xh next to the fp32 x, and the LayerNorm becomes fp32
// terms in the epilogue: no normalisation pass over x and no launch for it.
//
// The fp16 copy is centred per statistics group: the writer stores
// xh_k = fp16(x_k - m_g) with m_g the mean of the group g (64 channels) that
// holds k, so its rounding error scales with the group's spread, not with a
// common offset the row may carry (a row whose mean is 50x its standard
// deviation would otherwise lose ~50x the precision of fp16(LN(x))).  The
// consumer adds the group means back through per-group column sums:
//   sum_k x_k W'_jk - mu c_j = sum_k xh_k W'_jk + sum_g (m_g - mu) c_jg,
//   c_jg = sum over k in group g of W'_jk,
// with c_jg summed from the fp16-rounded W' the matrix cores multiply.
//
// The statistics come from the epilogue that writes x (the residual adds of
// proj and fc2, the patch-merge reduction): every 64-column group of a row
// leaves its own (mean, M2), M2 = sum of squared deviations from the group
// mean, computed two-pass over the group's fp32 values in registers.  The
// consumer combines a row's groups in a fixed order (Chan et al.'s pairwise
// update with equal counts):
//   mu = mean of the group means,  M2 = sum M2_g + 64 sum (mean_g - mu)^2,
//   var = M2 / n,
// so the result does not depend on which workgroup finished first.
#pragma once

#include "gemm_core.h"

namespace bfhip {

constexpr int kStatCols = 64;  // columns per statistics group

// One row's LayerNorm terms for a consumer over N statistics groups: the
// mean mu, r = 1/sqrt(var + 1e-5) and u_g = m_g - mu, the group means
// relative to the row mean (the centring correction above).
template <int N>
struct RowLn {
    static constexpr int kPad = (N + 3) / 4 * 4;  // u in whole 16-byte blocks
    float u[kPad];                                // zero past N
    float mean, r, unused[2];
};

// Combines equal-count (mean, M2) group partials of COLS columns each in
// index order into the row's RowLn; absent groups are passed as (0, 0).
template <int N, int COLS = kStatCols>
__device__ __forceinline__ RowLn<N> ln_combine(const float2 (&p)[N]) {
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < N; ++g) s += p[g].x;
    const float mean = s * (1.0f / N);
    float m2 = 0.0f, dev = 0.0f;
    RowLn<N> out{};
#pragma unroll
    for (int g = 0; g < N; ++g) {
        const float d = p[g].x - mean;
        m2 += p[g].y;
        dev += d * d;
        out.u[g] = d;
    }
    const float var = (m2 + (float)COLS * dev) * (1.0f / (COLS * N));
    out.mean = mean;
    out.r = rsqrtf(var + 1e-5f);
    return out;
}

// Statistics sources.  load(row) fetches a row's partials (issued at kernel
// start, so the loads overlap the main loop); finish() combines them.
// Row r of a stage's own tokens: stats[r * G + g].
template <int G>
struct LnRows {
    static constexpr int kGroups = G;
    struct Pre { float2 p[G]; };
    using Stat = RowLn<G>;
    const float2 *stats;
    __device__ Pre load(int row) const {
        Pre r;
        const float2 *p = stats + (size_t)row * G;
#pragma unroll
        for (int g = 0; g < G; ++g) r.p[g] = p[g];
        return r;
    }
    __device__ Stat finish(const Pre &r) const { return ln_combine(r.p); }
};

// Patch-merge row (n, oy, ox): its 2x2 source tokens of the previous stage
// ([B, H, W] tokens, G groups of COLS columns each), taps q = 2 dy + dx in
// order; a tap past an odd edge is a token of zeros (mean 0, M2 0), as the
// zero padding before the reference's unfold (swin_backbone.c:278-302).
// Group q * G + g covers folded columns q * C + g * COLS .. + COLS - 1.
template <int G, int COLS = kStatCols>
struct LnMerge {
    static constexpr int kGroups = 4 * G;
    struct Pre { float2 p[4 * G]; };
    using Stat = RowLn<4 * G>;
    const float2 *stats;
    int H, W;
    __device__ Pre load(int m) const {
        const int H2 = (H + 1) / 2, W2 = (W + 1) / 2;
        const int n = m / (H2 * W2), p = m - n * (H2 * W2), oy = p / W2, ox = p - oy * W2;
        Pre r;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sy = 2 * oy + (q >> 1), sx = 2 * ox + (q & 1);
            const bool in = sy < H && sx < W;
            const float2 *src = stats + (((size_t)n * H + (in ? sy : 0)) * W + (in ? sx : 0)) * G;
#pragma unroll
            for (int g = 0; g < G; ++g) r.p[q * G + g] = in ? src[g] : make_float2(0.0f, 0.0f);
        }
        return r;
    }
    __device__ Stat finish(const Pre &r) const { return ln_combine<4 * G, COLS>(r.p); }
};

struct LnNone {  // producers that take no LayerNorm on their input
    static constexpr int kGroups = 1;
    struct Pre {};
    using Stat = RowLn<1>;
    __device__ Pre load(int) const { return Pre{}; }
    __device__ Stat finish(const Pre &) const { return Stat{}; }
};

// Sum over each DPP row of 16 lanes, returned to every lane of the row:
// butterflies within quads (quad_perm), then rotations by 4 and 8 lanes
// (row_ror).  All in registers; deterministic for a given lane.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF,
                                                                0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp_mov<0x124>(v);  // row_ror:4
    v += dpp_mov<0x128>(v);  // row_ror:8
    return v;
}

// The centring correction on the matrix cores (the GEMM core's kCorrSteps):
// k-slots 2g and 2g + 1 of a row hold u_g split into two fp16 words
// (hi = fp16(u_g), lo = fp16(u_g - hi), so hi + lo carries u_g to ~22 bits;
// the core builds them from corr_u4), and both slots of column j hold
// fp16(c_jg); the table `corr` is [N][steps * 32] fp16 words, zero past 2 NG.
// The product is added to the accumulators before the epilogue, which then
// applies r acc + d.
template <int NG>
struct LnCorr {
    static constexpr int kSteps = (2 * NG + 31) / 32;
};

// u of groups 4q .. 4q + 3 (zero past NG): the groups behind k-slots
// 8q .. 8q + 7 of the correction operand.
template <int NG>
__device__ __forceinline__ float4 ln_corr_u4(const RowLn<NG> &st, int q) {
    constexpr int kBlocks = RowLn<NG>::kPad / 4;
    const float4 v = reinterpret_cast<const float4 *>(st.u)[q < kBlocks ? q : kBlocks - 1];
    return q < kBlocks ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ bf16x8 ln_corr_col(const bf16 *corr, int steps, int col, int N, int k0) {
    return col < N ? *reinterpret_cast<const bf16x8 *>(corr + (size_t)col * steps * 32 + k0) : bf16x8{};
}

// A column quad's shift (bias or folded d).
struct LnCol {
    int col;
    float4 d;
};

// r acc + d: acc already holds the centring correction.
template <int NG>
__device__ __forceinline__ float4 ln_apply(float4 v, const RowLn<NG> &st, const LnCol &c) {
    return make_float4(fmaf(st.r, v.x, c.d.x), fmaf(st.r, v.y, c.d.y), fmaf(st.r, v.z, c.d.z),
                       fmaf(st.r, v.w, c.d.w));
}

__device__ __forceinline__ void store_half4(bf16 *p, float4 y) {
    bf16x4 o;
    o[0] = to_half(y.x); o[1] = to_half(y.y); o[2] = to_half(y.z); o[3] = to_half(y.w);
    *reinterpret_cast<bf16x4 *>(p) = o;
}

// Writer of the residual stream: y = [LN-folded] acc + shift [+ x], stored as
// fp32 x, the centred fp16 copy xh = fp16(y - m_g), and per-64-column
// (m_g, M2_g) of y.  x, xh: [M, N] row-major; stats: [M, N / 64].  N % 64 ==
// 0 and 16-byte aligned buffers (host-checked); a tile's column quads of one
// 64-column group are 16 consecutive lanes, which reduce the group with
// cross-lane sums.
template <bool kLnIn, bool kResidual, class Src = LnNone>
struct EpiStatsRows {
    static constexpr bool kRowVector = true;
    static constexpr bool kRowStat = kLnIn;
    static constexpr bool kQuadRows = true;  // row16_sum over each 64-column group
    static constexpr int NG = Src::kGroups;
    static constexpr int kCorrSteps = kLnIn ? LnCorr<NG>::kSteps : 0;
    float *x;
    bf16 *xh;
    float2 *stats;
    const float *shift;  // bias (may be null), or the folded d with kLnIn
    const bf16 *corr;    // centring-correction table (kLnIn; LnCorr)
    Src src;             // row statistics of the LayerNorm input (kLnIn)
    int M, N;
    __device__ LnCol column(int col) const { return LnCol{col, load_quad(shift, col, N)}; }
    using Pre = typename Src::Pre;
    using Stat = typename Src::Stat;
    __device__ Pre stat_load(int row) const { return row < M ? src.load(row) : Pre{}; }
    __device__ Stat stat_finish(const Pre &p) const { return src.finish(p); }
    __device__ float4 corr_u4(const Stat &st, int q) const { return ln_corr_u4(st, q); }
    __device__ bf16x8 corr_col(int col, int k0) const {
        return ln_corr_col(corr, LnCorr<NG>::kSteps, col, N, k0);
    }
    template <int R>
    __device__ void rows(int row0, int step, const LnCol &c, const float4 (&v)[R],
                         const Stat *st = nullptr) const {
        if (c.col >= N) return;  // whole 64-column groups: uniform over the 16 lanes
        float4 y[R];
        if constexpr (kResidual) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int row = row0 + i * step;
                y[i] = row < M ? *reinterpret_cast<const float4 *>(x + (size_t)row * N + c.col)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const float4 t = kLnIn ? ln_apply(v[i], st[i * step], c) : add4(v[i], c.d);
            y[i] = kResidual ? add4(y[i], t) : t;
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            const float mean = row16_sum((y[i].x + y[i].y) + (y[i].z + y[i].w)) * (1.0f / kStatCols);
            const float a = y[i].x - mean, b = y[i].y - mean, cc = y[i].z - mean, d = y[i].w - mean;
            const float m2 = row16_sum((a * a + b * b) + (cc * cc + d * d));
            if (row < M) {
                *reinterpret_cast<float4 *>(x + (size_t)row * N + c.col) = y[i];
                store_half4(xh + (size_t)row * N + c.col, make_float4(a, b, cc, d));
                if ((c.col & (kStatCols - 1)) == 0)
                    stats[(size_t)row * (N / kStatCols) + c.col / kStatCols] = make_float2(mean, m2);
            }
        }
    }
};

// Reader of LN(x): out = fp16(act(r (acc + sum_g u_g c_jg) + d)) for the QKV
// (no activation) and fc1 (GELU) linears over the centred copy, the sum added
// on the matrix cores (kCorrSteps).  ld % 4 == 0, N % 4 == 0.
template <bool GELU, class Src>
struct EpiLnF16 {
    static constexpr bool kRowVector = true;
    static constexpr bool kRowStat = true;
    static constexpr int NG = Src::kGroups;
    static constexpr int kCorrSteps = LnCorr<NG>::kSteps;
    bf16 *out;
    const float *shift;
    const bf16 *corr;  // centring-correction table (LnCorr)
    Src src;
    int ld, M, N;
    __device__ LnCol column(int col) const { return LnCol{col, load_quad(shift, col, N)}; }
    using Pre = typename Src::Pre;
    using Stat = typename Src::Stat;
    __device__ Pre stat_load(int row) const { return row < M ? src.load(row) : Pre{}; }
    __device__ Stat stat_finish(const Pre &p) const { return src.finish(p); }
    __device__ float4 corr_u4(const Stat &st, int q) const { return ln_corr_u4(st, q); }
    __device__ bf16x8 corr_col(int col, int k0) const {
        return ln_corr_col(corr, LnCorr<NG>::kSteps, col, N, k0);
    }
    template <int R>
    __device__ void rows(int row0, int step, const LnCol &c, const float4 (&v)[R],
                         const Stat *st) const {
        if (c.col >= N) return;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            if (row >= M) break;
            float4 y = ln_apply(v[i], st[i * step], c);
            if (GELU) y = make_float4(gelu(y.x), gelu(y.y), gelu(y.z), gelu(y.w));
            store_half4(out + (size_t)row * ld + c.col, y);
        }
    }
};

// Patch embedding output over whole 96-channel rows: x = LN_p(acc + b) (the
// patch norm, reference swin_backbone.c patch embed) and xn = fp16(LN_1(x))
// (block 0's norm1), both two-pass fp32, eps 1e-5.  Two threads per row, 48
// channels each, normalise in registers and put the rows back into the
// staged tile; the tile's rows are one contiguous block of x (and of xn), so
// all threads then store it as consecutive 16-byte vectors.
struct EpiPatchNorms {
    static constexpr bool kRowVector = true;
    static constexpr bool kFullRow = true;
    static constexpr int C = 96, kHalf = 48;
    float *x;
    bf16 *xn;
    const float *bias, *g0, *b0, *g1, *b1;
    int M;
    static constexpr int kTileBarriers = 3;  // tile() synchronises three times
    template <class T>
    __device__ void tile(float *sC, int stride, int m0, int, int tid) const {
        static_assert(T::BN == C && T::kThreads == 2 * T::BM, "two threads per 96-channel row");
        const int r = tid >> 1, h = tid & 1, c0 = h * kHalf;
        float *rowp = sC + r * stride + c0;
        float v[kHalf];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < kHalf; i += 4) {
            const float4 a = *reinterpret_cast<const float4 *>(rowp + i);
            const float4 b = *reinterpret_cast<const float4 *>(bias + c0 + i);
            v[i] = a.x + b.x; v[i + 1] = a.y + b.y; v[i + 2] = a.z + b.z; v[i + 3] = a.w + b.w;
            s += (v[i] + v[i + 1]) + (v[i + 2] + v[i + 3]);
        }
        normalise(v, s, g0, b0, c0);
        // x rows back into the tile, then LN1 of them in place (one row half
        // of registers live instead of two).
        s = 0.0f;
#pragma unroll
        for (int i = 0; i < kHalf; ++i) s += v[i];
#pragma unroll
        for (int i = 0; i < kHalf; i += 4)
            *reinterpret_cast<float4 *>(rowp + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
        normalise(v, s, g1, b1, c0);
        lds_barrier();
        const int rows = min(T::BM, M - m0);
        float *xo = x + (size_t)m0 * C;
        for (int q = tid; q < rows * (C / 4); q += T::kThreads) {
            const int rr = q / (C / 4), cq = q - rr * (C / 4);
            *reinterpret_cast<float4 *>(xo + (size_t)q * 4) =
                *reinterpret_cast<const float4 *>(sC + rr * stride + cq * 4);
        }
        lds_barrier();
        // LN1 rows into the tile as fp16 words (row stride `stride` floats).
        bf16 *hrow = reinterpret_cast<bf16 *>(sC + r * stride) + c0;
#pragma unroll
        for (int i = 0; i < kHalf; i += 8) {
            bf16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = to_half(v[i + e]);
            *reinterpret_cast<bf16x8 *>(hrow + i) = o;
        }
        lds_barrier();
        bf16 *xno = xn + (size_t)m0 * C;
        for (int q = tid; q < rows * (C / 8); q += T::kThreads) {
            const int rr = q / (C / 8), cq = q - rr * (C / 8);
            *reinterpret_cast<bf16x8 *>(xno + (size_t)q * 8) =
                *reinterpret_cast<const bf16x8 *>(reinterpret_cast<const bf16 *>(sC + rr * stride) + cq * 8);
        }
    }

private:
    // v <- LN(v) * g + b over the row split across the lane pair (s: this
    // lane's partial sum of v).
    __device__ static void normalise(float (&v)[kHalf], float s, const float *g, const float *b,
                                     int c0) {
        const float mean = (s + __shfl_xor(s, 1)) * (1.0f / C);
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < kHalf; ++i) q += (v[i] - mean) * (v[i] - mean);
        const float rstd = rsqrtf((q + __shfl_xor(q, 1)) * (1.0f / C) + 1e-5f);
#pragma unroll
        for (int i = 0; i < kHalf; i += 4) {
            const float4 gg = *reinterpret_cast<const float4 *>(g + c0 + i);
            const float4 bb = *reinterpret_cast<const float4 *>(b + c0 + i);
            v[i] = (v[i] - mean) * rstd * gg.x + bb.x;
            v[i + 1] = (v[i + 1] - mean) * rstd * gg.y + bb.y;
            v[i + 2] = (v[i + 2] - mean) * rstd * gg.z + bb.z;
            v[i + 3] = (v[i + 3] - mean) * rstd * gg.w + bb.w;
        }
    }
};

// Patch-merge A operand gathered from the previous stage's fp16 tokens
// xh[B, H, W, C]: merged row m = (n, oy, ox) is the concatenation of its four
// 2x2 tokens, tap q = 2 dy + dx at k = q*C + c.  (The reference's unfold
// orders the row c*4 + q, swin_backbone.c:287-296; the reduction weights'
// columns are permuted to this order at create, which leaves the product
// unchanged.)  Taps past an odd edge and rows past the last read as zero.
// The LDS image and its swizzle are those of DmaRowsBf16; every 16-byte chunk
// lies inside one tap because C % 8 == 0.
template <int ROWS, int BK, int THREADS, int C>
struct DmaMergeRows {
    static constexpr int kCpr = BK / 8, kWaves = THREADS / kWave;
    static constexpr int kChunks = ROWS * kCpr;
    static_assert(kChunks % (kWave * kWaves) == 0, "tile must split evenly over the waves");
    static_assert(C % 8 == 0, "taps must hold whole 16-byte chunks");
    static constexpr int kIssue = kChunks / (kWave * kWaves);
    const bf16 *base;
    int batches, H, W;
    int wave;
    int tok[kIssue];   // token of tap 0, or -1 for a row past the last
    int taps[kIssue];  // bit q: tap q lies inside the image
    int kcol[kIssue];

    __device__ void setup(int r0, int tid) {
        wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        const int lane = tid % kWave;
        const int H2 = (H + 1) / 2, W2 = (W + 1) / 2, rows = batches * H2 * W2;
#pragma unroll
        for (int j = 0; j < kIssue; ++j) {
            const int q = (j * kWaves + wave) * kWave + lane;
            const int r = q / kCpr, slot = q % kCpr, m = r0 + r;
            kcol[j] = 8 * (slot ^ dma_swizzle<BK>(r));
            tok[j] = -1;
            taps[j] = 0;
            if (m < rows) {
                const int n = m / (H2 * W2), p = m - n * (H2 * W2), oy = p / W2, ox = p - oy * W2;
                tok[j] = (n * H + 2 * oy) * W + 2 * ox;
                const bool dx = 2 * ox + 1 < W, dy = 2 * oy + 1 < H;
                taps[j] = 1 | (dx ? 2 : 0) | (dy ? 4 : 0) | (dx && dy ? 8 : 0);
            }
        }
    }
    __device__ void issue(bf16 *lds, int k0) const {
        const __amdgpu_buffer_rsrc_t rsrc =
            buffer_rsrc(base, (uint32_t)batches * (uint32_t)H * (uint32_t)W * (uint32_t)C * 2u);
#pragma unroll
        for (int j = 0; j < kIssue; ++j) {
            const int k = k0 + kcol[j], q = k / C, c = k - q * C;
            const bool in = k < 4 * C && ((taps[j] >> q) & 1);
            const uint32_t off =
                in ? (uint32_t)((tok[j] + (q >> 1) * W + (q & 1)) * C + c) * 2u : kDmaOutOfRange;
            dma16(rsrc, lds + (j * kWaves + wave) * kWave * 8, off);
        }
    }
};

}  // namespace bfhip
