// Implicit-GEMM NCHW convolution operands for the MFMA GEMM core.
//
// GEMM view (same index map as reference src/cuda_ops.cu:23-69):
//   row m = n*OH*OW + oy*OW + ox           (output pixel)
//   red k = ci*KH*KW + ky*KW + kx          (input channel, tap)
//   col   = output channel
//   direct:     iy = oy*SH - PH + ky, ix = ox*SW - PW + kx
//   transposed: sy = oy + PH - ky, sx = ox + PW - kx; a tap exists only when
//               sy, sx >= 0 and divisible by the stride; iy = sy/SH, ix = sx/SW
//   taps outside [0,IH) x [0,IW) read zero.
// No im2col buffer exists: each thread owns one output pixel of the tile and
// gathers a run of consecutive k, so for every k the 64 lanes of a wave read
// 64 consecutive pixels of one input plane.
#pragma once

#include "gemm_core.h"

namespace bfhip {

struct ConvGeom {
    int N, Ci, IH, IW, OH, OW, KH, KW, SH, SW, PH, PW, transpose;
    int M, K;  // N*OH*OW, Ci*KH*KW
};

// ----------------------------------------------------------------- sources
// A source returns input value (n, c, iy, ix) for an in-bounds tap; prepare()
// sees the output pixel a thread owns before any load.  The NCHW gather below
// serves the stateless fp32 ABI; the contexts use the channels-last path at
// the end of this file.
struct SrcNCHW {
    const float *x;
    int C, H, W;
    __device__ void prepare(int, int, int) {}
    __device__ float operator()(int n, int c, int iy, int ix) const {
        return x[(((size_t)n * C + c) * H + iy) * W + ix];
    }
};

// ----------------------------------------------------------------- A loader
// KH/KW > 0 fix the kernel size at compile time; 0 means runtime geometry.
// F16 stages fp16 words instead of bf16 (for an fp16 tile).
template <int BM, int BK, int THREADS, int KH_, int KW_, class Src, bool F16 = false>
struct LoadConvA {
    static constexpr int kGroups = THREADS / BM;
    static constexpr int kPer = BK / kGroups;
    static_assert(THREADS % BM == 0, "one pixel per thread group");
    static_assert(kPer % 8 == 0, "each thread fills whole 16-byte chunks");
    Src src;
    ConvGeom g;
    int row, kg, n, iy0, ix0, oy, ox;
    bool ok;
    bf16 st[kPer];

    __device__ int kh() const { return KH_ ? KH_ : g.KH; }
    __device__ int kw() const { return KW_ ? KW_ : g.KW; }

    __device__ void setup(int m0, int tid) {
        row = tid % BM;
        kg = tid / BM;
        const int m = m0 + row;
        ok = m < g.M;
        const int ohw = g.OH * g.OW;
        const int mm = ok ? m : 0;
        n = mm / ohw;
        const int p = mm - n * ohw;
        oy = p / g.OW;
        ox = p - oy * g.OW;
        iy0 = oy * g.SH - g.PH;
        ix0 = ox * g.SW - g.PW;
        src.prepare(n, oy, ox);
    }

    __device__ void load(int k0) {
        int k = k0 + kg * kPer;
        const int KHW = kh() * kw();
        int ci = k / KHW, r = k - ci * KHW;
        int ky = r / kw(), kx = r - ky * kw();
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            float v = 0.0f;
            if (ok && k + e < g.K) {
                int iy, ix;
                bool tap = true;
                if (g.transpose) {
                    const int sy = oy + g.PH - ky, sx = ox + g.PW - kx;
                    tap = sy >= 0 && sx >= 0 && sy % g.SH == 0 && sx % g.SW == 0;
                    iy = tap ? sy / g.SH : -1;
                    ix = tap ? sx / g.SW : -1;
                } else {
                    iy = iy0 + ky;
                    ix = ix0 + kx;
                }
                if (tap && (unsigned)iy < (unsigned)g.IH && (unsigned)ix < (unsigned)g.IW)
                    v = src(n, ci, iy, ix);
            }
            st[e] = to_word(v, F16);
            if (++kx == kw()) {
                kx = 0;
                if (++ky == kh()) {
                    ky = 0;
                    ++ci;
                }
            }
        }
    }

    __device__ void store(bf16 *lds) const {
        bf16 *dst = lds + row * (BK + 8) + kg * kPer;
#pragma unroll
        for (int c = 0; c < kPer; c += 8) {
            bf16x8 v;
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = st[c + e];
            *reinterpret_cast<bf16x8 *>(dst + c) = v;
        }
    }
};

// A operand of a 4x4 / stride-4 / unpadded conv (the Swin patch embedding)
// from fp32 NCHW input: for a fixed (channel, ky) the four kx taps are four
// consecutive floats, so each thread fetches its k-run as float4s, and the
// lanes of a wave (consecutive output pixels ox) read 64 consecutive float4s
// of one image row.  Requires IW % 4 == 0, a 16-byte aligned base and the
// k order ci*16 + ky*4 + kx of LoadConvA.
template <int BM, int BK, int THREADS, bool F16 = false>
struct LoadPatch4x4 {
    static constexpr int kGroups = THREADS / BM;
    static constexpr int kPer = BK / kGroups;
    static_assert(THREADS % BM == 0 && kPer % 8 == 0, "whole 16-byte chunks per thread");
    const float *x;
    ConvGeom g;
    int row, kg;
    const float *pix;  // image n, row 4*oy, column 4*ox, channel 0
    bool ok;
    float4 raw[kPer / 4];  // fetched by load(), converted by store()
    bool val[kPer / 4];

    __device__ void setup(int m0, int tid) {
        row = tid % BM;
        kg = tid / BM;
        const int m = m0 + row, ohw = g.OH * g.OW;
        ok = m < g.M;
        const int mm = ok ? m : 0, n = mm / ohw, p = mm - n * ohw, oy = p / g.OW, ox = p - oy * g.OW;
        pix = x + (((size_t)n * g.Ci) * g.IH + 4 * oy) * g.IW + 4 * ox;
    }
    // Every float4 is read (an element past K or past the last row reads the
    // pixel's channel-0 run) before any is used; store() converts and zeroes,
    // so the reads stay in flight across the caller's MFMAs.
    __device__ void load(int k0) {
        const int k = k0 + kg * kPer;
#pragma unroll
        for (int q = 0; q < kPer; q += 4) {
            const int kk = k + q, ci = kk >> 4, ky = (kk >> 2) & 3;
            val[q / 4] = ok && kk < g.K;
            raw[q / 4] = *reinterpret_cast<const float4 *>(
                pix + (val[q / 4] ? ((size_t)ci * g.IH + ky) * g.IW : 0));
        }
    }
    __device__ void store(bf16 *lds) const {
        bf16 *dst = lds + row * (BK + 8) + kg * kPer;
#pragma unroll
        for (int c = 0; c < kPer; c += 8) {
            bf16x8 v;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4 f = val[c / 4 + h] ? raw[c / 4 + h] : make_float4(0.f, 0.f, 0.f, 0.f);
                v[4 * h + 0] = to_word(f.x, F16); v[4 * h + 1] = to_word(f.y, F16);
                v[4 * h + 2] = to_word(f.z, F16); v[4 * h + 3] = to_word(f.w, F16);
            }
            *reinterpret_cast<bf16x8 *>(dst + c) = v;
        }
    }
};

// Transposed-convolution weights are IOHW: B[co][k] = W[ci][co][ky][kx].
template <int ROWS, int BK, int THREADS>
struct LoadWeightIOHW {
    static constexpr int kPerRow = BK / 8;
    static constexpr int kChunks = ROWS * kPerRow;
    static constexpr int kPer = (kChunks + THREADS - 1) / THREADS;
    const float *w;
    int Co, K, KHW;
    int r0, tid;
    bf16x8 st[kPer];
    __device__ void setup(int origin, int t) { r0 = origin; tid = t; }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int c = tid + p * THREADS;
            const int co = r0 + c / kPerRow, gk = k0 + (c % kPerRow) * 8;
            bf16x8 v = {};
            if (c < kChunks && co < Co)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int k = gk + e;
                    if (k < K) {
                        const int ci = k / KHW, kk = k - ci * KHW;
                        v[e] = to_bf16(w[((size_t)ci * Co + co) * KHW + kk]);
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

// ----------------------------------------------------------- conv epilogues
// Final 1x1 of the depth head: channels [0,118) are depth logits, [118,198)
// context, both NCHW (reference split_depth_kernel, cuda_camera.cu:255-263).
struct EpiSplitDepth {
    static constexpr bool kRowVector = true;
    static constexpr bool kFullRow = true;
    float *logits, *context;
    const float *bias;
    int M, ohw, bins, ctx;
    // The staged fp32 tile is read column by column: consecutive threads take
    // consecutive 4-pixel quads of one channel, so a wave writes 16-byte
    // vectors in runs of BM/4 along a channel plane.
    template <class T>
    __device__ void tile(float *sC, int stride, int m0, int n0, int tid) const {
        constexpr int kQuads = T::BM / 4;
        for (int item = tid; item < T::BN * kQuads; item += T::kThreads) {
            const int c = item / kQuads, q = item - c * kQuads;
            const int col = n0 + c, row = m0 + 4 * q;
            if (col >= bins + ctx || row >= M) continue;
            const float b = bias[col];
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = sC[(4 * q + r) * stride + c] + b;
            const bool lo = col < bins;
            float *base = lo ? logits + (size_t)col * ohw : context + (size_t)(col - bins) * ohw;
            const int planes = lo ? bins : ctx;
            const int n = row / ohw, p = row - n * ohw;
            float *dst = base + (size_t)n * planes * ohw + p;
            if (row + 3 < M && p + 3 < ohw && ((uintptr_t)dst & 15) == 0) {
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = row + r;
                    if (rr >= M) break;
                    const int nn = rr / ohw, pp = rr - nn * ohw;
                    base[(size_t)nn * planes * ohw + pp] = v[r];
                }
            }
        }
    }
};

// Channel planes out[n][c][p] = relu(v + bias[c]) for GEMM row n*HW + p: the
// staged fp32 tile is read column by column, consecutive threads taking
// consecutive 4-row quads of one channel, so a wave writes 16-byte vectors in
// runs of BM/4 along a plane.  With rows in YFAST order this stores the x/y-
// transposed map of the last downsample conv (below) contiguously.
struct EpiPlanesNCHW {
    static constexpr bool kRowVector = true;
    static constexpr bool kFullRow = true;
    float *out;
    const float *bias;
    int M, C, hw;
    template <class T>
    __device__ void tile(float *sC, int stride, int m0, int n0, int tid) const {
        constexpr int kQuads = T::BM / 4;
        for (int item = tid; item < T::BN * kQuads; item += T::kThreads) {
            const int c = item / kQuads, q = item - c * kQuads;
            const int col = n0 + c, row = m0 + 4 * q;
            if (col >= C || row >= M) continue;
            const float b = bias[col];
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float o = sC[(4 * q + r) * stride + c] + b;
                v[r] = o > 0.0f ? o : 0.0f;
            }
            const int n = row / hw, p = row - n * hw;
            float *dst = out + ((size_t)n * C + col) * hw + p;
            if (row + 3 < M && p + 3 < hw && ((uintptr_t)dst & 15) == 0) {
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = row + r;
                    if (rr >= M) break;
                    const int nn = rr / hw, pp = rr - nn * hw;
                    out[((size_t)nn * C + col) * hw + pp] = v[r];
                }
            }
        }
    }
};


}  // namespace bfhip

namespace bfhip {

// ======================================================================
// Channels-last implicit GEMM.  Reduction order is k = (ky*KW + kx)*Ci + ci,
// so eight consecutive k are eight channels of one input pixel: one 16-byte
// load per chunk instead of eight scalar gathers.  Every source below keeps
// its channel count a multiple of 8.  Weights are stored [Co][KH][KW][Ci].
// ======================================================================

// Plain NHWC bf16 map x[n][iy][ix][C].
struct SrcNHWC {
    const bf16 *x;
    int C, H, W;
    struct Row {};
    using Raw = bf16x8;
    __device__ Row row(int, int, int) const { return {}; }
    __device__ Raw fetch(const Row &, int n, int iy, int ix, int c0) const {
        return *reinterpret_cast<const bf16x8 *>(x + (((size_t)n * H + iy) * W + ix) * C + c0);
    }
    __device__ bf16x8 finish(const Raw &r) const { return r; }
};

// Channel concat of two NHWC maps of the same size: [0,C0) from a, rest from b.
struct SrcNHWCConcat {
    const bf16 *a, *b;
    int C0, C1, H, W;
    struct Row {};
    using Raw = bf16x8;
    __device__ Row row(int, int, int) const { return {}; }
    __device__ Raw fetch(const Row &, int n, int iy, int ix, int c0) const {
        const size_t pix = ((size_t)n * H + iy) * W + ix;
        return c0 < C0 ? *reinterpret_cast<const bf16x8 *>(a + pix * C0 + c0)
                       : *reinterpret_cast<const bf16x8 *>(b + pix * C1 + (c0 - C0));
    }
    __device__ bf16x8 finish(const Raw &r) const { return r; }
};

// dtransform.0 fused into dtransform.3's gather: the 8 virtual channels of tap
// (iy, ix) are relu(depth*w[c] + b[c]) from one fp32 depth value, as fp16
// words when F16 is set, else bf16.
template <bool F16 = false>
struct SrcNHWCDepthAffine {
    const float *depth;
    const float *w, *b;
    int H, W;
    struct Row {};
    using Raw = float;
    __device__ Row row(int, int, int) const { return {}; }
    __device__ Raw fetch(const Row &, int n, int iy, int ix, int) const {
        return depth[((size_t)n * H + iy) * W + ix];
    }
    __device__ bf16x8 finish(const Raw &d) const {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = fmaf(d, w[e], 0.0f) + b[e];
            o[e] = to_word(v > 0.0f ? v : 0.0f, F16);
        }
        return o;
    }
};

template <int BM, int BK, int THREADS, int KH, int KW, class Src>
struct LoadConvNHWC {
    static constexpr int kPerRow = BK / 8;
    static constexpr int kChunks = BM * kPerRow;
    static constexpr int kPer = kChunks / THREADS;
    static constexpr int kRowStep = THREADS / kPerRow;
    static_assert(kChunks % THREADS == 0 && THREADS % kPerRow == 0, "tile/thread mismatch");
    Src src;
    ConvGeom g;
    int tid, cc;
    int n[kPer], iy0[kPer], ix0[kPer];
    bool ok[kPer];
    typename Src::Row rs[kPer];
    typename Src::Raw raw[kPer];  // fetched by load(), finished by store()
    bool val[kPer];

    __device__ void setup(int m0, int t) {
        tid = t;
        cc = t % kPerRow;
        const int ohw = g.OH * g.OW;
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int m = m0 + t / kPerRow + p * kRowStep;
            ok[p] = m < g.M;
            const int mm = ok[p] ? m : 0;
            n[p] = mm / ohw;
            const int q = mm - n[p] * ohw, oy = q / g.OW, ox = q - oy * g.OW;
            iy0[p] = oy * g.SH - g.PH;
            ix0[p] = ox * g.SW - g.PW;
            rs[p] = src.row(n[p], oy, ox);
        }
    }
    __device__ void load(int k0) {
        const int k = k0 + cc * 8;
        const bool kin = k < g.K;
        const int tap = kin ? k / g.Ci : 0, c0 = k - tap * g.Ci;
        const int ky = tap / KW, kx = tap - ky * KW;
        // Every chunk's read is issued (a zero tap reads pixel (n, 0, 0)
        // channel 0); store() applies the source's transform and the zeros,
        // so no read waits inside load().
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int iy = iy0[p] + ky, ix = ix0[p] + kx;
            val[p] = kin && ok[p] && (unsigned)iy < (unsigned)g.IH && (unsigned)ix < (unsigned)g.IW;
            raw[p] = src.fetch(rs[p], n[p], val[p] ? iy : 0, val[p] ? ix : 0, val[p] ? c0 : 0);
        }
    }
    __device__ void store(bf16 *lds) const {
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const bf16x8 zero = {};
            *reinterpret_cast<bf16x8 *>(lds + (tid / kPerRow + p * kRowStep) * (BK + 8) + cc * 8) =
                val[p] ? src.finish(raw[p]) : zero;
        }
    }
};

// LDS-DMA gather of channels-last taps for DmaTile pipelines: the A operand of
// a conv over one NHWC map, or over the channel concat of two maps of the same
// size (channels [0, C0) from a, [C0, C0 + C1) from b).  C0 and C1 are
// multiples of BK, so one k-tile lies inside one tap of one source: the tap
// and the source are uniform per stage and each lane moves one 16-byte chunk
// of 8 channels.  Taps outside the map read as zero through an out-of-range
// buffer offset.  Each source must span < 2 GiB.
//
// The lane's offset depends on the tap and the source only; it is computed
// when they change (every C/BK k-tiles) and the channel offset within the
// source rides in soffset, so most k-tiles issue with no vector arithmetic.
// YFAST orders the GEMM rows of each image column-major over output pixels
// (row = n*OH*OW + ox*OH + oy), so a store in row order writes an x/y-
// transposed map contiguously.
template <int ROWS, int BK, int THREADS, int KH, int KW, bool YFAST = false>
struct DmaConvNHWC {
    static constexpr int kCpr = BK / 8, kWaves = THREADS / kWave;
    static constexpr int kChunks = ROWS * kCpr;
    static_assert(kChunks % (kWave * kWaves) == 0, "tile must split evenly over the waves");
    static constexpr int kIssue = kChunks / (kWave * kWaves);
    const bf16 *a, *b;
    int C0, C1;
    ConvGeom g;
    int wave;         // wave-uniform (SGPR)
    int pix[kIssue];  // n * IH * IW of the lane's output pixel, or -1 past M
    int iy0[kIssue], ix0[kIssue];
    int cofs[kIssue];  // channel offset of the lane's chunk within the k-tile
    // Cache: tap and source of the offsets below (-1: none yet).
    int cached;
    uint32_t voff[kIssue];

    __device__ void setup(int m0, int tid) {
        wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        cached = -1;
        const int lane = tid % kWave, ohw = g.OH * g.OW;
#pragma unroll
        for (int j = 0; j < kIssue; ++j) {
            const int q = (j * kWaves + wave) * kWave + lane;
            const int r = q / kCpr, slot = q % kCpr, m = m0 + r;
            const int mm = m < g.M ? m : 0;
            const int n = mm / ohw, p = mm - n * ohw;
            const int oy = YFAST ? p % g.OH : p / g.OW, ox = YFAST ? p / g.OH : p % g.OW;
            pix[j] = m < g.M ? n * g.IH * g.IW : -1;
            iy0[j] = oy * g.SH - g.PH;
            ix0[j] = ox * g.SW - g.PW;
            cofs[j] = 8 * (slot ^ dma_swizzle<BK>(r));
        }
    }
    __device__ void issue(bf16 *lds, int k0) {
        const int ci = C0 + C1, tap = k0 / ci, cb = k0 - tap * ci;
        const bool hi = cb >= C0;
        const int cs = hi ? C1 : C0, c0 = hi ? cb - C0 : cb;
        const int key = 2 * tap + (hi ? 1 : 0);
        if (key != cached) {  // wave-uniform
            cached = key;
            const int ky = tap / KW, kx = tap - ky * KW;
#pragma unroll
            for (int j = 0; j < kIssue; ++j) {
                const int iy = iy0[j] + ky, ix = ix0[j] + kx;
                const bool in = pix[j] >= 0 && (unsigned)iy < (unsigned)g.IH && (unsigned)ix < (unsigned)g.IW;
                voff[j] = in ? (uint32_t)(((pix[j] + iy * g.IW + ix) * cs + cofs[j]) * 2) : kDmaOutOfRange;
            }
        }
        const uint32_t pixels = (uint32_t)g.N * g.IH * g.IW;
        const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(hi ? b : a, pixels * (uint32_t)cs * 2u);
#pragma unroll
        for (int j = 0; j < kIssue; ++j)
            dma16(rsrc, lds + (j * kWaves + wave) * kWave * 8, voff[j], 2u * (uint32_t)c0);
    }
};

// Row-vector conv epilogue for channels-last 16-bit maps: out[row * ld + col] =
// word(relu(v + bias)) for col < Co, Co % 4 == 0, ld >= Co a multiple of 4
// (a row stride above Co leaves the channels past Co untouched); words are
// bf16, or fp16 when f16 is set.
struct EpiConvNHWC {
    static constexpr bool kRowVector = true;
    bf16 *out;
    const float *bias;
    int M, Co;
    int f16;
    int ld;
    __device__ ColQuad column(int col) const { return ColQuad{col, load_quad(bias, col, Co)}; }
    template <int R>
    __device__ void rows(int row0, int step, const ColQuad &c, const float4 (&v)[R]) const {
        if (c.col >= Co) return;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            if (row >= M) break;
            const float4 y = add4(v[i], c.b);
            bf16x4 o;
            o[0] = to_word(y.x < 0.f ? 0.f : y.x, f16);
            o[1] = to_word(y.y < 0.f ? 0.f : y.y, f16);
            o[2] = to_word(y.z < 0.f ? 0.f : y.z, f16);
            o[3] = to_word(y.w < 0.f ? 0.f : y.w, f16);
            *reinterpret_cast<bf16x4 *>(out + (size_t)row * ld + c.col) = o;
        }
    }
};

// Conv epilogue writing bias+ReLU results as NHWC 16-bit words (internal
// maps; bf16, or fp16 when f16 is set) and/or NCHW fp32 (boundary outputs);
// either pointer may be null.
struct EpiConvOut {
    static constexpr bool kRowVector = false;
    bf16 *nhwc;
    float *nchw;
    const float *bias;
    int M, Co, ohw, relu;
    int f16;
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= Co) return;
        const float b = bias[col];
        f32x4 y;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            y[r] = v[r] + b;
            if (relu && y[r] < 0.0f) y[r] = 0.0f;
        }
        if (nhwc)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (row + r < M) nhwc[(size_t)(row + r) * Co + col] = to_word(y[r], f16);
        if (nchw) {
            const int n = row / ohw, p = row - n * ohw;
            if ((ohw & 3) == 0 && row + 3 < M) {
                *reinterpret_cast<f32x4 *>(nchw + ((size_t)n * Co + col) * ohw + p) = y;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = row + r;
                    if (rr >= M) break;
                    const int nn = rr / ohw, pp = rr - nn * ohw;
                    nchw[((size_t)nn * Co + col) * ohw + pp] = y[r];
                }
            }
        }
    }
};

// Lateral 1x1 conv of concat(lower, bilinear-up(upper)) (reference
// image_fpn.c fuse_level / bilinear_channel, align_corners = False) computed
// as W_lower . lower + up(W_upper . upper): a 1x1 conv acts on channels and
// the upsampling on pixels, both linearly, so they commute, and the upper
// half of the conv runs at the upper level's resolution.  This epilogue
// belongs to the GEMM over the lower channels: out[row][col] =
// word(relu(acc + bias[col] + bilinear(up)(pixel row)[col])), NHWC, where
// `up` is the fp32 product W_upper . upper, [n][h][w][Co], and output row =
// n*H*W + oy*W + ox.  Co % 4 == 0.
struct EpiUpAddNHWC {
    static constexpr bool kRowVector = true;
    bf16 *out;
    const float *bias, *up;
    int M, Co, H, W, h, w;
    int f16;
    __device__ ColQuad column(int col) const { return ColQuad{col, load_quad(bias, col, Co)}; }
    template <int R>
    __device__ void rows(int row0, int step, const ColQuad &c, const float4 (&v)[R]) const {
        if (c.col >= Co) return;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int row = row0 + i * step;
            if (row >= M) break;
            const int n = row / (H * W), p = row - n * (H * W), oy = p / W, ox = p - oy * W;
            float sy = ((float)oy + 0.5f) * (float)h / (float)H - 0.5f;
            float sx = ((float)ox + 0.5f) * (float)w / (float)W - 0.5f;
            sy = fmaxf(sy, 0.0f);
            sx = fmaxf(sx, 0.0f);
            const int y0 = (int)floorf(sy), x0 = (int)floorf(sx);
            const int y1 = min(y0 + 1, h - 1), x1 = min(x0 + 1, w - 1);
            const float fy = sy - (float)y0, fx = sx - (float)x0;
            const float *base = up + (size_t)n * h * w * Co + c.col;
            const float4 a = *reinterpret_cast<const float4 *>(base + ((size_t)y0 * w + x0) * Co);
            const float4 b = *reinterpret_cast<const float4 *>(base + ((size_t)y0 * w + x1) * Co);
            const float4 cc = *reinterpret_cast<const float4 *>(base + ((size_t)y1 * w + x0) * Co);
            const float4 d = *reinterpret_cast<const float4 *>(base + ((size_t)y1 * w + x1) * Co);
            const float va[4] = {a.x, a.y, a.z, a.w}, vb[4] = {b.x, b.y, b.z, b.w};
            const float vc[4] = {cc.x, cc.y, cc.z, cc.w}, vd[4] = {d.x, d.y, d.z, d.w};
            const float acc[4] = {v[i].x, v[i].y, v[i].z, v[i].w}, bias4[4] = {c.b.x, c.b.y, c.b.z, c.b.w};
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float top = va[e] * (1.0f - fx) + vb[e] * fx;
                const float bot = vc[e] * (1.0f - fx) + vd[e] * fx;
                float y = acc[e] + bias4[e] + (top * (1.0f - fy) + bot * fy);
                y = y < 0.0f ? 0.0f : y;
                o[e] = to_word(y, f16);
            }
            *reinterpret_cast<bf16x4 *>(out + (size_t)row * Co + c.col) = o;
        }
    }
};

// NCHW fp32 [N][C][HW] -> NHWC 16-bit words [N][HW][ld] (bf16, or fp16 when
// f16 is set; channels C..ld-1 of each row are left untouched) through a
// 64-pixel x 64-channel LDS tile (coalesced reads along pixels, 16-byte writes
// along channels).  C and ld must be multiples of 8.
__device__ __forceinline__ void pack_nhwc_block(const float *x, bf16 *y, int C, int HW, int f16,
                                                int ld, int n, int c0, int p0, float (&tile)[64][65]) {
    const int t = threadIdx.x;
    const float *src = x + (size_t)n * C * HW;
    // All 16 reads are issued before the first LDS store (an element outside
    // the map reads element 0 and stores 0), so their latencies overlap.
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int c = c0 + (t >> 6) + 4 * i, p = p0 + (t & 63);
        v[i] = src[(c < C && p < HW) ? (size_t)c * HW + p : 0];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int cl = (t >> 6) + 4 * i, pl = t & 63;
        tile[cl][pl] = (c0 + cl < C && p0 + pl < HW) ? v[i] : 0.0f;
    }
    __syncthreads();
    bf16 *dst = y + (size_t)n * HW * ld;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = t + 256 * i, pl = q >> 3, ch = (q & 7) * 8;
        const int p = p0 + pl, c = c0 + ch;
        if (p >= HW || c >= C) continue;
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = to_word(tile[ch + e][pl], f16);
        *reinterpret_cast<bf16x8 *>(dst + (size_t)p * ld + c) = v;
    }
}

static __global__ __launch_bounds__(256) void pack_nhwc_kernel(const float *x, bf16 *y, int C, int HW,
                                                               int f16, int ld) {
    __shared__ float tile[64][65];
    pack_nhwc_block(x, y, C, HW, f16, ld, blockIdx.z, blockIdx.y * 64, blockIdx.x * 64, tile);
}

inline void pack_nhwc(const float *x, bf16 *y, int N, int C, int HW, hipStream_t s,
                      bool f16 = false, int ld = 0) {
    hipLaunchKernelGGL(pack_nhwc_kernel, dim3((HW + 63) / 64, (C + 63) / 64, N), dim3(256), 0, s,
                       x, y, C, HW, (int)f16, ld ? ld : C);
}

// Several NCHW -> NHWC packs of the same batch in one launch (one grid over
// the 64 x 64 blocks of every map; row stride = C).
struct PackJob {
    const float *x;
    bf16 *y;
    int C, HW;
};
template <int J>
struct PackJobs {
    PackJob job[J];
};

template <int J>
__global__ __launch_bounds__(256) void pack_nhwc_many_kernel(PackJobs<J> jobs, int N, int f16) {
    __shared__ float tile[64][65];
    int b = (int)blockIdx.x;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const PackJob &pj = jobs.job[j];
        const int bp = (pj.HW + 63) / 64, bc = (pj.C + 63) / 64, count = bp * bc * N;
        if (b < count) {  // uniform over the workgroup
            const int n = b / (bp * bc), r = b - n * (bp * bc), cb = r / bp, pb = r - cb * bp;
            pack_nhwc_block(pj.x, pj.y, pj.C, pj.HW, f16, pj.C, n, cb * 64, pb * 64, tile);
            return;
        }
        b -= count;
    }
}

template <int J>
inline void pack_nhwc_many(const PackJobs<J> &jobs, int N, hipStream_t s, bool f16) {
    int blocks = 0;
    for (int j = 0; j < J; ++j)
        blocks += ((jobs.job[j].HW + 63) / 64) * ((jobs.job[j].C + 63) / 64) * N;
    hipLaunchKernelGGL((pack_nhwc_many_kernel<J>), dim3(blocks), dim3(256), 0, s, jobs, N, (int)f16);
}

}  // namespace bfhip
