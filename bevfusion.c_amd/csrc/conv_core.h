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
// sees the output pixel a thread owns before any load.
struct SrcNCHW {
    const float *x;
    int C, H, W;
    __device__ void prepare(int, int, int) {}
    __device__ float operator()(int n, int c, int iy, int ix) const {
        return x[(((size_t)n * C + c) * H + iy) * W + ix];
    }
};

// Channel concat of two NCHW maps of equal size: [0,C0) from a, [C0,C0+C1)
// from b (reference depth_concat_kernel, src/cuda_camera.cu:246-253).
struct SrcConcat2 {
    const float *a, *b;
    int C0, C1, H, W;
    __device__ void prepare(int, int, int) {}
    __device__ float operator()(int n, int c, int iy, int ix) const {
        const size_t hw = (size_t)iy * W + ix;
        return c < C0 ? a[((size_t)n * C0 + c) * H * W + hw]
                      : b[((size_t)n * C1 + (c - C0)) * H * W + hw];
    }
};

// Concat of a lower map with the bilinear (align_corners=False) upsample of an
// upper map, consumed by a 1x1 stride-1 convolution, so the tap position is
// the output pixel itself (reference fpn_concat_kernel, cuda_camera.cu:219-244;
// CPU bilinear_channel, image_fpn.c:123-142).
struct SrcUpConcat {
    const float *lower, *upper;
    int Cl, Cu, H, W, h, w;
    int y0, y1, x0, x1;
    float fy, fx;
    __device__ void prepare(int, int oy, int ox) {
        float sy = ((float)oy + 0.5f) * (float)h / (float)H - 0.5f;
        float sx = ((float)ox + 0.5f) * (float)w / (float)W - 0.5f;
        sy = fmaxf(sy, 0.0f);
        sx = fmaxf(sx, 0.0f);
        y0 = (int)floorf(sy);
        x0 = (int)floorf(sx);
        y1 = min(y0 + 1, h - 1);
        x1 = min(x0 + 1, w - 1);
        fy = sy - (float)y0;
        fx = sx - (float)x0;
    }
    __device__ float operator()(int n, int c, int iy, int ix) const {
        if (c < Cl) return lower[(((size_t)n * Cl + c) * H + iy) * W + ix];
        const float *p = upper + ((size_t)n * Cu + (c - Cl)) * h * w;
        const float top = p[y0 * w + x0] * (1.0f - fx) + p[y0 * w + x1] * fx;
        const float bot = p[y1 * w + x0] * (1.0f - fx) + p[y1 * w + x1] * fx;
        return top * (1.0f - fy) + bot * fy;
    }
};

// dtransform.0 (1x1 conv 1->C on dense depth, BN folded, ReLU) evaluated on
// the fly: channel c of tap (iy, ix) is relu(d*w[c] + b[c]).  Padding taps
// stay zero because the consumer's zero padding applies to this map.
struct SrcDepthAffine {
    const float *depth;
    const float *w, *b;
    int H, W;
    __device__ void prepare(int, int, int) {}
    __device__ float operator()(int n, int c, int iy, int ix) const {
        const float v = fmaf(depth[((size_t)n * H + iy) * W + ix], w[c], 0.0f) + b[c];
        return v > 0.0f ? v : 0.0f;
    }
};

// ----------------------------------------------------------------- A loader
// KH/KW > 0 fix the kernel size at compile time; 0 means runtime geometry.
template <int BM, int BK, int THREADS, int KH_, int KW_, class Src>
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
            st[e] = to_bf16(v);
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
    float *logits, *context;
    const float *bias;
    int M, ohw, bins, ctx;
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= bins + ctx) return;
        const float b = bias[col];
        float *base = col < bins ? logits + (size_t)col * ohw : context + (size_t)(col - bins) * ohw;
        const int planes = col < bins ? bins : ctx;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = row + r;
            if (rr >= M) break;
            const int n = rr / ohw, p = rr - n * ohw;
            base[(size_t)n * planes * ohw + p] = v[r] + b;
        }
    }
};

// Last downsample conv: BN-folded bias + ReLU, then the checkpoint's x/y
// permute out[c][x][y] = y(c, y, x) on a [C, H, W] map (reference
// transpose_xy_kernel, cuda_camera.cu:265-271; lss_downsample.c:142-146).
struct EpiTransposeXY {
    float *out;
    const float *bias;
    int M, C, H, W;
    __device__ void operator()(int row, int col, f32x4 v) const {
        if (col >= C) return;
        const float b = bias[col];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = row + r;
            if (rr >= M) break;
            const int hw = H * W, n = rr / hw, p = rr - n * hw, y = p / W, x = p - y * W;
            float o = v[r] + b;
            out[(((size_t)n * C + col) * W + x) * H + y] = o > 0.0f ? o : 0.0f;
        }
    }
};

}  // namespace bfhip
