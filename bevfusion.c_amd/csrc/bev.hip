// BEV stage context: fuser + SECOND backbone / deblocks + TransFusion shared
// conv and heatmap head (drop-in for reference src/cuda_bev_stage.cu).
//
// Every convolution is a channels-last implicit GEMM on the MFMA core with BN
// folded into [Co][KH][KW][Ci] weights and an fp32 bias at create (BatchNorm
// epsilon 1e-3, as cuda_bev_stage.cu:106-122).  Operands are fp16, not bf16:
// the stage chains up to 17 convolutions, and bf16's 8-bit mantissa rounding
// at every layer compounds to ~1 % relative error at the heatmap, while fp16
// (11 bits, same MFMA rate) keeps it near 0.1 %; post-BN activations are O(1)
// and well inside fp16's range.  Accumulation is fp32.  The boundary input is
// packed to NHWC fp16 once; every intermediate stays NHWC fp16, and the
// boundary outputs (NCHW fp32) are stored by epilogues:
//   deblock.0 (1x1) and deblock.1 store the NCHW `spatial` halves and the
//   channels-last maps the shared conv reads as one 512-channel concat;
//   deblock.1, ConvTranspose2d 2x2 stride 2, is one GEMM over the half-res
//   pixels (N = 4 taps x 256 channels) whose epilogue places tap (dy, dx) of
//   input pixel (y, x) at output pixel (2y + dy, 2x + dx);
//   the shared conv stores `shared` and its channels-last copy; the last
//   heatmap conv stores `heatmap` only.
#include "bf_cuda_bev.h"
#include "conv_layers.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <vector>

using namespace bfhip;

namespace {

constexpr float kBevBnEps = 1e-3f;

enum {
    kFuser,
    kBlock0,                    // 6 layers
    kDeblock0 = kBlock0 + 6,
    kBlock1,                    // 6 layers
    kShared = kBlock1 + 6,
    kHeatMid,
    kHeatOut,
    kConvs
};

// ConvTranspose2d 2x2 stride 2 as a GEMM over input pixels m = y * IW + x:
// column n = (dy * Co + co) * 2 + dx is output pixel (2y + dy, 2x + dx),
// channel co, so a tile's column pair (dx = 0, 1) holds two adjacent outputs.
// BN-folded bias + ReLU (passing NaN).  The staged tile is stored as NCHW
// fp32 runs (one float2 per input pixel and channel, consecutive threads on
// consecutive pixels) and NHWC fp16 rows (eight channels of one output pixel
// per 16-byte store).
struct EpiDeconv2x2 {
    static constexpr bool kRowVector = true;
    static constexpr bool kFullRow = true;
    bf16 *nhwc;
    float *nchw;
    const float *bias;
    int M, IW, Co, OW, ohw;
    template <class T>
    __device__ void tile(float *sC, int stride, int m0, int n0, int tid) const {
        static_assert(T::BN % 16 == 0, "whole chunks of eight column pairs");
        constexpr int kPairs = T::BN / 2, kChunks = kPairs / 8;
        for (int item = tid; item < kPairs * T::BM; item += T::kThreads) {
            const int j = item / T::BM, r = item - j * T::BM, m = m0 + r, n = n0 + 2 * j;
            if (m >= M || n >= 4 * Co) continue;
            const int dy = (n >> 1) / Co, co = (n >> 1) - dy * Co, y = m / IW, x = m - y * IW;
            const float b = bias[co];
            const float y0 = sC[r * stride + 2 * j] + b, y1 = sC[r * stride + 2 * j + 1] + b;
            const float v0 = y0 < 0.0f ? 0.0f : y0, v1 = y1 < 0.0f ? 0.0f : y1;
            float *dst = nchw + (size_t)co * ohw + (size_t)(2 * y + dy) * OW + 2 * x;
            if (((uintptr_t)dst & 7) == 0) {
                *reinterpret_cast<float2 *>(dst) = make_float2(v0, v1);
            } else {
                dst[0] = v0;
                dst[1] = v1;
            }
        }
        for (int item = tid; item < T::BM * 2 * kChunks; item += T::kThreads) {
            const int r = item / (2 * kChunks), rest = item - r * (2 * kChunks);
            const int dx = rest / kChunks, ch = rest - dx * kChunks, m = m0 + r;
            const int n = n0 + 16 * ch;  // the chunk's first column (Co % 8 == 0: one dy)
            if (m >= M || n >= 4 * Co) continue;
            const int dy = (n >> 1) / Co, co = (n >> 1) - dy * Co, y = m / IW, x = m - y * IW;
            const int p = (2 * y + dy) * OW + 2 * x + dx;
            bf16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float y = sC[r * stride + 16 * ch + 2 * e + dx] + bias[co + e];
                o[e] = to_word(y < 0.0f ? 0.0f : y, true);
            }
            *reinterpret_cast<bf16x8 *>(nhwc + (size_t)p * Co + co) = o;
        }
    }
};

// Tiles: the 3x3 convs run on the wave-specialised LDS-DMA core with four
// loader waves (one wave stops at 63 DMA instructions in flight), as 160 x 128
// tiles at full resolution (one tile per CU at 180 x 180) and 64 x 128 at half
// resolution; measured on MI355X through the conv loader at 180 x 180
// (block0.0 / block0.1 / shared / block1.1): 27.9 / 18.4 / 53.9 / 19.3 us vs
// 30.6 / 18.8 / 56.5 / 22.0 us on the plain core (64 x 128, 64 x 64 at half
// resolution).  The 1x1 deblock, the transposed deblock and the 10-channel
// heatmap output keep the plain core.  Every tile sums k in the same order,
// so the choice does not change results.
// The fuser's 336 input channels are not a multiple of the 64-deep DMA k-tile:
// its packed input is stored with a row stride of kFuserPad = 384 channels
// (336..383 zero, written once at create) and its weights carry zero input
// channels 336..383, so each 3x3 tap is six 64-deep k-steps (the zeros add
// exact zeros, at 1.14x the MFMA work).  As 128 x 256 tiles (eight waves of
// 64 x 64, three stages, four loader waves; 254 tiles at 180 x 180, one per
// CU) it measured 56.5 us on MI355X vs 94.5 us for the register-fed 128 x 128
// tile over the 336 channels.
using DFull = DmaTile<64, 128, 64, 2, 2, 2, true>;
using DHalf = DmaTile<64, 64, 64, 2, 2, 2, true>;
using SFull = DmaTile<160, 128, 64, 2, 4, 3, true>;
using SHalf = DmaTile<64, 128, 64, 2, 2, 3, true>;
using SFuser = DmaTile<128, 256, 64, 2, 4, 3, true>;
constexpr int kLoaders = 4;
constexpr int kFuserIn = 336, kFuserPad = 384;

}  // namespace

struct bf_cuda_bev_stage {
    size_t h, w, resident_bytes;
    unsigned char *params, *acts;
    ConvLayer L[kConvs];
    const bf16 *deconv_w;  // [4 * 256][256]: row (dy * 256 + co) * 2 + dx, column ci
    const float *deconv_b;
    // Channels-last fp16 maps: packed input (336 in rows of 384), ping-pong (<= 256),
    // deblock outputs (256 each, read together by the shared conv), shared.
    bf16 *in, *pa, *pb, *s0, *s1, *sh;
};

namespace {

// Folds the transposed deblock's BN into its [in][out][2][2] weights and
// stores them as the GEMM's [(dy * Co + co) * 2 + dx][ci] operand.
int fold_deconv(const bf_model *m, std::vector<float> &w, std::vector<float> &b, char *error,
                size_t cap) {
    const float *src = bind_f32(m, "backbone_2d.deblocks.1.0.weight", {256u, 256u, 2u, 2u},
                                error, cap);
    if (!src) return 0;
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float *p[4];
    char name[192];
    for (int i = 0; i < 4; ++i) {
        std::snprintf(name, sizeof(name), "backbone_2d.deblocks.1.1.%s", suffix[i]);
        if (!(p[i] = bind_f32(m, name, {256u}, error, cap))) return 0;
    }
    w.assign((size_t)4 * 256 * 256, 0.0f);
    b.assign(256, 0.0f);
    for (int co = 0; co < 256; ++co) {
        const float f = p[0][co] / std::sqrt(p[3][co] + kBevBnEps);
        b[co] = (0.0f - p[2][co]) * f + p[1][co];
        for (int ci = 0; ci < 256; ++ci)
            for (int t = 0; t < 4; ++t)  // t = dy * 2 + dx
                w[(((size_t)(t >> 1) * 256 + co) * 2 + (t & 1)) * 256 + ci] =
                    src[((size_t)ci * 256 + co) * 4 + t] * f;
    }
    return 1;
}

int build(bf_cuda_bev_stage *s, const bf_model *model, char *error, size_t cap) {
    const int H = (int)s->h, W = (int)s->w, H2 = H / 2, W2 = W / 2;
    struct Spec {
        const char *w, *b, *bn;
        int ci, co, k, stride, pad, ih, iw;
    };
    // Layer table of reference cuda_bev_stage.cu:239-255 (deblock.1 below).
    std::vector<Spec> spec;
    spec.push_back({"fuser.conv.0.weight", nullptr, "fuser.conv.1", 336, 256, 3, 1, 1, H, W});
    char names[2][6][2][64];  // outlives `spec` within this call
    for (int blk = 0; blk < 2; ++blk)
        for (int l = 0; l < 6; ++l) {
            std::snprintf(names[blk][l][0], 64, "backbone_2d.blocks.%d.%d.weight", blk, 3 * l + 1);
            std::snprintf(names[blk][l][1], 64, "backbone_2d.blocks.%d.%d", blk, 3 * l + 2);
        }
    for (int l = 0; l < 6; ++l)
        spec.push_back({names[0][l][0], nullptr, names[0][l][1], l ? 128 : 256, 128, 3, 1, 1, H, W});
    spec.push_back({"backbone_2d.deblocks.0.0.weight", nullptr, "backbone_2d.deblocks.0.1", 128, 256,
                    1, 1, 0, H, W});
    for (int l = 0; l < 6; ++l)
        spec.push_back({names[1][l][0], nullptr, names[1][l][1], l ? 256 : 128, 256, 3, l ? 1 : 2, 1,
                        l ? H2 : H, l ? W2 : W});
    spec.push_back({"dense_head.shared_conv.weight", "dense_head.shared_conv.bias", nullptr, 512, 128,
                    3, 1, 1, H, W});
    spec.push_back({"dense_head.heatmap_head.0.conv.weight", nullptr, "dense_head.heatmap_head.0.bn",
                    128, 128, 3, 1, 1, H, W});
    spec.push_back({"dense_head.heatmap_head.1.weight", "dense_head.heatmap_head.1.bias", nullptr, 128,
                    10, 3, 1, 1, H, W});
    ParamArena arena;
    size_t wo[kConvs], bo[kConvs];
    std::vector<float> fw, fb;
    for (int i = 0; i < kConvs; ++i) {
        const Spec &sp = spec[i];
        if (!fold_conv(model, sp.w, sp.b, sp.bn, sp.ci, sp.co, sp.k, kBevBnEps, fw, fb, error, cap))
            return 0;
        int ci = sp.ci;
        if (i == kFuser) {
            // [Co][3x3][336] -> [Co][3x3][384], zero input channels past 336.
            std::vector<float> padded((size_t)sp.co * 9 * kFuserPad, 0.0f);
            for (size_t r = 0; r < (size_t)sp.co * 9; ++r)
                std::copy(fw.begin() + r * sp.ci, fw.begin() + (r + 1) * sp.ci,
                          padded.begin() + r * kFuserPad);
            fw.swap(padded);
            ci = kFuserPad;
        }
        wo[i] = arena.add_f16(fw);
        bo[i] = arena.add_f32(fb);
        ConvLayer &l = s->L[i];
        l.ci = ci; l.co = sp.co; l.k = sp.k; l.stride = sp.stride; l.pad = sp.pad;
        l.n = 1; l.ih = sp.ih; l.iw = sp.iw;
        l.oh = (sp.ih + 2 * sp.pad - sp.k) / sp.stride + 1;
        l.ow = (sp.iw + 2 * sp.pad - sp.k) / sp.stride + 1;
    }
    if (!fold_deconv(model, fw, fb, error, cap)) return 0;
    const size_t dw = arena.add_f16(fw), db = arena.add_f32(fb);
    if (!hip_ok(hipMalloc(&s->params, arena.host.size()), error, cap, "allocate BEV parameters") ||
        !hip_ok(hipMemcpy(s->params, arena.host.data(), arena.host.size(), hipMemcpyHostToDevice),
                error, cap, "upload BEV parameters"))
        return 0;
    s->resident_bytes += arena.host.size();
    for (int i = 0; i < kConvs; ++i) {
        s->L[i].w = (const bf16 *)(s->params + wo[i]);
        s->L[i].b = (const float *)(s->params + bo[i]);
    }
    s->deconv_w = (const bf16 *)(s->params + dw);
    s->deconv_b = (const float *)(s->params + db);

    const size_t hw = (size_t)H * W;
    const size_t elems[6] = {kFuserPad * hw, 256 * hw, 256 * hw, 256 * hw, 256 * hw, 128 * hw};
    bf16 **slots[6] = {&s->in, &s->pa, &s->pb, &s->s0, &s->s1, &s->sh};
    size_t total = 0, offs[6];
    for (int i = 0; i < 6; ++i) {
        offs[i] = total;
        total += (elems[i] * 2 + 255) & ~size_t(255);
    }
    if (!hip_ok(hipMalloc(&s->acts, total), error, cap, "allocate BEV activations")) return 0;
    s->resident_bytes += total;
    for (int i = 0; i < 6; ++i) *slots[i] = (bf16 *)(s->acts + offs[i]);
    // The packed input's padding channels are never written by a kernel: zero
    // the map once.
    return hip_ok(hipMemset(s->in, 0, elems[0] * 2), error, cap, "clear the packed BEV input");
}

void forward_impl(bf_cuda_bev_stage *s, const float *input, float *spatial, float *shared,
                  float *heatmap, hipStream_t st) {
    const int H = (int)s->h, W = (int)s->w, H2 = H / 2, W2 = W / 2;
    const size_t hw = (size_t)H * W;
    pack_nhwc(input, s->in, 1, kFuserIn, H * W, st, true, kFuserPad);
    run_conv_spec<SFuser, 3, kLoaders>(s->L[kFuser], s->in, kFuserPad, nullptr, 0,
                                       nhwc_to(s->L[kFuser], s->pa, true), st);
    bf16 *cur = s->pa, *nxt = s->pb;
    for (int l = 0; l < 6; ++l) {
        const ConvLayer &c = s->L[kBlock0 + l];
        run_conv_spec<SFull, 3, kLoaders>(c, cur, c.ci, nullptr, 0, nhwc_to(c, nxt, true), st);
        std::swap(cur, nxt);
    }
    const ConvLayer &d0 = s->L[kDeblock0];
    run_conv_dma<DFull, 1>(d0, cur, 128, nullptr, 0, out_to(d0, s->s0, spatial, 1, true), st);
    for (int l = 0; l < 6; ++l) {
        const ConvLayer &c = s->L[kBlock1 + l];
        run_conv_spec<SHalf, 3, kLoaders>(c, cur, l == 0 ? 128 : 256, nullptr, 0,
                                          nhwc_to(c, nxt, true), st);
        std::swap(cur, nxt);
    }
    // deblock.1: [H2 W2 x 256] x [1024 x 256]^T, scattered to 2x resolution
    const int m = H2 * W2;
    DmaRowsBf16<DHalf::BM, DHalf::BK, DHalf::kThreads> al{cur, 256, m, 256};
    DmaRowsBf16<DHalf::BN, DHalf::BK, DHalf::kThreads> bl{s->deconv_w, 256, 1024, 256};
    launch_gemm_dma<DHalf>(al, bl,
                           EpiDeconv2x2{s->s1, spatial + 256 * hw, s->deconv_b, m, W2, 256, W,
                                        (int)hw},
                           m, 1024, 256, st);
    const ConvLayer &sc = s->L[kShared];
    run_conv_spec<SFull, 3, kLoaders>(sc, s->s0, 256, s->s1, 256, out_to(sc, s->sh, shared, 0, true),
                                      st);
    const ConvLayer &hm = s->L[kHeatMid];
    run_conv_spec<SFull, 3, kLoaders>(hm, s->sh, 128, nullptr, 0, nhwc_to(hm, s->pa, true), st);
    const ConvLayer &ho = s->L[kHeatOut];
    run_conv_dma<DHalf, 3>(ho, s->pa, 128, nullptr, 0, out_to(ho, nullptr, heatmap, 0, true), st);
}

}  // namespace

extern "C" void bf_cuda_bev_stage_destroy(bf_cuda_bev_stage *s) {
    if (!s) return;
    if (s->params) (void)hipFree(s->params);
    if (s->acts) (void)hipFree(s->acts);
    std::free(s);
}

extern "C" size_t bf_cuda_bev_stage_resident_bytes(const bf_cuda_bev_stage *s) {
    return s ? s->resident_bytes : 0;
}

extern "C" int bf_cuda_bev_stage_create(const bf_model *model, size_t height, size_t width,
                                        bf_cuda_bev_stage **out, char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!model || !out || !height || !width || (height & 1) || (width & 1) || height > INT_MAX ||
        width > INT_MAX)
        return fail(error, cap, "invalid HIP BEV stage contract");
    // 512-channel rows and NCHW offsets of the largest map must fit in int.
    if ((unsigned long long)512 * height * width > (unsigned long long)INT_MAX)
        return fail(error, cap, "HIP BEV stage shape is too large");
    bf_cuda_bev_stage *s = (bf_cuda_bev_stage *)std::calloc(1, sizeof(*s));
    if (!s) return fail(error, cap, "HIP BEV context allocation failed");
    s->h = height;
    s->w = width;
    if (!build(s, model, error, cap)) {
        bf_cuda_bev_stage_destroy(s);
        return 0;
    }
    *out = s;
    return 1;
}

extern "C" int bf_cuda_bev_stage_forward(bf_cuda_bev_stage *s, const float *input, float *spatial,
                                         float *shared, float *heatmap, void *stream, char *error,
                                         size_t cap) {
    if (!s || !input || !spatial || !shared || !heatmap)
        return fail(error, cap, "invalid HIP BEV forward buffers");
    forward_impl(s, input, spatial, shared, heatmap, reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "HIP BEV stage launch");
}
