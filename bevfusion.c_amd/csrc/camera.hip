// Camera neck context: GeneralizedLSSFPN + DepthLSS head + post-LSS
// downsample (drop-in for reference src/cuda_camera.cu).
//
// Every convolution is a channels-last implicit GEMM on the fp16 MFMA core
// (fp32 accumulation) with BN folded into fp16 [Co][KH][KW][Ci] weights and an
// fp32 bias at create.  Boundary maps (NCHW fp32 by the ABI) are packed to
// NHWC fp16 once; every intermediate stays NHWC fp16 (16-bit words in the
// bf16 container type).  The reference's glue passes become operand
// gathers or epilogues, so no concat / upsample / split / transpose buffer
// exists:
//   a lateral 1x1 conv over concat(lower, bilinear-up(upper)) runs as
//   W_lower . lower with up(W_upper . upper) added in its epilogue (the
//   upper product computed at the upper resolution, EpiUpAddNHWC);
//   dtransform.0 (1x1, 1->8) is evaluated inside dtransform.3's gather;
//   depthnet.0 reads concat(dtransform out, fpn0) taps directly;
//   depthnet.6 stores logits / context from its epilogue;
//   the last downsample conv stores the x/y-transposed map.
#include "bf_cuda_camera.h"
#include "bfhip_debug.h"
#include "bfhip_profile.h"
#include "conv_layers.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <vector>

using namespace bfhip;

namespace {

// BatchNorm epsilon of the camera modules (cuda_camera.cu:116-122).
constexpr float kCameraBnEps = 1e-5f;

enum {
    kLat1, kFpn1, kLat0, kFpn0, kDt1, kDt2, kDn0, kDn3, kDn6, kDs0, kDs1, kDs2, kLayers
};

}  // namespace

struct bf_cuda_camera_neck {
    size_t batches, h, w, h1, w1, h2, w2, bev_h, bev_w, resident_bytes;
    unsigned char *params, *acts;
    ConvLayer L[kLayers];
    const float *dt0_w, *dt0_b;  // dtransform.0 folded, fused into dtransform.3
    // Channels-last bf16 maps: packed Swin levels, FPN laterals / outputs,
    // depth encoder, depth trunk, packed BEV and downsample intermediates.
    bf16 *p0, *p1, *p2, *t1, *f1, *t0, *f0, *e1, *e2, *d0, *d1, *bp, *b0, *b1;
    // fp32 upper-level lateral products W_upper . upper: [B][h2][w2][256]
    // (lateral 1) and [B][h1][w1][256] (lateral 0).
    float *u1, *u0;
};

namespace {

// Tiles from sweeps of both cores on these shapes (MI355X).  DMA-fed: 64 x 128
// for the 256-channel 3x3 convs at 32x88 below full camera batch and the
// depthnet.6 1x1; the level-0 and level-1 3x3 convs, dtransform.6 and the
// downsample run on the wave-specialised core.
// Register-fed gather (depth affine source): a narrow tile for the
// 32-channel dtransform.3.
using D256 = DmaTile<64, 128, 64, 2, 2, 2, true>;  // 3x3 256-channel convs and depthnet.6 at level 0
// The level-0 3x3 convs with 256 outputs at full camera batch (M = 6 x 32 x
// 88 = 16896 rows) run 160-row x 128-channel tiles on the wave-specialised
// pipeline: 212 tiles in one round, each CU fetching 1.33 MB (instead of 2.65
// MB for the CUs that take three 64 x 128 tiles), eight compute waves of 80 x
// 32, three 64-deep stages (110 KiB of LDS) and four loader waves: operand
// fetch, not the MFMAs, bounds these convs, and one loader wave stops at its
// 63 in-flight DMA instructions.  Measured on MI355X through this loader
// (fpn_convs.0 / depthnet.0): 28.3 / 34.7 us, vs 31.2 / 38.5 us as 80 x 256
// stripes with two loader waves and 38.9 / 48.4 us with one; smaller batches
// keep the 64 x 128 tiles.
using S256 = DmaTile<160, 128, 64, 2, 4, 3, true>;
constexpr int kS256Loaders = 4;
inline bool use_s256(const ConvLayer &l) {
    return l.co == 256 && 2 * ((l.n * l.oh * l.ow + 159) / 160) >= 128;
}
// fpn_convs.1 at level 1 (M = 4224, two loader waves) and dtransform.6 (32
// input channels, so 32-deep k-steps) on the wave-specialised pipeline:
// measured through the conv loader on MI355X, 17.6 us (18.2 us with one loader
// wave, 19.3 us as 64 x 64 tiles) and 11.7 us.
using S64 = DmaTile<32, 64, 64, 1, 2, 4, true>;
constexpr int kS64Loaders = 2;
using S32 = DmaTile<32, 64, 32, 1, 2, 6, true>;
using T32 = Tile<128, 32, 32, 4, 1, true>;         // dtransform.3: 32 output channels
// The downsample's 80-channel maps are stored channels-last with a row
// stride of kDsPad = 96 (channels 80..95 zero, written once at create) and its
// weights carry zero input channels 80..95, so each 3x3 tap is three 32-deep
// k-steps on the LDS-DMA core (the zeros add exact zeros: same results as
// the 80-channel reduction, at 1.2x the MFMA work).  Tiles of 160 rows x all
// 80 output channels, five compute waves of 32 rows, on the wave-specialised
// pipeline with five loader waves; measured on MI355X (downsample.0 / .1 /
// .2): 45.7 / 15.4 / 15.4 us, vs 53.5 / 17.9 / 17.7 us on the plain LDS-DMA
// core (80-row tiles for .0).
constexpr int kDsPad = 96;
using DDs0 = DmaTile<160, 80, 32, 5, 1, 3, true>;   // downsample.0 at the full BEV grid
using DDs1 = DmaTile<160, 80, 32, 5, 1, 4, true>;   // downsample.1 / .2 at half resolution
constexpr int kDsLoaders = 5;

// The A-operand gather of each conv layer, with the tile, pipeline and loader
// instance the forward runs; `epi` consumes the product.  The forward passes
// its epilogues; bfhip_debug_camera_gather passes a row-major fp32 store over
// identity weights, which makes the product the gathered operand itself.
// 3x3 256 -> 256 convs over one map (a) or over concat(a, b).
template <class Epi>
void conv_256(const ConvLayer &l, const bf16 *a, int c0, const bf16 *b, int c1, const Epi &epi,
              hipStream_t s) {
    if (use_s256(l))
        run_conv_spec<S256, 3, kS256Loaders>(l, a, c0, b, c1, epi, s);
    else
        run_conv_dma<D256, 3>(l, a, c0, b, c1, epi, s);
}
template <class Epi>
void conv_fpn1(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    run_conv_spec<S64, 3, kS64Loaders>(l, in, 256, nullptr, 0, epi, s);
}
// dtransform.3 and .6 as jobs: the forward runs each in one launch with a
// lateral's lower half (neck_impl), the other entry points and the probes
// alone, with the same tile, loaders and epilogue.  dtransform.6 takes two
// loader waves so that its workgroup matches the lateral's four waves.
constexpr int kS32Loaders = 2;
template <class Epi>
auto dt1_job(const ConvLayer &l, const float *depth, const float *aw, const float *ab, const Epi &epi) {
    return conv_job<T32, 5, 5>(l, SrcNHWCDepthAffine<true>{depth, aw, ab, l.ih, l.iw}, epi);
}
template <class Epi>
auto dt2_job(const ConvLayer &l, const bf16 *in, const Epi &epi) {
    return conv_job_spec<S32, 5, kS32Loaders>(l, in, 32, nullptr, 0, epi);
}
template <class Epi>
void conv_dt1(const ConvLayer &l, const float *depth, const float *aw, const float *ab,
              const Epi &epi, hipStream_t s) {
    launch_gemm_job(dt1_job(l, depth, aw, ab, epi), s);
}
template <class Epi>
void conv_dt2(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    launch_gemm_job(dt2_job(l, in, epi), s);
}
template <class Epi>
void conv_dn6(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    run_conv_dma<D256, 1>(l, in, 256, nullptr, 0, epi, s);
}
template <class Epi>
void conv_ds0(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    run_conv_spec<DDs0, 3, kDsLoaders>(l, in, kDsPad, nullptr, 0, epi, s);
}
template <class Epi>
void conv_ds1(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    run_conv_spec<DDs1, 3, kDsLoaders>(l, in, kDsPad, nullptr, 0, epi, s);
}
// The checkpoint's x/y permute out[c][x][y] = y(c, y, x) (reference
// transpose_xy_kernel, cuda_camera.cu:265-271; lss_downsample.c:142-146):
// with the GEMM rows in x-major pixel order (YFAST) the transposed NCHW
// output is plain channel planes along the rows.
template <class Epi>
void conv_ds2(const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    run_conv_spec<DDs1, 3, kDsLoaders, true>(l, in, kDsPad, nullptr, 0, epi, s);
}

// FPN output conv: channels-last only, or also NCHW fp32 for the boundary.
template <class Epi>
void fpn_conv_epi(int layer, const ConvLayer &l, const bf16 *in, const Epi &epi, hipStream_t s) {
    if (layer == kFpn1)
        conv_fpn1(l, in, epi, s);
    else
        conv_256(l, in, 256, nullptr, 0, epi, s);
}
void fpn_conv(int layer, const ConvLayer &l, const bf16 *in, bf16 *nhwc, float *nchw, hipStream_t s) {
    if (nchw)
        fpn_conv_epi(layer, l, in, out_to(l, nhwc, nchw, 1, true), s);
    else
        fpn_conv_epi(layer, l, in, nhwc_to(l, nhwc, true), s);
}

// Lateral 1x1 conv `layer` over concat(lower [B][H][W][Cl], up(upper
// [B][h][w][Cu])): the upper product W[:, Cl:] . upper goes to `up` (fp32),
// then W[:, :Cl] . lower + bias + bilinear(up) (ReLU) to `out`.  The folded
// weights are [256][Cl + Cu] rows; each half is read in place.
// The top level's upper product (Cu = 768, M = 1056 at 6 x 256 x 704) runs
// as 32 x 32 tiles on the wave-specialised core with one loader wave (264
// tiles instead of 132): 5.0 vs 6.2 us measured on MI355X; the 4224-row one
// of the next level keeps 32 x 64 tiles (4.9 us; 6.4 us as 32 x 32).
using DLatUp = DmaTile<32, 64, 64, 1, 2, 3, true>;     // upper products (M = B*h*w)
using SLatUpDeep = DmaTile<32, 32, 64, 1, 1, 4, true>;  // upper products with Cu >= 512
using DLat = DmaTile<64, 64, 64, 2, 2, 2, true>;       // lower halves
// The lower half: out = relu(W[:, :Cl] . lower + bias + bilinear(up)), with
// the upsampling in the epilogue (EpiUpAddNHWC); w rows hold ldw columns.
auto lateral_lower_job(const bf16 *lower, int Cl, const bf16 *w, int ldw, const float *bias,
                       const float *up, bf16 *out, int M, int H, int W, int h, int wd) {
    using T = DLat;
    DmaRowsBf16<T::BM, T::BK, T::kThreads> al{lower, Cl, M, Cl};
    DmaRowsBf16<T::BN, T::BK, T::kThreads> bl{w, ldw, 256, Cl};
    return gemm_job<GemmCore::kDma, T>(al, bl, EpiUpAddNHWC{out, bias, up, M, 256, H, W, h, wd, 1},
                                       M, 256, Cl);
}
// The upper product W[:, Cl:] . upper into `up` (fp32).
void lateral_upper(const ConvLayer &l, int Cl, const bf16 *upper, int Cu, int h, int w, float *up,
                   hipStream_t s) {
    const int Mu = l.n * h * w, ci = Cl + Cu;
    if (Cu >= 512) {
        using T = SLatUpDeep;
        DmaRowsBf16<T::BM, T::BK, kWave> al{upper, Cu, Mu, Cu};
        DmaRowsBf16<T::BN, T::BK, kWave> bl{l.w + Cl, ci, 256, Cu};
        launch_gemm_spec<T>(al, bl, EpiRowsF32{up, nullptr, 256, Mu, 256, 0}, Mu, 256, Cu, s);
    } else {
        using T = DLatUp;
        DmaRowsBf16<T::BM, T::BK, T::kThreads> al{upper, Cu, Mu, Cu};
        DmaRowsBf16<T::BN, T::BK, T::kThreads> bl{l.w + Cl, ci, 256, Cu};
        launch_gemm_dma<T>(al, bl, EpiRowsF32{up, nullptr, 256, Mu, 256, 0}, Mu, 256, Cu, s);
    }
}
void lateral(const ConvLayer &l, const bf16 *lower, int Cl, int H, int W, const bf16 *upper, int Cu,
             int h, int w, float *up, bf16 *out, hipStream_t s) {
    lateral_upper(l, Cl, upper, Cu, h, w, up, s);
    launch_gemm_job(lateral_lower_job(lower, Cl, l.w, Cl + Cu, l.b, up, out, l.n * H * W, H, W, h, w), s);
}

void lateral1(bf_cuda_camera_neck *n, hipStream_t s) {
    lateral(n->L[kLat1], n->p1, 384, (int)n->h1, (int)n->w1, n->p2, 768, (int)n->h2, (int)n->w2,
            n->u1, n->t1, s);
}

void lateral0(bf_cuda_camera_neck *n, hipStream_t s) {
    lateral(n->L[kLat0], n->p0, 192, (int)n->h, (int)n->w, n->f1, 256, (int)n->h1, (int)n->w1, n->u0,
            n->t0, s);
}

// The three Swin levels to channels-last fp16 in one launch.
void pack_levels(bf_cuda_camera_neck *n, const float *s0, const float *s1, const float *s2,
                 hipStream_t s) {
    const int B = (int)n->batches;
    const int hw = (int)(n->h * n->w), hw1 = (int)(n->h1 * n->w1), hw2 = (int)(n->h2 * n->w2);
    pack_nhwc_many(PackJobs<3>{{{s0, n->p0, 192, hw}, {s1, n->p1, 384, hw1}, {s2, n->p2, 768, hw2}}}, B,
                   s, true);
}

// FPN from NCHW fp32 Swin levels; FPN levels land channels-last in f0/f1 and,
// when requested, also NCHW fp32 in out0/out1.
void fpn_impl(bf_cuda_camera_neck *n, const float *s0, const float *s1, const float *s2,
              float *out0, float *out1, hipStream_t s) {
    pack_levels(n, s0, s1, s2, s);
    lateral1(n, s);
    fpn_conv(kFpn1, n->L[kFpn1], n->t1, n->f1, out1, s);
    lateral0(n, s);
    fpn_conv(kFpn0, n->L[kFpn0], n->t0, n->f0, out0, s);
}

// One layer of the depth head (dtransform.3 .. depthnet.6); the forward and
// the profiling hooks launch through here.
void depth_layer(bf_cuda_camera_neck *n, int layer, const float *depth, float *logits,
                 float *context, hipStream_t s) {
    const int h = (int)n->h, w = (int)n->w;
    const ConvLayer &l = n->L[layer];
    switch (layer) {
        case kDt1: conv_dt1(l, depth, n->dt0_w, n->dt0_b, nhwc_to(l, n->e1, true), s); break;
        case kDt2: conv_dt2(l, n->e1, nhwc_to(l, n->e2, true), s); break;
        case kDn0: conv_256(l, n->e2, 64, n->f0, 256, nhwc_to(l, n->d0, true), s); break;
        case kDn3: conv_256(l, n->d0, 256, nullptr, 0, nhwc_to(l, n->d1, true), s); break;
        case kDn6:
            conv_dn6(l, n->d1, EpiSplitDepth{logits, context, l.b, l.n * h * w, h * w, 118, 80}, s);
            break;
        default: break;
    }
}

// One layer of the post-LSS downsample from the packed BEV in n->bp; the last
// one stores the x/y-transposed NCHW output.
void downsample_layer(bf_cuda_camera_neck *n, int layer, float *output, hipStream_t s) {
    const ConvLayer &l = n->L[layer];
    switch (layer) {
        case kDs0: conv_ds0(l, n->bp, nhwc_to(l, n->b0, true, kDsPad), s); break;
        case kDs1: conv_ds1(l, n->b0, nhwc_to(l, n->b1, true, kDsPad), s); break;
        case kDs2: conv_ds2(l, n->b1, EpiPlanesNCHW{output, l.b, l.oh * l.ow, 80, l.oh * l.ow}, s); break;
        default: break;
    }
}

// Depth head from the channels-last fpn0 in n->f0.
void depth_impl(bf_cuda_camera_neck *n, const float *depth, float *logits, float *context,
                hipStream_t s) {
    for (int layer : {kDt1, kDt2, kDn0, kDn3, kDn6}) depth_layer(n, layer, depth, logits, context, s);
}

// The depth encoder's two convs (dtransform.3 / .6) read only the dense depth,
// so the forward runs each in one launch with one of the FPN's lateral lower
// halves (gemm_pair_kernel): both grids are a few hundred latency-bound tiles
// (132 + 264, and 528 + 1056), and paired they fill the CUs the other leaves
// idle (frame -14 us measured on MI355X).
void dt1_lateral1(bf_cuda_camera_neck *n, const float *depth, hipStream_t s) {
    const ConvLayer &d = n->L[kDt1], &l = n->L[kLat1];
    const int h1 = (int)n->h1, w1 = (int)n->w1, h2 = (int)n->h2, w2 = (int)n->w2;
    launch_gemm_pair(dt1_job(d, depth, n->dt0_w, n->dt0_b, nhwc_to(d, n->e1, true)),
                     lateral_lower_job(n->p1, 384, l.w, 384 + 768, l.b, n->u1, n->t1, l.n * h1 * w1,
                                       h1, w1, h2, w2),
                     s);
}
void dt2_lateral0(bf_cuda_camera_neck *n, hipStream_t s) {
    const ConvLayer &d = n->L[kDt2], &l = n->L[kLat0];
    const int h = (int)n->h, w = (int)n->w, h1 = (int)n->h1, w1 = (int)n->w1;
    launch_gemm_pair(dt2_job(d, n->e1, nhwc_to(d, n->e2, true)),
                     lateral_lower_job(n->p0, 192, l.w, 192 + 256, l.b, n->u0, n->t0, l.n * h * w, h,
                                       w, h1, w1),
                     s);
}

// The whole neck: FPN and depth head with the two pairs above.
void neck_impl(bf_cuda_camera_neck *n, const float *s0, const float *s1, const float *s2,
               const float *depth, float *logits, float *context, hipStream_t s) {
    pack_levels(n, s0, s1, s2, s);
    lateral_upper(n->L[kLat1], 384, n->p2, 768, (int)n->h2, (int)n->w2, n->u1, s);
    dt1_lateral1(n, depth, s);
    fpn_conv(kFpn1, n->L[kFpn1], n->t1, n->f1, nullptr, s);
    lateral_upper(n->L[kLat0], 192, n->f1, 256, (int)n->h1, (int)n->w1, n->u0, s);
    dt2_lateral0(n, s);
    fpn_conv(kFpn0, n->L[kFpn0], n->t0, n->f0, nullptr, s);
    for (int layer : {kDn0, kDn3, kDn6}) depth_layer(n, layer, depth, logits, context, s);
}

int build(bf_cuda_camera_neck *n, const bf_model *model, char *error, size_t cap) {
    const int B = (int)n->batches, h = (int)n->h, w = (int)n->w;
    const int h1 = (int)n->h1, w1 = (int)n->w1, h2 = (int)n->h2, w2 = (int)n->w2;
    const int bh = (int)n->bev_h, bw = (int)n->bev_w;
    struct Spec {
        const char *w, *b, *bn;
        int ci, co, k, stride, pad, batch, ih, iw;
    };
    // Layer table of reference cuda_camera.cu:301-318 (dtransform.0 handled below).
    const Spec spec[kLayers] = {
        {"neck.lateral_convs.1.conv.weight", nullptr, "neck.lateral_convs.1.bn", 1152, 256, 1, 1, 0, B, h1, w1},
        {"neck.fpn_convs.1.conv.weight", nullptr, "neck.fpn_convs.1.bn", 256, 256, 3, 1, 1, B, h1, w1},
        {"neck.lateral_convs.0.conv.weight", nullptr, "neck.lateral_convs.0.bn", 448, 256, 1, 1, 0, B, h, w},
        {"neck.fpn_convs.0.conv.weight", nullptr, "neck.fpn_convs.0.bn", 256, 256, 3, 1, 1, B, h, w},
        {"vtransform.dtransform.3.weight", "vtransform.dtransform.3.bias", "vtransform.dtransform.4", 8, 32, 5, 4, 2, B, 8 * h, 8 * w},
        {"vtransform.dtransform.6.weight", "vtransform.dtransform.6.bias", "vtransform.dtransform.7", 32, 64, 5, 2, 2, B, 2 * h, 2 * w},
        {"vtransform.depthnet.0.weight", "vtransform.depthnet.0.bias", "vtransform.depthnet.1", 320, 256, 3, 1, 1, B, h, w},
        {"vtransform.depthnet.3.weight", "vtransform.depthnet.3.bias", "vtransform.depthnet.4", 256, 256, 3, 1, 1, B, h, w},
        {"vtransform.depthnet.6.weight", "vtransform.depthnet.6.bias", nullptr, 256, 198, 1, 1, 0, B, h, w},
        {"vtransform.downsample.0.weight", nullptr, "vtransform.downsample.1", 80, 80, 3, 1, 1, 1, bh, bw},
        {"vtransform.downsample.3.weight", nullptr, "vtransform.downsample.4", 80, 80, 3, 2, 1, 1, bh, bw},
        {"vtransform.downsample.6.weight", nullptr, "vtransform.downsample.7", 80, 80, 3, 1, 1, 1, bh / 2, bw / 2},
    };
    ParamArena arena;
    size_t wo[kLayers], bo[kLayers];
    std::vector<float> fw, fb;
    for (int i = 0; i < kLayers; ++i) {
        const Spec &sp = spec[i];
        if (!fold_conv(model, sp.w, sp.b, sp.bn, sp.ci, sp.co, sp.k, kCameraBnEps, fw, fb, error,
                       cap))
            return 0;
        int ci = sp.ci;
        if (i >= kDs0) {
            // [Co][3x3][80] -> [Co][3x3][kDsPad], zero input channels past 80.
            std::vector<float> padded((size_t)sp.co * 9 * kDsPad, 0.0f);
            for (size_t r = 0; r < (size_t)sp.co * 9; ++r)
                std::copy(fw.begin() + r * sp.ci, fw.begin() + (r + 1) * sp.ci,
                          padded.begin() + r * kDsPad);
            fw.swap(padded);
            ci = kDsPad;
        }
        wo[i] = arena.add_f16(fw);
        bo[i] = arena.add_f32(fb);
        ConvLayer &l = n->L[i];
        l.ci = ci; l.co = sp.co; l.k = sp.k; l.stride = sp.stride; l.pad = sp.pad;
        l.n = sp.batch; l.ih = sp.ih; l.iw = sp.iw;
        l.oh = (sp.ih + 2 * sp.pad - sp.k) / sp.stride + 1;
        l.ow = (sp.iw + 2 * sp.pad - sp.k) / sp.stride + 1;
    }
    if (!fold_conv(model, "vtransform.dtransform.0.weight", "vtransform.dtransform.0.bias",
                   "vtransform.dtransform.1", 1, 8, 1, kCameraBnEps, fw, fb, error, cap))
        return 0;
    const size_t dt0w = arena.add_f32(fw), dt0b = arena.add_f32(fb);
    if (!hip_ok(hipMalloc(&n->params, arena.host.size()), error, cap, "allocate camera parameters") ||
        !hip_ok(hipMemcpy(n->params, arena.host.data(), arena.host.size(), hipMemcpyHostToDevice),
                error, cap, "upload camera parameters"))
        return 0;
    n->resident_bytes += arena.host.size();
    for (int i = 0; i < kLayers; ++i) {
        n->L[i].w = (const bf16 *)(n->params + wo[i]);
        n->L[i].b = (const float *)(n->params + bo[i]);
    }
    n->dt0_w = (const float *)(n->params + dt0w);
    n->dt0_b = (const float *)(n->params + dt0b);

    const size_t hw = (size_t)h * w, hw1 = (size_t)h1 * w1, hw2 = (size_t)h2 * w2;
    const size_t bev = (size_t)bh * bw;
    const size_t elems[14] = {
        B * 192 * hw, B * 384 * hw1, B * 768 * hw2, B * 256 * hw1, B * 256 * hw1, B * 256 * hw,
        B * 256 * hw, B * 32 * 4 * hw, B * 64 * hw, B * 256 * hw, B * 256 * hw, kDsPad * bev,
        kDsPad * bev, kDsPad * (bev / 4)};
    bf16 **slots[14] = {&n->p0, &n->p1, &n->p2, &n->t1, &n->f1, &n->t0, &n->f0,
                        &n->e1, &n->e2, &n->d0, &n->d1, &n->bp, &n->b0, &n->b1};
    size_t total = 0, offs[14];
    for (int i = 0; i < 14; ++i) {
        offs[i] = total;
        total += (elems[i] * 2 + 255) & ~size_t(255);
    }
    const size_t u1_off = total, u0_off = u1_off + ((B * 256 * hw2 * 4 + 255) & ~size_t(255));
    total = u0_off + ((B * 256 * hw1 * 4 + 255) & ~size_t(255));
    if (!hip_ok(hipMalloc(&n->acts, total), error, cap, "allocate camera activations")) return 0;
    n->resident_bytes += total;
    for (int i = 0; i < 14; ++i) *slots[i] = (bf16 *)(n->acts + offs[i]);
    n->u1 = (float *)(n->acts + u1_off);
    n->u0 = (float *)(n->acts + u0_off);
    // The downsample maps' padding channels are never written by a kernel:
    // zero them (with the rest of those maps) once.
    if (!hip_ok(hipMemset(n->bp, 0, (size_t)(offs[13] - offs[11]) + elems[13] * 2), error, cap,
                "clear the downsample maps"))
        return 0;
    return 1;
}

}  // namespace

extern "C" void bf_cuda_camera_neck_destroy(bf_cuda_camera_neck *n) {
    if (!n) return;
    if (n->params) (void)hipFree(n->params);
    if (n->acts) (void)hipFree(n->acts);
    std::free(n);
}

extern "C" size_t bf_cuda_camera_neck_resident_bytes(const bf_cuda_camera_neck *n) {
    return n ? n->resident_bytes : 0;
}

extern "C" int bf_cuda_camera_neck_create(const bf_model *model, size_t batches, size_t h,
                                          size_t w, size_t bev_h, size_t bev_w,
                                          bf_cuda_camera_neck **out, char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!model || !out || !batches || !h || !w || !bev_h || !bev_w || (bev_h & 1) ||
        (bev_w & 1) || batches > INT_MAX || h > INT_MAX || w > INT_MAX || bev_h > INT_MAX ||
        bev_w > INT_MAX)
        return fail(error, cap, "invalid HIP camera-neck contract");
    // The depth encoder runs at 8x the feature resolution; its tap indices and
    // the 320-channel trunk rows must stay within int range.
    if ((unsigned long long)batches * 64 * h * w * 32 > (unsigned long long)INT_MAX ||
        (unsigned long long)80 * bev_h * bev_w > (unsigned long long)INT_MAX)
        return fail(error, cap, "HIP camera-neck shape is too large");
    bf_cuda_camera_neck *n = (bf_cuda_camera_neck *)std::calloc(1, sizeof(*n));
    if (!n) return fail(error, cap, "camera-neck host allocation failed");
    n->batches = batches; n->h = h; n->w = w;
    n->h1 = (h + 1) / 2; n->w1 = (w + 1) / 2;
    n->h2 = (n->h1 + 1) / 2; n->w2 = (n->w1 + 1) / 2;
    n->bev_h = bev_h; n->bev_w = bev_w;
    if (!build(n, model, error, cap)) {
        bf_cuda_camera_neck_destroy(n);
        return 0;
    }
    *out = n;
    return 1;
}

extern "C" int bf_cuda_camera_fpn_forward(bf_cuda_camera_neck *n, const float *s0,
                                          const float *s1, const float *s2, float *out0,
                                          float *out1, void *stream, char *error, size_t cap) {
    if (!n || !s0 || !s1 || !s2 || !out0 || !out1)
        return fail(error, cap, "invalid HIP FPN buffers");
    fpn_impl(n, s0, s1, s2, out0, out1, reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "HIP FPN launch");
}

extern "C" int bf_cuda_camera_depth_forward(bf_cuda_camera_neck *n, const float *fpn0,
                                            const float *depth, float *logits, float *context,
                                            void *stream, char *error, size_t cap) {
    if (!n || !fpn0 || !depth || !logits || !context)
        return fail(error, cap, "invalid HIP depth buffers");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    pack_nhwc(fpn0, n->f0, (int)n->batches, 256, (int)(n->h * n->w), s, true);
    depth_impl(n, depth, logits, context, s);
    return launch_ok(error, cap, "HIP depth launch");
}

extern "C" int bf_cuda_camera_neck_forward(bf_cuda_camera_neck *n, const float *s0,
                                           const float *s1, const float *s2, const float *depth,
                                           float *logits, float *context, void *stream,
                                           char *error, size_t cap) {
    if (!n || !s0 || !s1 || !s2 || !depth || !logits || !context)
        return fail(error, cap, "invalid HIP camera-neck buffers");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    neck_impl(n, s0, s1, s2, depth, logits, context, s);
    return launch_ok(error, cap, "HIP camera-neck launch");
}

extern "C" int bf_cuda_camera_downsample_forward(bf_cuda_camera_neck *n, const float *input,
                                                 float *output, void *stream, char *error,
                                                 size_t cap) {
    if (!n || !input || !output) return fail(error, cap, "invalid HIP downsample buffers");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    pack_nhwc(input, n->bp, 1, 80, (int)(n->bev_h * n->bev_w), s, true, kDsPad);
    for (int layer : {kDs0, kDs1, kDs2}) downsample_layer(n, layer, output, s);
    return launch_ok(error, cap, "HIP downsample launch");
}

extern "C" int bfhip_camera_profile_layer(bf_cuda_camera_neck *n, int layer, void *stream,
                                          char *error, size_t cap) {
    if (!n || layer < 0 || layer >= kLayers) return fail(error, cap, "invalid HIP camera layer");
    if (layer == kDt1 || layer == kDn6)
        return fail(error, cap, "camera layer %d reads or writes caller buffers; time it through "
                    "bfhip_camera_profile_layer_io", layer);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int h = (int)n->h, w = (int)n->w, h1 = (int)n->h1, w1 = (int)n->w1;
    const int h2 = (int)n->h2, w2 = (int)n->w2, bh = (int)n->bev_h, bw = (int)n->bev_w;
    const ConvLayer &l = n->L[layer];
    // Same kernels and shapes as the forward entry points, on context buffers.
    switch (layer) {
        case kLat1: lateral_upper(l, 384, n->p2, 768, h2, w2, n->u1, s); break;
        case kFpn1: fpn_conv(layer, l, n->t1, n->f1, nullptr, s); break;
        case kLat0: lateral_upper(l, 192, n->f1, 256, h1, w1, n->u0, s); break;
        case kFpn0: fpn_conv(layer, l, n->t0, n->f0, nullptr, s); break;
        case kDt2: dt2_lateral0(n, s); break;
        case kDn0: case kDn3: depth_layer(n, layer, nullptr, nullptr, nullptr, s); break;
        case kDs0: case kDs1: downsample_layer(n, layer, nullptr, s); break;
        case kDs2:
            run_conv_dma<DDs1, 3>(l, n->b1, kDsPad, nullptr, 0, nhwc_to(l, n->b0, true, kDsPad), s);
            break;
        default: break;
    }
    return launch_ok(error, cap, "launch HIP camera profiling layer");
}

extern "C" int bfhip_camera_profile_layer_io(bf_cuda_camera_neck *n, int layer, const float *input,
                                             float *out0, float *out1, void *stream, char *error,
                                             size_t cap) {
    if (!n || (layer != kDt1 && layer != kDn6 && layer != kDs2) || (layer == kDt1 && !input) ||
        (layer == kDn6 && (!out0 || !out1)) || (layer == kDs2 && !out0))
        return fail(error, cap, "invalid HIP camera layer profiling call");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (layer == kDs2)
        downsample_layer(n, layer, out0, s);
    else if (layer == kDt1)
        dt1_lateral1(n, input, s);
    else
        depth_layer(n, layer, input, out0, out1, s);
    return launch_ok(error, cap, "launch HIP camera layer profiling");
}

extern "C" int bfhip_camera_profile_pack(bf_cuda_camera_neck *n, const float *s0, const float *s1,
                                         const float *s2, void *stream, char *error, size_t cap) {
    if (!n || !s0 || !s1 || !s2) return fail(error, cap, "invalid HIP camera pack profiling call");
    pack_levels(n, s0, s1, s2, reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "launch HIP camera pack profiling");
}

// ---- Index probes (include/bfhip_debug.h) ----------------------------------
namespace {

// Device allocations of a probe, released on every return path.
struct ProbeBuffers {
    std::vector<void *> held;
    ProbeBuffers() = default;
    ProbeBuffers(const ProbeBuffers &) = delete;
    ProbeBuffers &operator=(const ProbeBuffers &) = delete;
    ~ProbeBuffers() {
        for (void *p : held) (void)hipFree(p);
    }
    void *upload(const void *host, size_t bytes, char *error, size_t cap) {
        void *p = nullptr;
        if (!hip_ok(hipMalloc(&p, bytes), error, cap, "allocate probe buffer")) return nullptr;
        held.push_back(p);
        if (!hip_ok(hipMemcpy(p, host, bytes, hipMemcpyHostToDevice), error, cap, "upload probe buffer"))
            return nullptr;
        return p;
    }
};

}  // namespace

extern "C" int bfhip_debug_camera_gather(bf_cuda_camera_neck *n, int layer, const void *src0,
                                         const void *src1, const float *affine, float *out,
                                         void *stream, char *error, size_t cap) {
    const bool conv = layer == kFpn1 || layer == kFpn0 || (layer >= kDt1 && layer <= kDs2);
    if (!n || !conv || !src0 || !out || (layer == kDn0 && !src1) || (layer == kDt1 && !affine))
        return fail(error, cap, "invalid camera gather probe");
    ConvLayer l = n->L[layer];
    const int K = l.ci * l.k * l.k, M = l.n * l.oh * l.ow;
    if ((long long)M * K > INT_MAX) return fail(error, cap, "camera gather probe is too large");
    // Identity weights (fp16 1.0 = 0x3C00 on the diagonal, K output columns)
    // and a zero bias: the product is the gathered operand, exactly.
    std::vector<uint16_t> ident((size_t)K * K, 0);
    for (int k = 0; k < K; ++k) ident[(size_t)k * K + k] = 0x3C00;
    const std::vector<float> zero(K, 0.0f);
    ProbeBuffers buf;
    l.w = static_cast<const bf16 *>(buf.upload(ident.data(), ident.size() * 2, error, cap));
    l.b = static_cast<const float *>(buf.upload(zero.data(), zero.size() * 4, error, cap));
    if (!l.w || !l.b) return 0;
    l.co = K;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const EpiRowsF32 epi{out, nullptr, K, M, K, 0};
    const bf16 *a = static_cast<const bf16 *>(src0), *b = static_cast<const bf16 *>(src1);
    switch (layer) {
        case kFpn1: case kFpn0: fpn_conv_epi(layer, l, a, epi, s); break;
        case kDt1: conv_dt1(l, static_cast<const float *>(src0), affine, affine + 8, epi, s); break;
        case kDt2: conv_dt2(l, a, epi, s); break;
        case kDn0: conv_256(l, a, 64, b, 256, epi, s); break;
        case kDn3: conv_256(l, a, 256, nullptr, 0, epi, s); break;
        case kDn6: conv_dn6(l, a, epi, s); break;
        case kDs0: conv_ds0(l, a, epi, s); break;
        case kDs1: conv_ds1(l, a, epi, s); break;
        case kDs2: conv_ds2(l, a, epi, s); break;
        default: break;
    }
    return launch_ok(error, cap, "launch camera gather probe") &&
           hip_ok(hipStreamSynchronize(s), error, cap, "camera gather probe");
}

extern "C" int bfhip_debug_fpn_upsample(bf_cuda_camera_neck *n, int level, const float *up,
                                        void *out, void *stream, char *error, size_t cap) {
    if (!n || (level != 0 && level != 1) || !up || !out)
        return fail(error, cap, "invalid FPN upsample probe");
    const ConvLayer &l = n->L[level == 0 ? kLat0 : kLat1];
    const int Cl = level == 0 ? 192 : 384;
    const int H = level == 0 ? (int)n->h : (int)n->h1, W = level == 0 ? (int)n->w : (int)n->w1;
    const int h = level == 0 ? (int)n->h1 : (int)n->h2, w = level == 0 ? (int)n->w1 : (int)n->w2;
    const int M = l.n * H * W;
    // Zero lower map, weights and bias: the epilogue adds the bilinear
    // upsampling of `up` to an exact zero.
    const std::vector<uint16_t> lower((size_t)M * Cl, 0), weights((size_t)256 * Cl, 0);
    const std::vector<float> bias(256, 0.0f);
    ProbeBuffers buf;
    const void *dl = buf.upload(lower.data(), lower.size() * 2, error, cap);
    const void *dw = buf.upload(weights.data(), weights.size() * 2, error, cap);
    const void *db = buf.upload(bias.data(), bias.size() * 4, error, cap);
    if (!dl || !dw || !db) return 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    launch_gemm_job(lateral_lower_job(static_cast<const bf16 *>(dl), Cl, static_cast<const bf16 *>(dw),
                                      Cl, static_cast<const float *>(db), up, static_cast<bf16 *>(out),
                                      M, H, W, h, w),
                    s);
    return launch_ok(error, cap, "launch FPN upsample probe") &&
           hip_ok(hipStreamSynchronize(s), error, cap, "FPN upsample probe");
}
