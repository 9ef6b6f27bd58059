// Camera neck context: GeneralizedLSSFPN + DepthLSS head + post-LSS
// downsample (drop-in for reference src/cuda_camera.cu).
//
// Every convolution is an implicit GEMM on the bf16 MFMA core with BN folded
// into bf16 weights and an fp32 bias at create.  The reference's glue passes
// become operand gathers or epilogues, so no concat / upsample / split /
// transpose buffer exists:
//   lateral 1x1 convs read concat(lower, bilinear-up(upper)) taps directly;
//   dtransform.0 (1x1, 1->8) is evaluated inside dtransform.3's gather;
//   depthnet.0 reads concat(dtransform out, fpn0) taps directly;
//   depthnet.6 stores logits / context from its epilogue;
//   the last downsample conv stores the x/y-transposed map.
#include "bf_cuda_camera.h"
#include "conv_core.h"
#include "host_util.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <vector>

using namespace bfhip;

namespace {

struct ConvLayer {
    const bf16 *w;
    const float *b;
    int ci, co, k, stride, pad, n, ih, iw, oh, ow;
};

enum {
    kLat1, kFpn1, kLat0, kFpn0, kDt1, kDt2, kDn0, kDn3, kDn6, kDs0, kDs1, kDs2, kLayers
};

}  // namespace

struct bf_cuda_camera_neck {
    size_t batches, h, w, h1, w1, h2, w2, bev_h, bev_w, resident_bytes;
    unsigned char *params, *acts;
    ConvLayer L[kLayers];
    const float *dt0_w, *dt0_b;  // dtransform.0 folded, fused into dtransform.3
    float *t1, *fpn1, *t0, *fpn0, *e1, *e2, *d0, *d1, *bev0, *bev1;
};

namespace {

// Binds conv (+ optional bias, + optional BN), folds BN in fp32 exactly as the
// reference (cuda_camera.cu:116-122), and returns folded weight/bias on host.
int fold_conv(const bf_model *m, const char *wname, const char *bname, const char *bn,
              int ci, int co, int k, std::vector<float> &w, std::vector<float> &b,
              char *error, size_t cap) {
    const uint32_t uco = (uint32_t)co, uci = (uint32_t)ci, uk = (uint32_t)k;
    const float *src = bind_f32(m, wname, {uco, uci, uk, uk}, error, cap);
    if (!src) return 0;
    const size_t span = (size_t)ci * k * k;
    w.assign(src, src + span * co);
    b.assign(co, 0.0f);
    if (bname) {
        const float *sb = bind_f32(m, bname, {uco}, error, cap);
        if (!sb) return 0;
        b.assign(sb, sb + co);
    }
    if (bn) {
        static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
        const float *p[4];
        char name[192];
        for (int i = 0; i < 4; ++i) {
            std::snprintf(name, sizeof(name), "%s.%s", bn, suffix[i]);
            if (!(p[i] = bind_f32(m, name, {uco}, error, cap))) return 0;
        }
        for (int o = 0; o < co; ++o) {
            const float f = p[0][o] / std::sqrt(p[3][o] + 1e-5f);
            b[o] = (b[o] - p[2][o]) * f + p[1][o];
            for (size_t i = 0; i < span; ++i) w[(size_t)o * span + i] *= f;
        }
    }
    return 1;
}

ConvGeom geom_of(const ConvLayer &l) {
    ConvGeom g{};
    g.N = l.n; g.Ci = l.ci; g.IH = l.ih; g.IW = l.iw; g.OH = l.oh; g.OW = l.ow;
    g.KH = l.k; g.KW = l.k; g.SH = l.stride; g.SW = l.stride; g.PH = l.pad; g.PW = l.pad;
    g.transpose = 0;
    g.M = l.n * l.oh * l.ow;
    g.K = l.ci * l.k * l.k;
    return g;
}

template <class T, int KH, int KW, class Src, class Epi>
void run_conv(const ConvLayer &l, const Src &src, const Epi &epi, hipStream_t s) {
    const ConvGeom g = geom_of(l);
    LoadConvA<T::BM, T::BK, T::kThreads, KH, KW, Src> al{};
    al.src = src;
    al.g = g;
    LoadRowsBf16<T::BN, T::BK, T::kThreads> bl{l.w, g.K, l.co, g.K};
    launch_gemm<T>(al, bl, epi, g.M, l.co, g.K, s);
}

using T256 = Tile<64, 128, 64, 2, 2>;   // 256 / 198 output channels
using T32 = Tile<128, 32, 32, 4, 1>;    // dtransform.3: 32 channels
using T64 = Tile<64, 64, 64, 2, 2>;     // dtransform.6: 64 channels
using T80 = Tile<64, 80, 64, 2, 1>;     // downsample: 80 channels

EpiNCHW nchw(const ConvLayer &l, float *out, int relu = 1) {
    return EpiNCHW{out, l.b, l.n * l.oh * l.ow, l.co, l.oh * l.ow, relu};
}

void fpn_impl(bf_cuda_camera_neck *n, const float *s0, const float *s1, const float *s2,
              float *out0, float *out1, hipStream_t s) {
    const int B = (int)n->batches;
    const int h = (int)n->h, w = (int)n->w, h1 = (int)n->h1, w1 = (int)n->w1;
    const int h2 = (int)n->h2, w2 = (int)n->w2;
    SrcUpConcat up1{s1, s2, 384, 768, h1, w1, h2, w2};
    run_conv<T256, 1, 1>(n->L[kLat1], up1, nchw(n->L[kLat1], n->t1), s);
    run_conv<T256, 3, 3>(n->L[kFpn1], SrcNCHW{n->t1, 256, h1, w1}, nchw(n->L[kFpn1], out1), s);
    SrcUpConcat up0{s0, out1, 192, 256, h, w, h1, w1};
    run_conv<T256, 1, 1>(n->L[kLat0], up0, nchw(n->L[kLat0], n->t0), s);
    run_conv<T256, 3, 3>(n->L[kFpn0], SrcNCHW{n->t0, 256, h, w}, nchw(n->L[kFpn0], out0), s);
    (void)B;
}

void depth_impl(bf_cuda_camera_neck *n, const float *fpn0, const float *depth, float *logits,
                float *context, hipStream_t s) {
    const int h = (int)n->h, w = (int)n->w;
    SrcDepthAffine dsrc{depth, n->dt0_w, n->dt0_b, 8 * h, 8 * w};
    run_conv<T32, 5, 5>(n->L[kDt1], dsrc, nchw(n->L[kDt1], n->e1), s);
    run_conv<T64, 5, 5>(n->L[kDt2], SrcNCHW{n->e1, 32, 2 * h, 2 * w}, nchw(n->L[kDt2], n->e2), s);
    run_conv<T256, 3, 3>(n->L[kDn0], SrcConcat2{n->e2, fpn0, 64, 256, h, w},
                         nchw(n->L[kDn0], n->d0), s);
    run_conv<T256, 3, 3>(n->L[kDn3], SrcNCHW{n->d0, 256, h, w}, nchw(n->L[kDn3], n->d1), s);
    const ConvLayer &l = n->L[kDn6];
    run_conv<T256, 1, 1>(l, SrcNCHW{n->d1, 256, h, w},
                         EpiSplitDepth{logits, context, l.b, l.n * h * w, h * w, 118, 80}, s);
}

int build(bf_cuda_camera_neck *n, const bf_model *model, char *error, size_t cap) {
    const int B = (int)n->batches, h = (int)n->h, w = (int)n->w;
    const int h1 = (int)n->h1, w1 = (int)n->w1;
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
        if (!fold_conv(model, sp.w, sp.b, sp.bn, sp.ci, sp.co, sp.k, fw, fb, error, cap)) return 0;
        wo[i] = arena.add_bf16(fw);
        bo[i] = arena.add_f32(fb);
        ConvLayer &l = n->L[i];
        l.ci = sp.ci; l.co = sp.co; l.k = sp.k; l.stride = sp.stride; l.pad = sp.pad;
        l.n = sp.batch; l.ih = sp.ih; l.iw = sp.iw;
        l.oh = (sp.ih + 2 * sp.pad - sp.k) / sp.stride + 1;
        l.ow = (sp.iw + 2 * sp.pad - sp.k) / sp.stride + 1;
    }
    if (!fold_conv(model, "vtransform.dtransform.0.weight", "vtransform.dtransform.0.bias",
                   "vtransform.dtransform.1", 1, 8, 1, fw, fb, error, cap))
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

    // Activations (fp32 NCHW): level-1 lateral / output, level-0 lateral /
    // output, depth encoder maps, trunk maps, downsample intermediates.
    const size_t hw = (size_t)h * w, hw1 = (size_t)h1 * w1;
    const size_t sizes[10] = {
        (size_t)B * 256 * hw1, (size_t)B * 256 * hw1, (size_t)B * 256 * hw, (size_t)B * 256 * hw,
        (size_t)B * 32 * 4 * hw, (size_t)B * 64 * hw, (size_t)B * 256 * hw, (size_t)B * 256 * hw,
        (size_t)80 * bh * bw, (size_t)80 * (bh / 2) * (bw / 2)};
    size_t total = 0, offs[10];
    for (int i = 0; i < 10; ++i) {
        offs[i] = total;
        total += (sizes[i] * 4 + 255) & ~size_t(255);
    }
    if (!hip_ok(hipMalloc(&n->acts, total), error, cap, "allocate camera activations")) return 0;
    n->resident_bytes += total;
    float **slots[10] = {&n->t1, &n->fpn1, &n->t0, &n->fpn0, &n->e1,
                         &n->e2, &n->d0,   &n->d1, &n->bev0, &n->bev1};
    for (int i = 0; i < 10; ++i) *slots[i] = (float *)(n->acts + offs[i]);
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
    depth_impl(n, fpn0, depth, logits, context, reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "HIP depth launch");
}

extern "C" int bf_cuda_camera_neck_forward(bf_cuda_camera_neck *n, const float *s0,
                                           const float *s1, const float *s2, const float *depth,
                                           float *logits, float *context, void *stream,
                                           char *error, size_t cap) {
    if (!n || !s0 || !s1 || !s2 || !depth || !logits || !context)
        return fail(error, cap, "invalid HIP camera-neck buffers");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    fpn_impl(n, s0, s1, s2, n->fpn0, n->fpn1, s);
    depth_impl(n, n->fpn0, depth, logits, context, s);
    return launch_ok(error, cap, "HIP camera-neck launch");
}

extern "C" int bf_cuda_camera_downsample_forward(bf_cuda_camera_neck *n, const float *input,
                                                 float *output, void *stream, char *error,
                                                 size_t cap) {
    if (!n || !input || !output) return fail(error, cap, "invalid HIP downsample buffers");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int bh = (int)n->bev_h, bw = (int)n->bev_w;
    run_conv<T80, 3, 3>(n->L[kDs0], SrcNCHW{input, 80, bh, bw}, nchw(n->L[kDs0], n->bev0), s);
    run_conv<T80, 3, 3>(n->L[kDs1], SrcNCHW{n->bev0, 80, bh, bw}, nchw(n->L[kDs1], n->bev1), s);
    const ConvLayer &l = n->L[kDs2];
    run_conv<T80, 3, 3>(l, SrcNCHW{n->bev1, 80, bh / 2, bw / 2},
                        EpiTransposeXY{output, l.b, l.oh * l.ow, 80, l.oh, l.ow}, s);
    return launch_ok(error, cap, "HIP downsample launch");
}
