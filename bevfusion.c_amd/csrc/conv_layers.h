// Host-side helpers shared by the conv contexts (camera neck, BEV stage):
// a bound, BN-folded channels-last conv layer and its launchers on the MFMA
// GEMM core.
#pragma once

#include "conv_core.h"
#include "host_util.h"

#include <cmath>
#include <cstdio>
#include <vector>

namespace bfhip {

struct ConvLayer {
    const bf16 *w;
    const float *b;
    int ci, co, k, stride, pad, n, ih, iw, oh, ow;
};

// Binds conv (+ optional bias, + optional BN), folds BN in fp32 as the
// reference contexts do (f = gamma / sqrt(var + eps), b' = (b - mean) f + beta,
// w' = w f per output channel; cuda_camera.cu:116-122, cuda_bev_stage.cu:
// 106-122) and returns the folded weights permuted to [Co][KH][KW][Ci]
// (channels-last reduction order) plus the fp32 bias.
inline int fold_conv(const bf_model *m, const char *wname, const char *bname, const char *bn,
                     int ci, int co, int k, float eps, std::vector<float> &w,
                     std::vector<float> &b, char *error, size_t cap) {
    const uint32_t uco = (uint32_t)co, uci = (uint32_t)ci, uk = (uint32_t)k;
    const float *src = bind_f32(m, wname, {uco, uci, uk, uk}, error, cap);
    if (!src) return 0;
    const size_t span = (size_t)ci * k * k;
    std::vector<float> folded(src, src + span * co);
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
            const float f = p[0][o] / std::sqrt(p[3][o] + eps);
            b[o] = (b[o] - p[2][o]) * f + p[1][o];
            for (size_t i = 0; i < span; ++i) folded[(size_t)o * span + i] *= f;
        }
    }
    w.resize(span * co);
    for (int o = 0; o < co; ++o)
        for (int c = 0; c < ci; ++c)
            for (int t = 0; t < k * k; ++t)
                w[((size_t)o * k * k + t) * ci + c] = folded[((size_t)o * ci + c) * k * k + t];
    return 1;
}

inline ConvGeom geom_of(const ConvLayer &l) {
    ConvGeom g{};
    g.N = l.n; g.Ci = l.ci; g.IH = l.ih; g.IW = l.iw; g.OH = l.oh; g.OW = l.ow;
    g.KH = l.k; g.KW = l.k; g.SH = l.stride; g.SW = l.stride; g.PH = l.pad; g.PW = l.pad;
    g.transpose = 0;
    g.M = l.n * l.oh * l.ow;
    g.K = l.ci * l.k * l.k;
    return g;
}

// Register-fed gather of any NHWC-style source (channel counts multiples of 8).
template <class T, int KH, int KW, class Src, class Epi>
void run_conv(const ConvLayer &l, const Src &src, const Epi &epi, hipStream_t s) {
    const ConvGeom g = geom_of(l);
    LoadConvNHWC<T::BM, T::BK, T::kThreads, KH, KW, Src> al{};
    al.src = src;
    al.g = g;
    LoadRowsBf16<T::BN, T::BK, T::kThreads> bl{l.w, g.K, l.co, g.K};
    launch_gemm<T>(al, bl, epi, g.M, l.co, g.K, s);
}

// LDS-DMA pipeline for convs over plain or concatenated channels-last maps
// whose channel counts are multiples of the k-tile.
template <class T, int K, class Epi, bool YFAST = false>
void run_conv_dma(const ConvLayer &l, const bf16 *a, int c0, const bf16 *b, int c1, const Epi &epi,
                  hipStream_t s) {
    const ConvGeom g = geom_of(l);
    DmaConvNHWC<T::BM, T::BK, T::kThreads, K, K, YFAST> al{a, b, c0, c1, g};
    DmaRowsBf16<T::BN, T::BK, T::kThreads> bl{l.w, g.K, l.co, g.K};
    launch_gemm_dma<T>(al, bl, epi, g.M, l.co, g.K, s);
}

// Wave-specialised LDS-DMA pipeline (gemm_spec_kernel) for the same convs,
// with LW loader waves.
template <class T, int K, int LW = 1, bool YFAST = false, class Epi>
void run_conv_spec(const ConvLayer &l, const bf16 *a, int c0, const bf16 *b, int c1, const Epi &epi,
                   hipStream_t s) {
    const ConvGeom g = geom_of(l);
    DmaConvNHWC<T::BM, T::BK, LW * kWave, K, K, YFAST> al{a, b, c0, c1, g};
    DmaRowsBf16<T::BN, T::BK, LW * kWave> bl{l.w, g.K, l.co, g.K};
    launch_gemm_spec<T>(al, bl, epi, g.M, l.co, g.K, s);
}

// The same convs as jobs of gemm_pair_kernel (gemm_core.h), for a launch
// shared with an independent layer.
template <class T, int KH, int KW, class Src, class Epi>
auto conv_job(const ConvLayer &l, const Src &src, const Epi &epi) {
    const ConvGeom g = geom_of(l);
    LoadConvNHWC<T::BM, T::BK, T::kThreads, KH, KW, Src> al{};
    al.src = src;
    al.g = g;
    LoadRowsBf16<T::BN, T::BK, T::kThreads> bl{l.w, g.K, l.co, g.K};
    return gemm_job<GemmCore::kReg, T>(al, bl, epi, g.M, l.co, g.K);
}
template <class T, int K, int LW, class Epi>
auto conv_job_spec(const ConvLayer &l, const bf16 *a, int c0, const bf16 *b, int c1, const Epi &epi) {
    const ConvGeom g = geom_of(l);
    DmaConvNHWC<T::BM, T::BK, LW * kWave, K, K, false> al{a, b, c0, c1, g};
    DmaRowsBf16<T::BN, T::BK, LW * kWave> bl{l.w, g.K, l.co, g.K};
    return gemm_job<GemmCore::kSpec, T>(al, bl, epi, g.M, l.co, g.K);
}

inline EpiConvOut out_to(const ConvLayer &l, bf16 *nhwc, float *nchw = nullptr, int relu = 1,
                         bool f16 = false) {
    return EpiConvOut{nhwc, nchw, l.b, l.n * l.oh * l.ow, l.co, l.oh * l.ow, relu, (int)f16};
}

inline EpiConvNHWC nhwc_to(const ConvLayer &l, bf16 *nhwc, bool f16 = false, int ld = 0) {
    return EpiConvNHWC{nhwc, l.b, l.n * l.oh * l.ow, l.co, (int)f16, ld ? ld : l.co};
}

}  // namespace bfhip
