// Stateless fp32-boundary operators: bf_cuda_gemm_f32 and bf_cuda_conv2d_f32
// (drop-ins for reference src/cuda_ops.cu:147-208).
//
// Both run the bf16 MFMA GEMM core.  Operands arrive as fp32 and are rounded
// to bf16 while they are staged into LDS; the convolution never materialises
// an im2col matrix (conv_core.h gathers taps straight from NCHW).
#include "bf_cuda_ops.h"
#include "conv_core.h"

#include <climits>

using namespace bfhip;

namespace {

template <class T, bool VEC>
void gemm_f32_launch(const float *x, const float *w, const float *b, float *y, int M, int K,
                     int N, int relu, hipStream_t s) {
    LoadRowsF32<T::BM, T::BK, T::kThreads, VEC> al{x, K, M, K};
    LoadRowsF32<T::BN, T::BK, T::kThreads, VEC> bl{w, K, N, K};
    EpiRowsF32 epi{y, b, N, M, N, relu};
    launch_gemm<T>(al, bl, epi, M, N, K, s);
}

template <bool VEC>
void gemm_f32_dispatch(const float *x, const float *w, const float *b, float *y, int M, int K,
                       int N, int relu, hipStream_t s) {
    // 144 < N <= 288 (N = 288, K = 96): 32 x 144 tiles,
    // whole column halves, 704 workgroups at M = 11264.  Measured on MI355X
    // at config 1: 9.6 us vs 10.5 us as 128 x 128 tiles (whose third column
    // tile is 75 % empty); the kernel is bound by its fp32 operand reads
    // (5.0 us without the store) and output writes (6.6 us without the
    // loads), not by the tile.
    if (N <= 32)
        gemm_f32_launch<Tile<128, 32, 32, 4, 1>, VEC>(x, w, b, y, M, K, N, relu, s);
    else if (N <= 64)
        gemm_f32_launch<Tile<128, 64, 32, 4, 1>, VEC>(x, w, b, y, M, K, N, relu, s);
    else if (N > 144 && N <= 288)
        gemm_f32_launch<Tile<32, 144, 32, 2, 3>, VEC>(x, w, b, y, M, K, N, relu, s);
    else
        gemm_f32_launch<Tile<128, 128, 32, 2, 2>, VEC>(x, w, b, y, M, K, N, relu, s);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <class T>
void conv_dispatch_tile(const ConvGeom &g, int Co, const float *x, const float *w,
                        const float *b, float *y, int relu, hipStream_t s) {
    LoadConvA<T::BM, T::BK, T::kThreads, 0, 0, SrcNCHW> al{};
    al.src = SrcNCHW{x, g.Ci, g.IH, g.IW};
    al.g = g;
    EpiNCHW epi{y, b, g.M, Co, g.OH * g.OW, relu};
    if (g.transpose) {
        LoadWeightIOHW<T::BN, T::BK, T::kThreads> bl{w, Co, g.K, g.KH * g.KW};
        launch_gemm<T>(al, bl, epi, g.M, Co, g.K, s);
    } else if ((g.K & 3) == 0 && aligned16(w)) {
        LoadRowsF32<T::BN, T::BK, T::kThreads, true> bl{w, g.K, Co, g.K};
        launch_gemm<T>(al, bl, epi, g.M, Co, g.K, s);
    } else {
        LoadRowsF32<T::BN, T::BK, T::kThreads, false> bl{w, g.K, Co, g.K};
        launch_gemm<T>(al, bl, epi, g.M, Co, g.K, s);
    }
}

}  // namespace

extern "C" int bf_cuda_conv2d_f32(const bf_cuda_conv2d_desc *d, const float *input,
                                  const float *weight, const float *bias, float *output,
                                  void *stream, char *error, size_t cap) {
    // Contract checks of reference cuda_ops.cu:150-170, in the same order.
    if (!d || !input || !weight || !output || d->batches <= 0 || d->input_channels <= 0 ||
        d->output_channels <= 0 || d->input_height <= 0 || d->input_width <= 0 ||
        d->kernel_height <= 0 || d->kernel_width <= 0 || d->stride_height <= 0 ||
        d->stride_width <= 0 || d->padding_height < 0 || d->padding_width < 0 ||
        d->output_height <= 0 || d->output_width <= 0 ||
        (d->transpose != 0 && d->transpose != 1) || (d->relu != 0 && d->relu != 1))
        return fail(error, cap, "invalid HIP convolution contract");
    const long long batch_rows = (long long)d->batches * d->output_height;
    if (batch_rows > INT_MAX / d->output_width)
        return fail(error, cap, "HIP convolution is too large");
    const long long channel_reduction = (long long)d->input_channels * d->kernel_height;
    if (channel_reduction > INT_MAX / d->kernel_width)
        return fail(error, cap, "HIP convolution reduction is too large");
    if ((d->output_channels + 15LL) / 16 > 65535)
        return fail(error, cap, "HIP convolution has too many output channels");
    ConvGeom g{};
    g.N = d->batches; g.Ci = d->input_channels; g.IH = d->input_height; g.IW = d->input_width;
    g.OH = d->output_height; g.OW = d->output_width; g.KH = d->kernel_height;
    g.KW = d->kernel_width; g.SH = d->stride_height; g.SW = d->stride_width;
    g.PH = d->padding_height; g.PW = d->padding_width; g.transpose = d->transpose;
    g.M = (int)(batch_rows * d->output_width);
    g.K = (int)(channel_reduction * d->kernel_width);
    const int Co = d->output_channels;
    const long long tiles = ((long long)g.M + 127) / 128 * ((Co + 31LL) / 32);
    if (tiles > INT_MAX) return fail(error, cap, "HIP convolution grid is too large");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (Co <= 32)
        conv_dispatch_tile<Tile<128, 32, 32, 4, 1>>(g, Co, input, weight, bias, output, d->relu, s);
    else if (Co <= 64)
        conv_dispatch_tile<Tile<128, 64, 32, 4, 1>>(g, Co, input, weight, bias, output, d->relu, s);
    else
        conv_dispatch_tile<Tile<128, 128, 32, 2, 2>>(g, Co, input, weight, bias, output, d->relu, s);
    return launch_ok(error, cap, "HIP convolution launch");
}

extern "C" int bf_cuda_gemm_f32(const float *input, const float *weight, const float *bias,
                                float *output, int rows, int in_f, int out_f, int relu,
                                void *stream, char *error, size_t cap) {
    // Contract checks of reference cuda_ops.cu:192-196.
    if (!input || !weight || !output || rows <= 0 || in_f <= 0 || out_f <= 0 ||
        (relu != 0 && relu != 1))
        return fail(error, cap, "invalid HIP GEMM contract");
    if ((out_f + 15LL) / 16 > 65535)
        return fail(error, cap, "HIP GEMM has too many output features");
    if (((long long)rows + 127) / 128 * ((out_f + 31LL) / 32) > INT_MAX)
        return fail(error, cap, "HIP GEMM is too large");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((in_f & 3) == 0 && aligned16(input) && aligned16(weight))
        gemm_f32_dispatch<true>(input, weight, bias, output, rows, in_f, out_f, relu, s);
    else
        gemm_f32_dispatch<false>(input, weight, bias, output, rows, in_f, out_f, relu, s);
    return launch_ok(error, cap, "HIP GEMM launch");
}
