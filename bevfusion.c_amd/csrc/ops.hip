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

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <class T, bool VEC>
void gemm_f32_launch(const float *x, const float *w, const float *b, float *y, int M, int K,
                     int N, int relu, hipStream_t s) {
    LoadRowsF32<T::BM, T::BK, T::kThreads, VEC> al{x, K, M, K};
    LoadRowsF32<T::BN, T::BK, T::kThreads, VEC> bl{w, K, N, K};
    EpiRowsF32 epi{y, b, N, M, N, relu};
    launch_gemm<T>(al, bl, epi, M, N, K, s);
}

// Short reductions (K <= 128, the stateless linear of BASELINE config 1):
// one pass per row panel with every load issued up front, instead of the
// tiled core's K/32 rounds of global -> registers -> LDS -> MFMA.  The grid
// is (row panels of 128) x (2 column halves).  A workgroup copies its half
// of W into LDS as fp32 with buffer_load ... lds (no register round trip;
// the 16-byte chunks of each row are XOR-swizzled so that fragment reads are
// conflict-free), while each wave loads its 16 x K slice of X straight into
// MFMA operand registers.  It then walks its column blocks: Y^T block =
// W block * X^T on the bf16 MFMA, W fragments rounded to bf16 as they are
// read, so each lane ends up holding 4 consecutive output columns of one row
// and stores them as one float4.  Operands are rounded to bf16 exactly as the
// tiled core rounds them, the k order of the accumulation is the same
// (32-deep MFMA steps in increasing k) and the bias is added after it, so the
// two paths agree bit for bit.  Requires K % 4 == 0, N % 4 == 0 and 16-byte
// aligned X, W, bias and Y.  Measured on MI355X at config 1 (M = 11264,
// K = 96, N = 288; HIP-graph replays): 8.05 us (the tiled core: 9.4 us).
// Staging W per workgroup is what costs: with all 288 columns in one
// workgroup and W converted through registers it took 6.3 of 12.5 us; half
// the columns per workgroup and eight waves brought that form to 7.8 us,
// and the same kernel with no W, X or Y traffic still takes 3.1 us.
constexpr int kPanelWaves = 8;
constexpr int kPanelThreads = kPanelWaves * kWave;
constexpr int kPanelRows = 16 * kPanelWaves;
constexpr int kPanelMaxFrags = 9;  // column blocks per half: N <= 288

inline int panel_cols(int N) { return 16 * (((N + 15) / 16 + 1) / 2); }  // per column half
inline size_t panel_lds_bytes(int N, int ks) { return (size_t)panel_cols(N) * 8 * ks * 16; }

template <int KS>
__global__ __launch_bounds__(kPanelThreads) void gemm_f32_panel_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ y, int M, int K, int N, int NC, int relu) {
    extern __shared__ __attribute__((aligned(16))) float swf[];
    constexpr int kChunks = 8 * KS;  // 16-byte chunks per padded W row
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = (int)blockIdx.y * NC;
    const int nc = min(NC, N - n0);  // columns of this half
    const int row = (int)blockIdx.x * kPanelRows + 16 * wave + (lane & 15);
    const bool row_ok = row < M;

    // W rows n0 .. n0 + NC - 1 -> LDS: LDS chunk L = n * kChunks + s holds
    // global chunk c = s ^ (n & 7) of row n0 + n (zero past N or K).
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(w, (uint32_t)N * K * 4);
    const int total = NC * kChunks;
    for (int i = wave; i * 64 < total; i += kPanelWaves) {
        const int L = 64 * i + lane;
        const int n = L / kChunks, c = (L % kChunks) ^ (n & 7);
        const bool in = L < total && n < nc && 4 * c < K;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void *)(swf + 256 * i), 16,
            in ? (uint32_t)(((n0 + n) * K + 4 * c) * 4) : kDmaOutOfRange, 0, 0, 0);
    }
    // This lane's X operands (row `row`, k = 32 ks + 8 (lane >> 4) .. + 7)
    // and the bias of its column quads 16 f + 4 (lane >> 4), f < NC / 16.
    const int col4 = 4 * (lane >> 4);
    float4 xa[KS][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 32 * ks + 8 * (lane >> 4) + 4 * h;
            xa[ks][h] = row_ok && k < K ? *reinterpret_cast<const float4 *>(x + (size_t)row * K + k)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    float4 bq[kPanelMaxFrags];
#pragma unroll
    for (int f = 0; f < kPanelMaxFrags; ++f)
        bq[f] = bias && 16 * f + col4 < nc ? *reinterpret_cast<const float4 *>(bias + n0 + 16 * f + col4)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
    bf16x8 xb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const float t[8] = {xa[ks][0].x, xa[ks][0].y, xa[ks][0].z, xa[ks][0].w,
                            xa[ks][1].x, xa[ks][1].y, xa[ks][1].z, xa[ks][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xb[ks][e] = to_bf16(t[e]);
    }
    wait_vmcnt<0>();
    __syncthreads();

    const int nl = lane & 15;  // the lane's W row within a column block
#pragma unroll
    for (int f = 0; f < kPanelMaxFrags; ++f) {
        if (16 * f >= NC) break;
        const int n = 16 * f + nl;
        const float *wr = swf + n * kChunks * 4;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int c = 8 * ks + 2 * (lane >> 4);
            const float4 lo = *reinterpret_cast<const float4 *>(wr + 4 * (c ^ (n & 7)));
            const float4 hi = *reinterpret_cast<const float4 *>(wr + 4 * ((c + 1) ^ (n & 7)));
            const bf16x8 a = {to_bf16(lo.x), to_bf16(lo.y), to_bf16(lo.z), to_bf16(lo.w),
                              to_bf16(hi.x), to_bf16(hi.y), to_bf16(hi.z), to_bf16(hi.w)};
            acc = mfma16(a, xb[ks], acc);
        }
        // acc[r]: output column n0 + 16 f + 4 (lane >> 4) + r of row `row`.
        const int col = 16 * f + col4;
        float4 v = make_float4(acc[0] + bq[f].x, acc[1] + bq[f].y, acc[2] + bq[f].z, acc[3] + bq[f].w);
        if (relu) {  // NaN passes through, as in the reference's ReLU
            v.x = v.x < 0.f ? 0.f : v.x; v.y = v.y < 0.f ? 0.f : v.y;
            v.z = v.z < 0.f ? 0.f : v.z; v.w = v.w < 0.f ? 0.f : v.w;
        }
        if (row_ok && col < nc) *reinterpret_cast<float4 *>(y + (size_t)row * N + n0 + col) = v;
    }
}

// The panel kernel for (M, K, N), or false when the shape is not one it takes.
bool gemm_f32_panel(const float *x, const float *w, const float *b, float *y, int M, int K, int N,
                    int relu, hipStream_t s) {
    if (K > 128 || (K & 3) || (N & 3) || N <= 144 || N > 2 * 16 * kPanelMaxFrags ||
        (long long)N * K * 4 >= (1ll << 31) || !aligned16(x) || !aligned16(w) || !aligned16(y) ||
        (b && !aligned16(b)))
        return false;
    const int ks = (K + 31) / 32;
    const size_t lds = panel_lds_bytes(N, ks);
    if (lds > 65536) return false;
    const dim3 grid((M + kPanelRows - 1) / kPanelRows, 2);
    const int nc = panel_cols(N);
    switch (ks) {
        case 1: hipLaunchKernelGGL(gemm_f32_panel_kernel<1>, grid, dim3(kPanelThreads), lds, s, x, w, b, y, M, K, N, nc, relu); break;
        case 2: hipLaunchKernelGGL(gemm_f32_panel_kernel<2>, grid, dim3(kPanelThreads), lds, s, x, w, b, y, M, K, N, nc, relu); break;
        case 3: hipLaunchKernelGGL(gemm_f32_panel_kernel<3>, grid, dim3(kPanelThreads), lds, s, x, w, b, y, M, K, N, nc, relu); break;
        default: hipLaunchKernelGGL(gemm_f32_panel_kernel<4>, grid, dim3(kPanelThreads), lds, s, x, w, b, y, M, K, N, nc, relu); break;
    }
    return true;
}

template <bool VEC>
void gemm_f32_dispatch(const float *x, const float *w, const float *b, float *y, int M, int K,
                       int N, int relu, hipStream_t s) {
    // 144 < N <= 288 (shapes the panel kernel does not take: K > 128 or
    // unaligned operands): 32 x 144 tiles, whole column halves; at BASELINE
    // config 1 (M = 11264, N = 288, K = 96) on MI355X 9.6 us vs 10.5 us as
    // 128 x 128 tiles (whose third column tile is 75 % empty).
    if (N <= 32)
        gemm_f32_launch<Tile<128, 32, 32, 4, 1>, VEC>(x, w, b, y, M, K, N, relu, s);
    else if (N <= 64)
        gemm_f32_launch<Tile<128, 64, 32, 4, 1>, VEC>(x, w, b, y, M, K, N, relu, s);
    else if (N > 144 && N <= 288)
        gemm_f32_launch<Tile<32, 144, 32, 2, 3>, VEC>(x, w, b, y, M, K, N, relu, s);
    else
        gemm_f32_launch<Tile<128, 128, 32, 2, 2>, VEC>(x, w, b, y, M, K, N, relu, s);
}

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
    if (gemm_f32_panel(input, weight, bias, output, rows, in_f, out_f, relu, s))
        ;  // short reduction: one pass per row panel
    else if ((in_f & 3) == 0 && aligned16(input) && aligned16(weight))
        gemm_f32_dispatch<true>(input, weight, bias, output, rows, in_f, out_f, relu, s);
    else
        gemm_f32_dispatch<false>(input, weight, bias, output, rows, in_f, out_f, relu, s);
    return launch_ok(error, cap, "HIP GEMM launch");
}
