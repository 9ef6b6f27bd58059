/*
 * Stateless operator boundary, served on AMD gfx950 by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_ops.h:15-49 (implemented there
 * by src/cuda_ops.cu:147-208).  The names and the C ABI are unchanged so the
 * reference runtime and its callers (cuda_swin.cu:244,372; cuda_camera.cu:214;
 * cuda_bev_stage.cu:308; cuda_transfusion.cu:251) link without edits.
 *
 * Conventions (reference bf_cuda_ops.h:10-14, cuda_ops.cu:13-21,150-170):
 *   - all tensor pointers are device pointers;
 *   - `stream` is a hipStream_t (NULL = the default stream);
 *   - returns 1 on success, 0 on failure with a message written to
 *     error[0..error_cap) (error may be NULL or error_cap 0);
 *   - the contract is validated before anything is launched, launch errors
 *     are reported from hipGetLastError.
 * Arithmetic: fp32 in, fp32 out; operands are rounded to bf16 on the way into
 * the matrix cores and products accumulate in fp32.  Inf/NaN propagate.
 */
#ifndef BF_CUDA_OPS_H
#define BF_CUDA_OPS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Convolution descriptor; weights are OIHW, or IOHW when transpose == 1
 * (reference bf_cuda_ops.h:15-31). */
typedef struct {
    int batches;
    int input_channels;
    int output_channels;
    int input_height;
    int input_width;
    int kernel_height;
    int kernel_width;
    int stride_height;
    int stride_width;
    int padding_height;
    int padding_width;
    int output_height;
    int output_width;
    int transpose;
    int relu;
} bf_cuda_conv2d_desc;

/* NCHW implicit-GEMM convolution with optional bias and fused ReLU
 * (replaces reference src/cuda_ops.cu:147-186). */
int bf_cuda_conv2d_f32(const bf_cuda_conv2d_desc *desc,
                       const float *input,
                       const float *weight,
                       const float *bias,
                       float *output,
                       void *stream,
                       char *error, size_t error_cap);

/* Row-major output[M,N] = input[M,K] * weight[N,K]^T + bias[N], optional
 * fused ReLU (replaces reference src/cuda_ops.cu:188-208). */
int bf_cuda_gemm_f32(const float *input, const float *weight,
                     const float *bias, float *output,
                     int rows, int input_features, int output_features,
                     int relu, void *stream,
                     char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
