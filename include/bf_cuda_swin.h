/*
 * Fixed-shape Swin-T camera backbone context, served on AMD gfx950 by
 * libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_swin.h:12-31 (implemented there
 * by src/cuda_swin.cu:249-421).  Same names, argument meaning and error
 * convention (1 = success, 0 = failure with a message in error[0..cap)).
 *
 *   create:   binds the Swin-T tensors of a BFW container by name and shape
 *             (reference cuda_swin.cu:290-317), converts linear weights to
 *             fp16 and uploads them (the forward multiplies fp16 operands
 *             with fp32 accumulation); input height/width must be multiples
 *             of 4.  The model mapping need only outlive this call.
 *   forward:  images [B,3,H,W] fp32 -> stage outputs
 *             [B,192,H/8,W/8], [B,384,H/16,W/16], [B,768,H/32,ceil(W/32)]
 *             fp32 NCHW; all device pointers; stream is a hipStream_t.
 *             Allocates nothing, so it may be captured into a HIP graph.
 *             One forward at a time per context.
 */
#ifndef BF_CUDA_SWIN_H
#define BF_CUDA_SWIN_H

#include "bf_model.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_swin bf_cuda_swin;

int bf_cuda_swin_create(const bf_model *model, size_t batches,
                        size_t input_height, size_t input_width,
                        bf_cuda_swin **out,
                        char *error, size_t error_cap);
void bf_cuda_swin_destroy(bf_cuda_swin *swin);
size_t bf_cuda_swin_resident_bytes(const bf_cuda_swin *swin);

int bf_cuda_swin_forward(bf_cuda_swin *swin,
                         const float *images_b3hw_device,
                         float *stage1_b192hw_device,
                         float *stage2_b384hw_device,
                         float *stage3_b768hw_device,
                         void *stream,
                         char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
