/*
 * BEV stage context on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_bev.h:12-32 (implemented there
 * by src/cuda_bev_stage.cu:220-343): same names, argument meaning and error
 * convention (1 = success, 0 = failure with a message in error[0..error_cap)).
 *
 * The stage is the fuser conv (336 -> 256), the SECOND backbone (two blocks of
 * six 3x3 convs, the second at half resolution) with its two deblocks (1x1 and
 * a transposed 2x2 stride-2 conv), and TransFusion's shared conv and heatmap
 * head: 18 BN-folded convolutions (BatchNorm epsilon 1e-3) whose weights come
 * from the model under the checkpoint's names.  Fixed shape, batch one;
 * height and width must be even.  All tensor pointers are device pointers;
 * stream is a hipStream_t or NULL.  Forward allocates nothing, so it can be
 * captured into a HIP graph; one forward at a time per context.
 *
 *   input   [1,336,H,W] fp32 (image BEV 80 channels, then lidar BEV 256)
 *   spatial [1,512,H,W] fp32 (deblock outputs, concatenated)
 *   shared  [1,128,H,W] fp32
 *   heatmap [1,10,H,W]  fp32 raw logits
 */
#ifndef BF_CUDA_BEV_H
#define BF_CUDA_BEV_H

#include "bf_model.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_bev_stage bf_cuda_bev_stage;

int bf_cuda_bev_stage_create(const bf_model *model, size_t height, size_t width,
                             bf_cuda_bev_stage **out,
                             char *error, size_t error_cap);
void bf_cuda_bev_stage_destroy(bf_cuda_bev_stage *stage);

int bf_cuda_bev_stage_forward(bf_cuda_bev_stage *stage,
                              const float *input_b336hw_device,
                              float *spatial_b512hw_device,
                              float *shared_b128hw_device,
                              float *heatmap_b10hw_device,
                              void *stream,
                              char *error, size_t error_cap);

size_t bf_cuda_bev_stage_resident_bytes(const bf_cuda_bev_stage *stage);

#ifdef __cplusplus
}
#endif

#endif
