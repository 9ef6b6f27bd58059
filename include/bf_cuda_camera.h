/*
 * Camera neck context (GeneralizedLSSFPN, DepthLSS head, post-LSS
 * downsample), served on AMD gfx950 by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_camera.h:12-63 (implemented
 * there by src/cuda_camera.cu:273-426).  Same names, argument meaning and
 * error convention.  All BatchNorm layers are folded into the convolution
 * weights at create (w*g/sqrt(v+eps), (b-m)*f+beta, eps 1e-5; reference
 * cuda_camera.cu:116-122); bev_height and bev_width must be even.
 * Device pointers throughout; stream is a hipStream_t.  Forward entry points
 * allocate nothing.  One forward at a time per context.
 */
#ifndef BF_CUDA_CAMERA_H
#define BF_CUDA_CAMERA_H

#include "bf_model.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_camera_neck bf_cuda_camera_neck;

int bf_cuda_camera_neck_create(const bf_model *model,
                               size_t camera_batches,
                               size_t feature_height,
                               size_t feature_width,
                               size_t bev_height,
                               size_t bev_width,
                               bf_cuda_camera_neck **out,
                               char *error, size_t error_cap);
void bf_cuda_camera_neck_destroy(bf_cuda_camera_neck *neck);
size_t bf_cuda_camera_neck_resident_bytes(const bf_cuda_camera_neck *neck);

/* Swin inputs [BN,192,H,W], [BN,384,ceil(H/2),ceil(W/2)],
 * [BN,768,ceil(H/4),ceil(W/4)] -> FPN levels [BN,256,H,W],
 * [BN,256,ceil(H/2),ceil(W/2)]. */
int bf_cuda_camera_fpn_forward(bf_cuda_camera_neck *neck,
                               const float *swin0_device,
                               const float *swin1_device,
                               const float *swin2_device,
                               float *fpn0_device,
                               float *fpn1_device,
                               void *stream,
                               char *error, size_t error_cap);

/* fpn0 [BN,256,H,W] + dense depth [BN,1,8H,8W] -> depth logits
 * [BN,118,H,W] and context [BN,80,H,W]. */
int bf_cuda_camera_depth_forward(bf_cuda_camera_neck *neck,
                                 const float *fpn0_device,
                                 const float *dense_depth_device,
                                 float *depth_logits_device,
                                 float *context_device,
                                 void *stream,
                                 char *error, size_t error_cap);

/* FPN followed by the depth head; FPN outputs stay context-owned. */
int bf_cuda_camera_neck_forward(bf_cuda_camera_neck *neck,
                                const float *swin0_device,
                                const float *swin1_device,
                                const float *swin2_device,
                                const float *dense_depth_device,
                                float *depth_logits_device,
                                float *context_device,
                                void *stream,
                                char *error, size_t error_cap);

/* BEV [1,80,X,Y] -> [1,80,Y/2,X/2] including the checkpoint x/y transpose. */
int bf_cuda_camera_downsample_forward(bf_cuda_camera_neck *neck,
                                      const float *full_bev_device,
                                      float *image_bev_device,
                                      void *stream,
                                      char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
