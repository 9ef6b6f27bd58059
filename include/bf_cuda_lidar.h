/*
 * SECOND sparse LiDAR encoder on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_lidar.h:11-43 (implemented
 * there by src/cuda_lidar.cu:86-139): same names, argument meaning and error
 * convention (1 = success, 0 = failure with a message in error[0..error_cap)).
 *
 * create binds the checkpoint's backbone_3d.* weights (input SubM conv
 * 5 -> 16, four stages of two residual SubM blocks at 16/32/64/128 channels
 * entered by 3x3x3 stride-2 convs, the (3,1,1)/(2,1,1) output conv), folds
 * eval BatchNorm (epsilon 1e-3) and sizes every buffer for `sparse_capacity`
 * active sites per layer and the batches x depth x height x width input grid.
 * forward takes device voxel coordinates (batch, z, y, x) and MeanVFE
 * features [N,5] — the count as a host size_t or, in the _count_device
 * form, as one device uint32 — and writes the dense [B,128,D',H',W'] BEV
 * (logically [B,256,H',W'] at the production D' = 2), zero where no site is
 * active.  Sites beyond the capacity are dropped, as the reference GPU path
 * does.  stream is a hipStream_t or NULL; one forward at a time per context.
 */
#ifndef BF_CUDA_LIDAR_H
#define BF_CUDA_LIDAR_H

#include "bf_sparse_types.h"
#include "bf_model.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_lidar_backbone bf_cuda_lidar_backbone;

int bf_cuda_lidar_backbone_create(const bf_model *model,
                                  size_t batches,
                                  size_t input_depth,
                                  size_t input_height,
                                  size_t input_width,
                                  size_t sparse_capacity,
                                  bf_cuda_lidar_backbone **out,
                                  char *error, size_t error_cap);
void bf_cuda_lidar_backbone_destroy(bf_cuda_lidar_backbone *backbone);
size_t bf_cuda_lidar_backbone_resident_bytes(const bf_cuda_lidar_backbone *backbone);

int bf_cuda_lidar_backbone_forward(bf_cuda_lidar_backbone *backbone,
                                   const bf_coord4 *voxel_coords_device,
                                   const float *voxel_features_v5_device,
                                   size_t voxel_count,
                                   float *dense_bev_device,
                                   void *stream,
                                   char *error, size_t error_cap);
int bf_cuda_lidar_backbone_forward_count_device(bf_cuda_lidar_backbone *backbone,
                                                const bf_coord4 *voxel_coords_device,
                                                const float *voxel_features_v5_device,
                                                const unsigned *voxel_count_device,
                                                float *dense_bev_device,
                                                void *stream,
                                                char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
