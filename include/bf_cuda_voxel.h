/*
 * Voxeliser with MeanVFE on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_voxel.h:10-31 (implemented
 * there by src/cuda_voxel.cu:157-307): same names, argument meaning and
 * error convention (1 = success, 0 = failure with a message in
 * error[0..error_cap)).
 *
 * Points [P,5] (x, y, z, intensity, time) in, device pointers throughout;
 * stream is a hipStream_t or NULL.  Voxels come out in first-encounter order
 * exactly as the reference CPU voxeliser makes them (a voxel is created at
 * its first point until max_voxels exist, keeps its first
 * max_points_per_voxel points, non-finite and out-of-range points are
 * rejected): coords [V] (batch 0, z, y, x), mean features [V,5] (the mean of
 * the kept points, summed in input order, bit-identical to the CPU MeanVFE)
 * and the voxel count as one device uint32.  config->point_features must be 5.
 * create clears a dense per-cell word grid (4 bytes per voxel cell); a call
 * allocates nothing, issues no memset and no host synchronisation (it can be
 * captured in a HIP graph); one call at a time per context.
 */
#ifndef BF_CUDA_VOXEL_H
#define BF_CUDA_VOXEL_H

#include "bf_sparse_types.h"
#include "bf_voxel.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_voxelizer bf_cuda_voxelizer;

int bf_cuda_voxelizer_create(const bf_voxel_config *config,
                             size_t max_input_points,
                             bf_cuda_voxelizer **out,
                             char *error, size_t error_cap);
void bf_cuda_voxelizer_destroy(bf_cuda_voxelizer *voxelizer);
size_t bf_cuda_voxelizer_resident_bytes(const bf_cuda_voxelizer *voxelizer);

int bf_cuda_voxelize_mean_f32(bf_cuda_voxelizer *voxelizer,
                              const float *points_p5_device,
                              size_t point_count,
                              bf_coord4 *coords_device,
                              float *mean_features_v5_device,
                              unsigned *voxel_count_device,
                              void *stream,
                              char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
