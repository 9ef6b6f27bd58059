/*
 * LiDAR-to-image depth raster on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_depth_raster.h:7-29
 * (implemented there by src/cuda_depth_raster.cu:34-38): same names,
 * argument meaning and error convention (1 = success, 0 = failure with a
 * message in error[0..error_cap)).
 *
 * Batch-one frame contract: points [P,5] x/y/z/intensity/time; the lidar
 * augmentation [16], lidar-to-image [N,16] and image augmentation [N,16]
 * row-major 4x4 matrices and the output [N,H,W] are device pointers; stream
 * is a hipStream_t or NULL.  A point projects into camera n at pixel
 * (floor x, floor y) with depth clamp(z, 1e-5, 1e5); later input points win
 * pixel collisions, exactly as the ordered scalar assignment of the
 * reference CPU raster, and every depth is bit-identical to it.  A singular
 * lidar augmentation leaves the image zero.  Rasterising allocates nothing
 * and issues no memset (graph-capturable); one call at a time per context.
 */
#ifndef BF_CUDA_DEPTH_RASTER_H
#define BF_CUDA_DEPTH_RASTER_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_depth_raster bf_cuda_depth_raster;

int bf_cuda_depth_raster_create(size_t max_points, size_t cameras,
                                size_t image_height, size_t image_width,
                                bf_cuda_depth_raster **out,
                                char *error, size_t error_cap);
void bf_cuda_depth_raster_destroy(bf_cuda_depth_raster *raster);
size_t bf_cuda_depth_raster_resident_bytes(const bf_cuda_depth_raster *raster);

int bf_cuda_depth_rasterize_f32(bf_cuda_depth_raster *raster,
                                const float *points_p5_device,
                                size_t point_count,
                                const float *lidar_augmentation_16_device,
                                const float *lidar_to_image_n16_device,
                                const float *image_augmentation_n16_device,
                                float *dense_depth_nhw_device,
                                void *stream,
                                char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
