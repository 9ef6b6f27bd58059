/*
 * Frame boundary of the BEVFusion runtime (batch one, six cameras).
 *
 * Same type as the reference's include/bf_runtime.h:14-27, so frames read by
 * a BFI reader or built by a caller pass to bf_cuda_runtime_infer unchanged.
 * The reference's scalar CPU runtime declared beside it there
 * (bf_runtime_create / bf_runtime_infer_cpu_ref / bf_runtime_workspace_bytes)
 * is not served by libbfhip.so.
 */
#ifndef BF_RUNTIME_H
#define BF_RUNTIME_H

#include "bevfusion.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    /* [6,3,256,704], already resized and normalised (ImageNet mean/std). */
    const float *camera_images;
    /* [point_count,5]: x, y, z, intensity, timestamp in the augmented lidar frame. */
    const float *points;
    size_t point_count;
    /* Row-major homogeneous 4x4 matrices. */
    const float *camera_intrinsics_6x16;
    const float *camera_to_lidar_6x16;
    const float *image_augmentation_6x16;
    const float *lidar_augmentation_16;
    const float *lidar_to_image_6x16;
} bf_frame_input;

#ifdef __cplusplus
}
#endif

#endif
