// Launch-only forms the GPU runtime composes into one HIP graph (hidden,
// not part of the C ABI).  The point count is read from device memory and
// grids are sized by a host bound, so one captured graph serves frames of any
// point count up to the bound.
#pragma once

#include "bevfusion.h"
#include "bf_cuda_depth_raster.h"
#include "bf_cuda_transfusion.h"
#include "bf_cuda_voxel.h"

#include <stddef.h>

namespace bfhip {

__attribute__((visibility("hidden"))) int depth_rasterize_count_device(
    bf_cuda_depth_raster *raster, const float *points, const unsigned *count_device,
    size_t bound, const float *lidar_aug, const float *lidar_to_image, const float *image_aug,
    float *depth, void *stream, char *error, size_t cap);

__attribute__((visibility("hidden"))) int voxelize_count_device(
    bf_cuda_voxelizer *voxelizer, const float *points, const unsigned *count_device,
    size_t bound, bf_coord4 *coords, float *means, unsigned *voxel_count, void *stream,
    char *error, size_t cap);

// Decode kernel only; the detections stay in the decoder's device buffer.
__attribute__((visibility("hidden"))) int transfusion_decode_launch(
    bf_cuda_transfusion *decoder, const bf_transfusion_raw_outputs *outputs, float threshold,
    void *stream, const bf_detections **device_detections, char *error, size_t cap);

}  // namespace bfhip
