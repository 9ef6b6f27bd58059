/*
 * Full BEVFusion inference on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_runtime.h:12-43 (implemented
 * there by src/cuda_runtime.cu:53-98): same names, argument meaning and
 * error convention (1 = success, 0 = failure with a message in
 * error[0..error_cap)).
 *
 * create opens the BFW checkpoint and builds every context of the frame:
 * depth raster, voxeliser (range [-54,54]x[-54,54]x[-5,3] m, 0.075 x 0.075 x
 * 0.2 m voxels, 10 points each), SECOND encoder (41 x 1440 x 1440 grid),
 * Swin-T, camera neck, LSS plan (118 depth bins, 360 x 360 BEV), BEV stage
 * and the TransFusion decoder (180 x 180, 200 proposals).  voxel_capacity must
 * not exceed sparse_capacity.
 *
 * infer copies the frame to the device (the only host->device traffic),
 * replays three HIP graphs -- the LiDAR branch (voxeliser, sparse encoder) on
 * a second stream, concurrent with the camera branch (depth raster, Swin-T,
 * neck, lift-splat, downsample), then BEV stage, TransFusion and the
 * canonical decode at score threshold 0 -- and copies the detections back.
 * The LiDAR branch starts once the points are uploaded, while the images
 * still are.  The point count travels in device memory, so the graphs,
 * captured on the first frame, serve every frame.
 * The LSS cell lists are rebuilt (outside the graph) only when the
 * calibration differs from the previous frame's.  Singular intrinsics,
 * image-augmentation or lidar-augmentation rotations are rejected as in the
 * reference.  One infer at a time per runtime.
 *
 * debug_bev_stats: sum |x| and max |x| of the image BEV [80,180,180] and the
 * LiDAR BEV [256,180,180] of the last frame; debug_hashes: an order-free
 * hash of eleven intermediate tensors (dense depth, the three Swin stages,
 * depth logits, context, full and downsampled image BEV, LiDAR BEV, shared
 * feature, dense heatmap), each the XOR over elements i of
 * mix64((i << 32) ^ bits(x_i)) with the splitmix64 finaliser.
 */
#ifndef BF_CUDA_RUNTIME_H
#define BF_CUDA_RUNTIME_H

#include "bf_runtime.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_runtime bf_cuda_runtime;

int bf_cuda_runtime_create(const char *model_path,
                           size_t point_capacity,
                           size_t voxel_capacity,
                           size_t sparse_capacity,
                           bf_cuda_runtime **out,
                           char *error, size_t error_cap);
void bf_cuda_runtime_destroy(bf_cuda_runtime *runtime);

int bf_cuda_runtime_infer(bf_cuda_runtime *runtime,
                          const bf_frame_input *frame,
                          bf_detections *detections,
                          char *error, size_t error_cap);

size_t bf_cuda_runtime_resident_bytes(const bf_cuda_runtime *runtime);

int bf_cuda_runtime_debug_bev_stats(const bf_cuda_runtime *runtime,
                                    float stats4_host[4],
                                    char *error, size_t error_cap);

int bf_cuda_runtime_debug_hashes(const bf_cuda_runtime *runtime,
                                 unsigned long long hashes11_host[11],
                                 char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
