/*
 * Lift-splat-shoot pooling on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda.h:11-87 (implemented there by
 * src/cuda_lss.cu): same names, argument meaning and error convention
 * (1 = success, 0 = failure with a message in error[0..error_cap)).  All
 * tensor pointers are device pointers; stream is a hipStream_t or NULL.
 *
 *   depth_logits [B,N,D,H,W], context [B,N,C,H,W], geometry [B,N,D,H,W,3]
 *   (metric points), bev [B,C*Z,X,Y] fp32 (bf_lss.h); D <= 128.
 *
 * Routes:
 *   bf_cuda_lss_lift_pool_f32 / _ranks_f32   stateless; accumulate with
 *       float atomics as the reference does, so the summation order (and the
 *       last bits of a cell) may differ between calls.
 *   bf_cuda_lss_plan_*                        deterministic and atomics-free:
 *       prepare maps every sample to its BEV cell and lists each cell's
 *       samples in ascending sample order (a stable sort by cell);
 *       forward = depth softmax + a gather per cell in that fixed order, so
 *       repeated forwards are bit-identical.  forward allocates nothing and
 *       may be captured into a HIP graph; one forward at a time per plan.
 * A point lands in cell trunc((p - minimum) / step) per axis when inside the
 * grid; its rank within a batch is (z * X + x) * Y + y, -1 outside.
 */
#ifndef BF_CUDA_H
#define BF_CUDA_H

#include "bf_lss.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int bf_cuda_available(char *error, size_t error_cap);

int bf_cuda_lss_lift_pool_f32(
    const float *depth_logits_device,
    const float *context_device,
    const float *geometry_device,
    float *bev_device,
    const bf_lss_desc *desc,
    void *stream,
    char *error, size_t error_cap);

/* [B,N,D,H,W,3] metric geometry -> B*N*D*H*W int32 cell ranks (-1 outside). */
int bf_cuda_lss_geometry_to_ranks_f32(
    const float *geometry_device,
    int *ranks_device,
    const bf_lss_desc *desc,
    void *stream,
    char *error, size_t error_cap);

int bf_cuda_lss_lift_pool_ranks_f32(
    const float *depth_logits_device,
    const float *context_device,
    const int *ranks_device,
    float *bev_device,
    const bf_lss_desc *desc,
    void *stream,
    char *error, size_t error_cap);

typedef struct bf_cuda_lss_plan bf_cuda_lss_plan;

int bf_cuda_lss_plan_create(
    const bf_lss_desc *desc,
    bf_cuda_lss_plan **out,
    char *error, size_t error_cap);
void bf_cuda_lss_plan_destroy(bf_cuda_lss_plan *plan);
size_t bf_cuda_lss_plan_resident_bytes(const bf_cuda_lss_plan *plan);

/* Cell lists from metric geometry. */
int bf_cuda_lss_plan_prepare_geometry_f32(
    bf_cuda_lss_plan *plan,
    const float *geometry_device,
    void *stream,
    char *error, size_t error_cap);

/* Cell lists straight from the calibration (no geometry tensor): frustum
 * [D,H,W,3], per-camera rotation/intrinsics/post-rotation [B,N,3,3] and
 * translations [B,N,3]; the per-batch extra rotation [B,3,3] / translation
 * [B,3] may be NULL.  A camera whose post-rotation or intrinsics is singular
 * contributes no samples. */
int bf_cuda_lss_plan_prepare_calibration_f32(
    bf_cuda_lss_plan *plan,
    const float *frustum_dhw3_device,
    const float *camera_rotation_bn33_device,
    const float *camera_translation_bn3_device,
    const float *intrinsics_bn33_device,
    const float *post_rotation_bn33_device,
    const float *post_translation_bn3_device,
    const float *extra_rotation_b33_device,
    const float *extra_translation_b3_device,
    void *stream,
    char *error, size_t error_cap);

int bf_cuda_lss_plan_forward_f32(
    bf_cuda_lss_plan *plan,
    const float *depth_logits_device,
    const float *context_device,
    float *bev_device,
    void *stream,
    char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
