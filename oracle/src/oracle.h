/*
 * CPU oracle: a C11 restatement of the reference's scalar CPU path for the
 * camera dense-contraction hot path. TEST INFRASTRUCTURE ONLY: it is the
 * checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * compare the HIP library against; no product code links or calls it.
 *
 * Function names, argument meaning, workspace sizes and error behaviour follow
 * the reference headers they restate:
 *   bf_kernels.h        -> reference include/bf_kernels.h:11-87, src/kernels_ref.c:16-475
 *   bf_swin.h           -> reference include/bf_swin.h:7-46,     src/swin.c:16-311
 *   bf_swin_backbone.h  -> reference include/bf_swin_backbone.h, src/swin_backbone.c:38-352
 *   bf_image_fpn.h      -> reference include/bf_image_fpn.h,     src/image_fpn.c:73-197
 *   bf_depth_head.h     -> reference include/bf_depth_head.h,    src/depth_head.c:96-190
 *   bf_lss_downsample.h -> reference include/bf_lss_downsample.h, src/lss_downsample.c:70-148
 *   bf_lss.h            -> reference include/bf_lss.h:18-46,     src/lss.c:8-241
 *   bf_bev_stage.h      -> reference include/bf_bev_stage.h,     src/bev_stage.c:16-227
 *   bf_transfusion*.h   -> reference include/bf_transfusion*.h,  src/transfusion.c:8-193,
 *                          src/transfusion_decoder.c:23-456
 *   bf_depth_raster.h   -> reference include/bf_depth_raster.h,  src/depth_raster.c:14-105
 *   bf_voxel.h          -> reference include/bf_voxel.h:30-45,   src/voxel.c:13-151
 *   bf_lidar_backbone.h -> reference include/bf_lidar_backbone.h, src/lidar_backbone.c:86-273,
 *                          with MeanVFE and the sparse conv of src/kernels_ref.c:477-772
 * Floating-point operation order matches the reference per output element, so
 * the scalar build (no OpenMP, BF_CPU_SCALAR=1) is bit-identical to the
 * reference compiled from its own sources (oracle/_ref).
 */
#ifndef BF_ORACLE_H
#define BF_ORACLE_H

#include "bevfusion.h"
#include "bf_sparse_types.h"
#include "bf_lss.h"
#include "bf_voxel.h"
#include "bf_model.h"
#include "bf_transfusion_decoder.h"
#include "bf_runtime.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- operator library (bf_kernels.h) ---------------------------------- */
typedef struct {
    size_t n, in_channels, in_height, in_width;
    size_t out_channels, kernel_height, kernel_width;
    size_t stride_height, stride_width;
    size_t pad_height, pad_width;
    size_t dilation_height, dilation_width;
    size_t groups;
} bf_conv2d_desc;

typedef struct {
    size_t n, in_channels, in_height, in_width;
    size_t out_channels, kernel_height, kernel_width;
    size_t stride_height, stride_width;
    size_t pad_height, pad_width;
    size_t output_pad_height, output_pad_width;
    size_t dilation_height, dilation_width;
    size_t groups;
} bf_conv_transpose2d_desc;

const char *bf_cpu_kernel_backend(void);
int bf_conv2d_output_shape(const bf_conv2d_desc *d, size_t *oh, size_t *ow);
int bf_conv2d_f32_ref(const float *input, const float *weight, const float *bias,
                      float *output, const bf_conv2d_desc *d);
int bf_conv2d_f32(const float *input, const float *weight, const float *bias,
                  float *output, const bf_conv2d_desc *d);
int bf_conv_transpose2d_output_shape(const bf_conv_transpose2d_desc *d,
                                     size_t *oh, size_t *ow);
int bf_conv_transpose2d_f32_ref(const float *input, const float *weight_iohw,
                                const float *bias, float *output,
                                const bf_conv_transpose2d_desc *d);
void bf_linear_f32_ref(const float *input, const float *weight, const float *bias,
                       float *output, size_t rows, size_t in_f, size_t out_f);
void bf_linear_f32(const float *input, const float *weight, const float *bias,
                   float *output, size_t rows, size_t in_f, size_t out_f);
void bf_batch_norm_2d_f32_ref(const float *input, const float *scale,
                              const float *bias, const float *mean,
                              const float *variance, float epsilon, float *output,
                              size_t n, size_t channels, size_t height, size_t width);
void bf_batch_norm_2d_f32(const float *input, const float *scale,
                          const float *bias, const float *mean,
                          const float *variance, float epsilon, float *output,
                          size_t n, size_t channels, size_t height, size_t width);
void bf_layer_norm_f32_ref(const float *input, const float *scale, const float *bias,
                           float epsilon, float *output, size_t rows, size_t channels);
void bf_layer_norm_f32(const float *input, const float *scale, const float *bias,
                       float epsilon, float *output, size_t rows, size_t channels);
void bf_softmax_f32_ref(const float *input, float *output, size_t rows, size_t columns);
void bf_gelu_f32_ref(const float *input, float *output, size_t count);
void bf_gelu_f32(const float *input, float *output, size_t count);
void bf_relu_f32_ref(const float *input, float *output, size_t count);
void bf_relu_f32(const float *input, float *output, size_t count);

/* ---- shifted-window attention (bf_swin.h) ----------------------------- */
typedef struct {
    size_t batches, height, width, channels, heads, window_size, shift_size;
} bf_swin_window_desc;

int bf_swin_window_attention_f32_ref(
    const float *windows, const float *qkv_weight, const float *qkv_bias,
    const float *relative_bias, const int64_t *relative_index,
    const float *mask, size_t mask_windows,
    const float *projection_weight, const float *projection_bias,
    float *output, size_t total_windows, size_t tokens, size_t channels,
    size_t heads, size_t relative_bias_rows);
int bf_swin_shifted_window_f32_ref(
    const float *query, const float *qkv_weight, const float *qkv_bias,
    const float *relative_bias, const int64_t *relative_index,
    const float *projection_weight, const float *projection_bias,
    float *output, const bf_swin_window_desc *desc);
size_t bf_swin_shifted_window_workspace_bytes(const bf_swin_window_desc *desc);
int bf_swin_shifted_window_f32_workspace_ref(
    const float *query, const float *qkv_weight, const float *qkv_bias,
    const float *relative_bias, const int64_t *relative_index,
    const float *projection_weight, const float *projection_bias,
    float *output, const bf_swin_window_desc *desc,
    void *workspace, size_t workspace_bytes);

/* ---- Swin-T backbone (bf_swin_backbone.h) ----------------------------- */
typedef struct bf_swin_backbone bf_swin_backbone;
typedef struct {
    size_t height[3], width[3], channels[3];
} bf_swin_backbone_shapes;
int bf_swin_backbone_create(const bf_model *model, bf_swin_backbone **out,
                            char *error, size_t cap);
void bf_swin_backbone_destroy(bf_swin_backbone *net);
int bf_swin_backbone_output_shapes(size_t input_height, size_t input_width,
                                   bf_swin_backbone_shapes *shapes);
size_t bf_swin_backbone_workspace_bytes(size_t batches, size_t input_height,
                                        size_t input_width);
int bf_swin_backbone_forward_ref(const bf_swin_backbone *net, const float *input,
                                 size_t batches, size_t input_height,
                                 size_t input_width, float *out1, float *out2,
                                 float *out3, void *workspace,
                                 size_t workspace_bytes, char *error, size_t cap);

/* ---- image FPN (bf_image_fpn.h) --------------------------------------- */
typedef struct bf_image_fpn bf_image_fpn;
int bf_image_fpn_create(const bf_model *model, bf_image_fpn **out,
                        char *error, size_t cap);
void bf_image_fpn_destroy(bf_image_fpn *fpn);
size_t bf_image_fpn_workspace_bytes(size_t height, size_t width);
int bf_image_fpn_forward_ref(const bf_image_fpn *fpn, const float *input0,
                             const float *input1, const float *input2,
                             size_t batches, size_t h0, size_t w0,
                             float *output0, float *output1, void *workspace,
                             size_t workspace_bytes, char *error, size_t cap);

/* ---- DepthLSS head (bf_depth_head.h) ---------------------------------- */
typedef struct bf_depth_head bf_depth_head;
int bf_depth_head_create(const bf_model *model, bf_depth_head **out,
                         char *error, size_t cap);
void bf_depth_head_destroy(bf_depth_head *head);
size_t bf_depth_head_workspace_bytes(size_t height, size_t width);
int bf_depth_head_forward_ref(const bf_depth_head *head, const float *features,
                              const float *depth, size_t camera_batches,
                              size_t height, size_t width, float *logits,
                              float *context, void *workspace,
                              size_t workspace_bytes, char *error, size_t cap);

/* ---- post-LSS downsample (bf_lss_downsample.h) ------------------------ */
typedef struct bf_lss_downsample bf_lss_downsample;
int bf_lss_downsample_create(const bf_model *model, bf_lss_downsample **out,
                             char *error, size_t cap);
void bf_lss_downsample_destroy(bf_lss_downsample *down);
size_t bf_lss_downsample_workspace_bytes(size_t height, size_t width);
int bf_lss_downsample_forward_ref(const bf_lss_downsample *down, const float *input,
                                  size_t batches, size_t height, size_t width,
                                  float *output, void *workspace,
                                  size_t workspace_bytes, char *error, size_t cap);

/* ---- LiDAR side (bf_depth_raster.h, bf_voxel.h, bf_lidar_backbone.h) -- */
int bf_depth_rasterize_f32_ref(const float *points, size_t point_count, size_t point_stride,
                               const float *lidar_augmentation, const float *lidar_to_image,
                               const float *image_augmentation, float *dense_depth,
                               size_t batches, size_t cameras, size_t image_height,
                               size_t image_width);
int bf_voxel_grid_shape(const bf_voxel_config *config, size_t grid_xyz[3]);
size_t bf_voxelize_workspace_bytes(const bf_voxel_config *config);
int bf_voxelize_f32_workspace_ref(const float *points, size_t point_count, size_t point_stride,
                                  int32_t batch_index, const bf_voxel_config *config,
                                  float *voxels, bf_coord4 *coords, int64_t *counts,
                                  size_t *voxel_count, bf_voxel_stats *stats, void *workspace,
                                  size_t workspace_bytes);
void bf_mean_vfe_f32_ref(const float *points, const int64_t *counts, float *output,
                         size_t voxels, size_t max_points, size_t channels);
int bf_sparse_conv3d_output_shape(const bf_sparse_conv3d_desc *desc, size_t *depth,
                                  size_t *height, size_t *width);
size_t bf_sparse_conv3d_workspace_bytes(size_t input_capacity, size_t output_capacity);
int bf_sparse_conv3d_f32_workspace_ref(const bf_coord4 *input_coords,
                                       const float *input_features, size_t input_count,
                                       const float *weight_kdhwio, const float *bias,
                                       bf_coord4 *output_coords, float *output_features,
                                       size_t output_capacity, size_t *output_count,
                                       const bf_sparse_conv3d_desc *desc, void *workspace,
                                       size_t workspace_bytes);
typedef struct bf_lidar_backbone bf_lidar_backbone;
int bf_lidar_backbone_create(const bf_model *model, bf_lidar_backbone **out, char *error,
                             size_t cap);
void bf_lidar_backbone_destroy(bf_lidar_backbone *backbone);
size_t bf_lidar_backbone_workspace_bytes(size_t capacity);
int bf_lidar_backbone_output_shape(size_t depth, size_t height, size_t width, size_t *out_depth,
                                   size_t *out_height, size_t *out_width);
/* voxel features [N,5] MeanVFE; dense [B,128,D',H',W'] (logically [B,256,H',W']). */
int bf_lidar_backbone_forward_ref(const bf_lidar_backbone *backbone,
                                  const bf_coord4 *voxel_coords, const float *voxel_features,
                                  size_t voxel_count, size_t batches, size_t depth,
                                  size_t height, size_t width, size_t capacity, float *dense,
                                  void *workspace, size_t workspace_bytes, char *error,
                                  size_t cap);

/* ---- shared helpers (internal to the oracle) --------------------------- */
int bf_oracle_fail(char *error, size_t cap, const char *fmt, ...);
int bf_oracle_mul(size_t a, size_t b, size_t *out);
const void *bf_oracle_bind(const bf_model *model, const char *name, uint32_t dtype,
                           uint32_t rank, const uint32_t *dims,
                           char *error, size_t cap);

/* ---- BEV stage (bf_bev_stage.h) --------------------------------------- */
typedef struct bf_bev_stage bf_bev_stage;
int bf_bev_stage_create(const bf_model *model, bf_bev_stage **out, char *error,
                        size_t error_cap);
void bf_bev_stage_destroy(bf_bev_stage *stage);
size_t bf_bev_stage_workspace_bytes(size_t height, size_t width);
/* input [B,336,H,W] (image 80 channels, then lidar 256); spatial [B,512,H,W];
 * shared [B,128,H,W]; heatmap [B,10,H,W] raw logits. */
int bf_bev_stage_forward_ref(const bf_bev_stage *stage, const float *input_b336hw,
                             size_t batches, size_t height, size_t width,
                             float *spatial_b512hw, float *shared_b128hw,
                             float *heatmap_b10hw, void *workspace, size_t workspace_bytes,
                             char *error, size_t error_cap);

/* ---- TransFusion head (bf_transfusion.h, bf_transfusion_decoder.h) ---- */
int bf_transfusion_select_proposals_f32_ref(const float *dense_heatmap_logits_bchw,
                                            float *suppressed_heatmap_bchw,
                                            float *proposal_scores_bk, int64_t *proposal_classes_bk,
                                            int64_t *proposal_indices_bk, size_t batches,
                                            size_t classes, size_t height, size_t width,
                                            size_t proposals, size_t nms_kernel_size);
int bf_transfusion_decode_raw_f32_ref(const float *heatmap_logits_bcp,
                                      const float *query_heatmap_scores_bcp,
                                      const int64_t *query_labels_bp, const float *center_b2p,
                                      const float *height_b1p, const float *dimension_log_b3p,
                                      const float *rotation_sincos_b2p, const float *velocity_b2p,
                                      float *boxes_bp9, float *scores_bp, int64_t *labels_bp,
                                      size_t batches, size_t classes, size_t proposals,
                                      float feature_stride, const float voxel_size_xy[2],
                                      const float point_cloud_minimum_xy[2]);
int bf_transfusion_filter_detections(const float *boxes_bp9, const float *scores_bp,
                                     const int64_t *labels_bp, size_t batches, size_t proposals,
                                     float score_threshold, const float post_center_range[6],
                                     bf_detections *output);
typedef struct bf_transfusion_decoder bf_transfusion_decoder;
int bf_transfusion_decoder_create(const bf_model *model, bf_transfusion_decoder **out,
                                  char *error, size_t error_cap);
void bf_transfusion_decoder_destroy(bf_transfusion_decoder *decoder);
size_t bf_transfusion_decoder_workspace_bytes(size_t height, size_t width, size_t proposals);
int bf_transfusion_decoder_forward_ref(const bf_transfusion_decoder *decoder,
                                       const float *shared_b128hw,
                                       const float *dense_heatmap_logits_b10hw, size_t batches,
                                       size_t height, size_t width, size_t proposals,
                                       bf_transfusion_raw_outputs *outputs, void *workspace,
                                       size_t workspace_bytes, char *error, size_t error_cap);

/* ---- frame runtime (reference include/bf_runtime.h:29-49) ------------- */
typedef struct bf_runtime bf_runtime;
int bf_runtime_create(const char *model_path, bf_runtime **out, char *error, size_t cap);
void bf_runtime_destroy(bf_runtime *runtime);
size_t bf_runtime_workspace_bytes(size_t point_capacity, size_t voxel_capacity,
                                  size_t sparse_capacity);
int bf_runtime_infer_cpu_ref(const bf_runtime *runtime, const bf_frame_input *frame,
                             size_t point_capacity, size_t voxel_capacity,
                             size_t sparse_capacity, bf_detections *detections,
                             void *workspace, size_t workspace_bytes, char *error, size_t cap);

/* ---- lift-splat pooling (bf_lss.h) ------------------------------------ */
int bf_lss_geometry_f32_ref(const float *frustum_dhw3, const float *camera_to_lidar_rotation,
                            const float *camera_to_lidar_translation, const float *intrinsics,
                            const float *post_rotation, const float *post_translation,
                            const float *extra_rotation, const float *extra_translation,
                            float *geometry_bndhw3, size_t batches, size_t cameras,
                            size_t depth_bins, size_t height, size_t width);
int bf_lss_lift_f32_ref(const float *depth_logits_bndhw, const float *context_bnchw,
                        float *lifted_bndhwc, const bf_lss_desc *desc);
int bf_lss_bev_pool_f32_ref(const float *lifted_bndhwc, const float *geometry_bndhw3,
                            float *bev_bczxy, const bf_lss_desc *desc);
int bf_lss_lift_pool_f32_ref(const float *depth_logits_bndhw, const float *context_bnchw,
                             const float *geometry_bndhw3, float *bev_bczxy,
                             const bf_lss_desc *desc);
/* Test helper (no reference counterpart): per-sample cell rank within its
 * batch, (z * X + x) * Y + y, -1 outside the grid. */
int bf_oracle_lss_ranks(const float *geometry_bndhw3, int32_t *ranks, const bf_lss_desc *desc);

#ifdef __cplusplus
}
#endif

#endif
