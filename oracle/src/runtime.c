/* CPU restatement of the reference's scalar frame runtime (TEST
 * INFRASTRUCTURE ONLY): reference src/runtime.c:238-413, batch one, six
 * cameras, the same module chain and constants:
 *   LiDAR   voxelise (range [-54,54]^2 x [-5,3] m, 0.075/0.075/0.2 m voxels,
 *           10 points, voxel_capacity) -> MeanVFE -> SECOND encoder on the
 *           41 x 1440 x 1440 grid -> LiDAR BEV [256,180,180];
 *   camera  depth raster of the points -> Swin-T -> FPN -> depth head ->
 *           LSS geometry + lift-splat (118 bins, 360 x 360 x 1 cells of
 *           0.3 m from (-54,-54,-10)) -> downsample -> image BEV [80,180,180];
 *   fusion  concat (image, LiDAR) -> BEV stage -> TransFusion (200
 *           proposals) -> box decode (stride 8, 0.075 m voxels, minimum -54)
 *           -> filter at score 0 inside [-61.2,61.2]^2 x [-10,10].
 * The workspace is planned as one region per buffer (no phase reuse), so
 * bf_runtime_workspace_bytes differs from the reference's peak-reuse plan;
 * every result is the same computation. */
#include "oracle.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CAMS 6u
#define IMG_H 256u
#define IMG_W 704u
#define FEAT_H 32u
#define FEAT_W 88u
#define BINS 118u
#define CTX 80u
#define FULL 360u
#define BEV 180u
#define PROPOSALS 200u

struct bf_runtime {
    bf_model *model;
    bf_swin_backbone *swin;
    bf_image_fpn *fpn;
    bf_depth_head *depth;
    bf_lss_downsample *down;
    bf_lidar_backbone *lidar;
    bf_bev_stage *bev;
    bf_transfusion_decoder *decoder;
    const float *frustum;
};

static void release(bf_runtime *r) {
    if (!r) return;
    bf_transfusion_decoder_destroy(r->decoder);
    bf_bev_stage_destroy(r->bev);
    bf_lidar_backbone_destroy(r->lidar);
    bf_lss_downsample_destroy(r->down);
    bf_depth_head_destroy(r->depth);
    bf_image_fpn_destroy(r->fpn);
    bf_swin_backbone_destroy(r->swin);
    bf_model_close(r->model);
    free(r);
}

int bf_runtime_create(const char *path, bf_runtime **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!path || !out) return bf_oracle_fail(error, cap, "invalid runtime arguments");
    bf_runtime *r = (bf_runtime *)calloc(1, sizeof(*r));
    if (!r) return bf_oracle_fail(error, cap, "runtime allocation failed");
    const uint32_t dims[4] = {BINS, FEAT_H, FEAT_W, 3};
    if (!bf_model_open(path, &r->model, error, cap) ||
        !bf_swin_backbone_create(r->model, &r->swin, error, cap) ||
        !bf_image_fpn_create(r->model, &r->fpn, error, cap) ||
        !bf_depth_head_create(r->model, &r->depth, error, cap) ||
        !bf_lss_downsample_create(r->model, &r->down, error, cap) ||
        !bf_lidar_backbone_create(r->model, &r->lidar, error, cap) ||
        !bf_bev_stage_create(r->model, &r->bev, error, cap) ||
        !bf_transfusion_decoder_create(r->model, &r->decoder, error, cap) ||
        !(r->frustum = (const float *)bf_oracle_bind(r->model, "vtransform.frustum",
                                                     BF_DTYPE_F32, 4, dims, error, cap))) {
        release(r);
        return 0;
    }
    *out = r;
    return 1;
}

void bf_runtime_destroy(bf_runtime *r) { release(r); }

/* Region sizes, in bytes, in carving order. */
enum {
    R_LIDAR_BEV, R_IMAGE_BEV, R_VOXELS, R_COORDS, R_COUNTS, R_VFE, R_VOXEL_WS, R_LIDAR_WS,
    R_DEPTH, R_POINTS6, R_LOGITS, R_CONTEXT, R_GEOMETRY, R_FULL_BEV, R_S0, R_S1, R_S2, R_SWIN_WS,
    R_F0, R_F1, R_FPN_WS, R_HEAD_WS, R_DOWN_WS, R_FUSION, R_SPATIAL, R_SHARED, R_HEATMAP,
    R_BEV_WS, R_DEC_WS, R_RAW, R_LABELS, R_BOXES, R_SCORES, R_OUT_LABELS, R_COUNT
};

static int plan(size_t points, size_t voxels, size_t sparse, size_t size[R_COUNT]) {
    if (!points || points > SIZE_MAX / 64 || !voxels || voxels > 160000 || !sparse ||
        sparse < voxels)
        return 0;
    const size_t F = sizeof(float), plane = (size_t)BEV * BEV;
    const bf_voxel_config vc = {{-54.0f, -54.0f, -5.0f}, {54.0f, 54.0f, 3.0f},
                                {0.075f, 0.075f, 0.2f}, 5, 10, voxels};
    size[R_LIDAR_BEV] = 256 * plane * F;
    size[R_IMAGE_BEV] = CTX * plane * F;
    size[R_VOXELS] = voxels * 10 * 5 * F;
    size[R_COORDS] = voxels * sizeof(bf_coord4);
    size[R_COUNTS] = voxels * sizeof(int64_t);
    size[R_VFE] = voxels * 5 * F;
    size[R_VOXEL_WS] = bf_voxelize_workspace_bytes(&vc);
    size[R_LIDAR_WS] = bf_lidar_backbone_workspace_bytes(sparse);
    size[R_DEPTH] = (size_t)CAMS * IMG_H * IMG_W * F;
    size[R_POINTS6] = points * 6 * F;
    size[R_LOGITS] = (size_t)CAMS * BINS * FEAT_H * FEAT_W * F;
    size[R_CONTEXT] = (size_t)CAMS * CTX * FEAT_H * FEAT_W * F;
    size[R_GEOMETRY] = (size_t)CAMS * BINS * FEAT_H * FEAT_W * 3 * F;
    size[R_FULL_BEV] = (size_t)CTX * FULL * FULL * F;
    size[R_S0] = (size_t)CAMS * 192 * 32 * 88 * F;
    size[R_S1] = (size_t)CAMS * 384 * 16 * 44 * F;
    size[R_S2] = (size_t)CAMS * 768 * 8 * 22 * F;
    size[R_SWIN_WS] = bf_swin_backbone_workspace_bytes(CAMS, IMG_H, IMG_W);
    size[R_F0] = (size_t)CAMS * 256 * 32 * 88 * F;
    size[R_F1] = (size_t)CAMS * 256 * 16 * 44 * F;
    size[R_FPN_WS] = bf_image_fpn_workspace_bytes(FEAT_H, FEAT_W);
    size[R_HEAD_WS] = bf_depth_head_workspace_bytes(FEAT_H, FEAT_W);
    size[R_DOWN_WS] = bf_lss_downsample_workspace_bytes(FULL, FULL);
    size[R_FUSION] = 336 * plane * F;
    size[R_SPATIAL] = 512 * plane * F;
    size[R_SHARED] = 128 * plane * F;
    size[R_HEATMAP] = 10 * plane * F;
    size[R_BEV_WS] = bf_bev_stage_workspace_bytes(BEV, BEV);
    size[R_DEC_WS] = bf_transfusion_decoder_workspace_bytes(BEV, BEV, PROPOSALS);
    size[R_RAW] = (2 + 1 + 3 + 2 + 2 + 10 + 10) * PROPOSALS * F;
    size[R_LABELS] = 2 * PROPOSALS * sizeof(int64_t);
    size[R_BOXES] = PROPOSALS * 9 * F;
    size[R_SCORES] = PROPOSALS * F;
    size[R_OUT_LABELS] = PROPOSALS * sizeof(int64_t);
    for (int i = 0; i < R_COUNT; ++i)
        if (!size[i]) return 0;
    return 1;
}

size_t bf_runtime_workspace_bytes(size_t points, size_t voxels, size_t sparse) {
    size_t size[R_COUNT], total = 0;
    if (!plan(points, voxels, sparse, size)) return 0;
    for (int i = 0; i < R_COUNT; ++i) total += (size[i] + 63) & ~(size_t)63;
    return total;
}

/* Rotation rows and translation column of row-major 4x4 matrices. */
static void split4(const float *m4, float *rot, float *trans, size_t count) {
    for (size_t i = 0; i < count; ++i)
        for (int r = 0; r < 3; ++r) {
            for (int c = 0; c < 3; ++c) rot[9 * i + 3 * r + c] = m4[16 * i + 4 * r + c];
            trans[3 * i + r] = m4[16 * i + 4 * r + 3];
        }
}

int bf_runtime_infer_cpu_ref(const bf_runtime *r, const bf_frame_input *f, size_t points,
                             size_t voxels, size_t sparse, bf_detections *detections,
                             void *workspace, size_t workspace_bytes, char *error, size_t cap) {
    size_t size[R_COUNT];
    if (!r || !f || !f->camera_images || !f->points || !f->camera_intrinsics_6x16 ||
        !f->camera_to_lidar_6x16 || !f->image_augmentation_6x16 || !f->lidar_augmentation_16 ||
        !f->lidar_to_image_6x16 || !detections || !workspace ||
        !plan(points, voxels, sparse, size) ||
        workspace_bytes < bf_runtime_workspace_bytes(points, voxels, sparse) ||
        f->point_count > points)
        return bf_oracle_fail(error, cap, "invalid runtime frame, capacity, or workspace");
    void *at[R_COUNT];
    unsigned char *base = (unsigned char *)workspace;
    for (int i = 0; i < R_COUNT; ++i) {
        at[i] = base;
        base += (size[i] + 63) & ~(size_t)63;
    }
    float *lidar_bev = at[R_LIDAR_BEV], *image_bev = at[R_IMAGE_BEV];
    const size_t plane = (size_t)BEV * BEV;

    /* LiDAR branch. */
    const bf_voxel_config vc = {{-54.0f, -54.0f, -5.0f}, {54.0f, 54.0f, 3.0f},
                                {0.075f, 0.075f, 0.2f}, 5, 10, voxels};
    size_t voxel_count = 0;
    bf_voxel_stats stats;
    if (!bf_voxelize_f32_workspace_ref(f->points, f->point_count, 5, 0, &vc, at[R_VOXELS],
                                       at[R_COORDS], at[R_COUNTS], &voxel_count, &stats,
                                       at[R_VOXEL_WS], size[R_VOXEL_WS]) ||
        !voxel_count)
        return bf_oracle_fail(error, cap, "runtime voxelization produced no voxels");
    bf_mean_vfe_f32_ref(at[R_VOXELS], at[R_COUNTS], at[R_VFE], voxel_count, 10, 5);
    if (!bf_lidar_backbone_forward_ref(r->lidar, at[R_COORDS], at[R_VFE], voxel_count, 1, 41,
                                       1440, 1440, sparse, lidar_bev, at[R_LIDAR_WS],
                                       size[R_LIDAR_WS], error, cap))
        return 0;

    /* Camera branch. */
    float *pts6 = at[R_POINTS6];
    for (size_t p = 0; p < f->point_count; ++p) {
        pts6[6 * p] = 0.0f;
        memcpy(pts6 + 6 * p + 1, f->points + 5 * p, 5 * sizeof(float));
    }
    if (!bf_depth_rasterize_f32_ref(pts6, f->point_count, 6, f->lidar_augmentation_16,
                                    f->lidar_to_image_6x16, f->image_augmentation_6x16,
                                    at[R_DEPTH], 1, CAMS, IMG_H, IMG_W))
        return bf_oracle_fail(error, cap, "runtime depth rasterization failed");
    if (!bf_swin_backbone_forward_ref(r->swin, f->camera_images, CAMS, IMG_H, IMG_W, at[R_S0],
                                      at[R_S1], at[R_S2], at[R_SWIN_WS], size[R_SWIN_WS], error,
                                      cap) ||
        !bf_image_fpn_forward_ref(r->fpn, at[R_S0], at[R_S1], at[R_S2], CAMS, FEAT_H, FEAT_W,
                                  at[R_F0], at[R_F1], at[R_FPN_WS], size[R_FPN_WS], error, cap) ||
        !bf_depth_head_forward_ref(r->depth, at[R_F0], at[R_DEPTH], CAMS, FEAT_H, FEAT_W,
                                   at[R_LOGITS], at[R_CONTEXT], at[R_HEAD_WS], size[R_HEAD_WS],
                                   error, cap))
        return 0;
    float rot[CAMS * 9], trans[CAMS * 3], intr[CAMS * 9], unused[CAMS * 3];
    float post_rot[CAMS * 9], post_trans[CAMS * 3], extra_rot[9], extra_trans[3];
    split4(f->camera_to_lidar_6x16, rot, trans, CAMS);
    split4(f->camera_intrinsics_6x16, intr, unused, CAMS);
    split4(f->image_augmentation_6x16, post_rot, post_trans, CAMS);
    split4(f->lidar_augmentation_16, extra_rot, extra_trans, 1);
    const bf_lss_desc lss = {1, CAMS, BINS, FEAT_H, FEAT_W, CTX, {-54.0f, -54.0f, -10.0f},
                             {0.3f, 0.3f, 20.0f}, {FULL, FULL, 1}};
    if (!bf_lss_geometry_f32_ref(r->frustum, rot, trans, intr, post_rot, post_trans, extra_rot,
                                 extra_trans, at[R_GEOMETRY], 1, CAMS, BINS, FEAT_H, FEAT_W) ||
        !bf_lss_lift_pool_f32_ref(at[R_LOGITS], at[R_CONTEXT], at[R_GEOMETRY], at[R_FULL_BEV],
                                  &lss))
        return bf_oracle_fail(error, cap, "runtime lift-splat failed");
    if (!bf_lss_downsample_forward_ref(r->down, at[R_FULL_BEV], 1, FULL, FULL, image_bev,
                                       at[R_DOWN_WS], size[R_DOWN_WS], error, cap))
        return 0;

    /* Fusion, BEV stage, decoder, decode. */
    float *fusion = at[R_FUSION], *raw = at[R_RAW];
    memcpy(fusion, image_bev, CTX * plane * sizeof(float));
    memcpy(fusion + CTX * plane, lidar_bev, 256 * plane * sizeof(float));
    if (!bf_bev_stage_forward_ref(r->bev, fusion, 1, BEV, BEV, at[R_SPATIAL], at[R_SHARED],
                                  at[R_HEATMAP], at[R_BEV_WS], size[R_BEV_WS], error, cap))
        return 0;
    int64_t *labels = at[R_LABELS];
    bf_transfusion_raw_outputs out = {raw, raw + 2 * PROPOSALS, raw + 3 * PROPOSALS,
                                      raw + 6 * PROPOSALS, raw + 8 * PROPOSALS,
                                      raw + 10 * PROPOSALS, raw + 20 * PROPOSALS, labels,
                                      labels + PROPOSALS};
    if (!bf_transfusion_decoder_forward_ref(r->decoder, at[R_SHARED], at[R_HEATMAP], 1, BEV, BEV,
                                            PROPOSALS, &out, at[R_DEC_WS], size[R_DEC_WS], error,
                                            cap))
        return 0;
    const float voxel_xy[2] = {0.075f, 0.075f}, minimum_xy[2] = {-54.0f, -54.0f};
    const float range[6] = {-61.2f, -61.2f, -10.0f, 61.2f, 61.2f, 10.0f};
    if (!bf_transfusion_decode_raw_f32_ref(out.heatmap_logits_b10p, out.query_heatmap_scores_b10p,
                                           out.query_labels_bp, out.center_b2p, out.height_b1p,
                                           out.dimension_log_b3p, out.rotation_sincos_b2p,
                                           out.velocity_b2p, at[R_BOXES], at[R_SCORES],
                                           at[R_OUT_LABELS], 1, 10, PROPOSALS, 8.0f, voxel_xy,
                                           minimum_xy) ||
        !bf_transfusion_filter_detections(at[R_BOXES], at[R_SCORES], at[R_OUT_LABELS], 1,
                                          PROPOSALS, 0.0f, range, detections))
        return bf_oracle_fail(error, cap, "runtime canonical decode failed");
    return 1;
}
