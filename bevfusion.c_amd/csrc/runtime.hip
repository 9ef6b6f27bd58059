// Full-frame BEVFusion runtime (drop-in for reference src/cuda_runtime.cu:53-98).
//
// Three HIP graphs per runtime, captured on the first frame.  The frame's
// host arrays are copied into fixed device buffers (the point count as a
// device word) and the graphs replay the chain:
//   main   points + matrices upload -> fork
//   side   (after fork) LiDAR graph: voxeliser -> SECOND encoder -> join
//   main   images + calibration upload -> camera graph: depth raster ->
//          Swin-T -> FPN + depth head -> lift-splat -> downsample
//   main   (after join) tail graph: BEV stage -> TransFusion -> decode
//          (threshold 0) -> detections copied back
// The two branches are independent until the BEV stage and neither fills the
// chip (the deep sparse convs run one wave per SIMD, the camera GEMMs are
// small), so they run concurrently, and the LiDAR branch starts while the
// images are still being uploaded.  Events order the graph launches; both
// streams keep the default priority.  The two modality BEVs are written
// straight into their channel ranges of the fused [336,180,180] input (image
// channels 0-79, LiDAR 80-335), so the reference's concat copy disappears.
// Kernels that depend on the point count read it from device memory and are
// sized by the point capacity, so the graph is independent of the frame.
// The LSS cell lists depend on the calibration only; they are rebuilt on the
// stream before the replay when the calibration differs from the previous
// frame's (as cuda_runtime.cu:87-88 does).
#include "bf_cuda.h"
#include "bf_cuda_bev.h"
#include "bf_cuda_camera.h"
#include "bf_cuda_depth_raster.h"
#include "bf_cuda_lidar.h"
#include "bf_cuda_runtime.h"
#include "bf_cuda_swin.h"
#include "bf_cuda_transfusion.h"
#include "bf_cuda_voxel.h"
#include "bf_model.h"
#include "bfhip_debug.h"
#include "hip_common.h"
#include "internal.h"

#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace bfhip;

namespace {

constexpr int kCams = 6, kImgH = 256, kImgW = 704, kFeatH = 32, kFeatW = 88, kBins = 118;
constexpr int kCtx = 80, kFull = 360, kBev = 180, kProposals = 200;
constexpr size_t kPlane = (size_t)kBev * kBev;
constexpr int kCalib = 54 + 18 + 54 + 54 + 18 + 9 + 3;  // rotations/translations, as uploaded

// Rotation rows and translation column of row-major 4x4 matrices.
void extract(const float *m4, float *rot, float *trans, int count) {
    for (int i = 0; i < count; ++i) {
        const float *m = m4 + 16 * i;
        for (int r = 0; r < 3; ++r) {
            for (int c = 0; c < 3; ++c) rot[9 * i + 3 * r + c] = m[4 * r + c];
            trans[3 * i + r] = m[4 * r + 3];
        }
    }
}

// The reference's singularity test (cuda_runtime.cu:63): |det| in double
// above the least normal float.
bool invertible(const float *m) {
    const double d = (double)m[0] * (m[4] * m[8] - m[5] * m[7]) +
                     (double)m[1] * (m[5] * m[6] - m[3] * m[8]) +
                     (double)m[2] * (m[3] * m[7] - m[4] * m[6]);
    return std::isfinite(d) && std::fabs(d) > FLT_MIN;
}

// sum |x| (double partials) and max |x| per workgroup.
__global__ __launch_bounds__(256) void stats_partial_kernel(const float *__restrict__ x, size_t n,
                                                            double *__restrict__ sums,
                                                            float *__restrict__ maxima) {
    __shared__ double ss[256];
    __shared__ float mm[256];
    double s = 0.0;
    float m = 0.0f;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float a = fabsf(x[i]);
        s += a;
        m = fmaxf(m, a);
    }
    ss[threadIdx.x] = s;
    mm[threadIdx.x] = m;
    __syncthreads();
    for (unsigned o = 128; o; o >>= 1) {
        if (threadIdx.x < o) {
            ss[threadIdx.x] += ss[threadIdx.x + o];
            mm[threadIdx.x] = fmaxf(mm[threadIdx.x], mm[threadIdx.x + o]);
        }
        __syncthreads();
    }
    if (!threadIdx.x) {
        sums[blockIdx.x] = ss[0];
        maxima[blockIdx.x] = mm[0];
    }
}

__global__ void stats_final_kernel(const double *__restrict__ sums,
                                   const float *__restrict__ maxima, int parts,
                                   float *__restrict__ out) {
    if (threadIdx.x || blockIdx.x) return;
    double s = 0.0;
    float m = 0.0f;
    for (int i = 0; i < parts; ++i) {
        s += sums[i];
        m = fmaxf(m, maxima[i]);
    }
    out[0] = (float)s;
    out[1] = m;
}

// splitmix64 finaliser.
__device__ __forceinline__ unsigned long long mix64(unsigned long long v) {
    v ^= v >> 30;
    v *= 0xbf58476d1ce4e5b9ull;
    v ^= v >> 27;
    v *= 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

__global__ __launch_bounds__(256) void hash_partial_kernel(const float *__restrict__ x, size_t n,
                                                           unsigned long long *__restrict__ parts) {
    __shared__ unsigned long long h[256];
    unsigned long long v = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        v ^= mix64(((unsigned long long)i << 32) ^ __float_as_uint(x[i]));
    h[threadIdx.x] = v;
    __syncthreads();
    for (unsigned o = 128; o; o >>= 1) {
        if (threadIdx.x < o) h[threadIdx.x] ^= h[threadIdx.x + o];
        __syncthreads();
    }
    if (!threadIdx.x) parts[blockIdx.x] = h[0];
}

__global__ void hash_final_kernel(const unsigned long long *__restrict__ parts, int count,
                                  unsigned long long *__restrict__ out) {
    if (threadIdx.x || blockIdx.x) return;
    unsigned long long v = 0;
    for (int i = 0; i < count; ++i) v ^= parts[i];
    *out = v;
}

}  // namespace

struct bf_cuda_runtime {
    size_t point_capacity, voxel_capacity, sparse_capacity, resident_bytes;
    hipStream_t stream, side;
    hipEvent_t fork, join;
    bf_cuda_depth_raster *raster;
    bf_cuda_voxelizer *voxelizer;
    bf_cuda_lidar_backbone *lidar;
    bf_cuda_swin *swin;
    bf_cuda_camera_neck *camera;
    bf_cuda_lss_plan *lss;
    bf_cuda_bev_stage *bev;
    bf_cuda_transfusion *decoder;
    unsigned char *arena;
    // Frame inputs.
    float *images, *points, *lidar_aug, *lidar_to_image, *image_aug, *calib, *frustum;
    unsigned *point_count;
    // Graph intermediates.
    float *dense_depth, *swin0, *swin1, *swin2, *depth_logits, *context, *full_image_bev;
    float *fusion, *image_bev, *lidar_bev, *spatial, *shared, *heatmap;
    bf_coord4 *voxel_coords;
    float *voxel_features;
    unsigned *voxel_count;
    bf_transfusion_raw_outputs raw;
    const bf_detections *detections;
    hipGraphExec_t graph[3];  // LiDAR, camera, tail
    bool use_graph, calib_valid;
    bool inject_failure;  // bfhip_debug_runtime_fail_next armed
    float calib_key[kCalib];
};

namespace {

// The launches of one frame in three parts: the LiDAR branch (on r->side),
// the camera branch and the tail (on r->stream).
int enqueue_lidar(bf_cuda_runtime *r, char *error, size_t cap) {
    void *l = r->side;
    return voxelize_count_device(r->voxelizer, r->points, r->point_count, r->point_capacity,
                                 r->voxel_coords, r->voxel_features, r->voxel_count, l, error,
                                 cap) &&
           bf_cuda_lidar_backbone_forward_count_device(r->lidar, r->voxel_coords,
                                                       r->voxel_features, r->voxel_count,
                                                       r->lidar_bev, l, error, cap);
}

int enqueue_camera(bf_cuda_runtime *r, char *error, size_t cap) {
    void *s = r->stream;
    return depth_rasterize_count_device(r->raster, r->points, r->point_count, r->point_capacity,
                                        r->lidar_aug, r->lidar_to_image, r->image_aug,
                                        r->dense_depth, s, error, cap) &&
           bf_cuda_swin_forward(r->swin, r->images, r->swin0, r->swin1, r->swin2, s, error, cap) &&
           bf_cuda_camera_neck_forward(r->camera, r->swin0, r->swin1, r->swin2, r->dense_depth,
                                       r->depth_logits, r->context, s, error, cap) &&
           bf_cuda_lss_plan_forward_f32(r->lss, r->depth_logits, r->context, r->full_image_bev, s,
                                        error, cap) &&
           bf_cuda_camera_downsample_forward(r->camera, r->full_image_bev, r->image_bev, s, error,
                                             cap);
}

int enqueue_tail(bf_cuda_runtime *r, char *error, size_t cap) {
    void *s = r->stream;
    return bf_cuda_bev_stage_forward(r->bev, r->fusion, r->spatial, r->shared, r->heatmap, s,
                                     error, cap) &&
           bf_cuda_transfusion_forward(r->decoder, r->shared, r->heatmap, &r->raw, s, error,
                                       cap) &&
           transfusion_decode_launch(r->decoder, &r->raw, 0.0f, s, &r->detections, error, cap);
}

typedef int (*Part)(bf_cuda_runtime *, char *, size_t);

// Part k of the frame on `stream`: replayed from its graph (captured on first
// use), or launched eagerly when graphs are off.
int run_part(bf_cuda_runtime *r, int k, Part part, hipStream_t stream, char *error, size_t cap) {
    if (!r->use_graph) return part(r, error, cap);
    if (!r->graph[k]) {
        if (!hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), error, cap,
                    "begin runtime graph capture"))
            return 0;
        const int ok = part(r, error, cap);
        hipGraph_t g = nullptr;
        const hipError_t end = hipStreamEndCapture(stream, &g);
        if (!ok) {
            if (g) (void)hipGraphDestroy(g);
            return 0;
        }
        // The LiDAR stream is a blocking stream (it carries a CU mask): work
        // that another host thread puts on the legacy null stream while the
        // first frame captures it synchronises with it implicitly, which
        // invalidates the capture.
        if (!hip_ok(end, error, cap,
                    k == 0 ? "end runtime graph capture (LiDAR stream; was the legacy null stream "
                             "used by another thread during the first frame?)"
                           : "end runtime graph capture"))
            return 0;
        const hipError_t inst = hipGraphInstantiate(&r->graph[k], g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (!hip_ok(inst, error, cap, "instantiate runtime graph")) {
            r->graph[k] = nullptr;
            return 0;
        }
    }
    return hip_ok(hipGraphLaunch(r->graph[k], stream), error, cap, "launch HIP runtime graph");
}

}  // namespace

extern "C" void bf_cuda_runtime_destroy(bf_cuda_runtime *r) {
    if (!r) return;
    if (r->stream) (void)hipStreamSynchronize(r->stream);
    if (r->side) (void)hipStreamSynchronize(r->side);
    for (hipGraphExec_t g : r->graph)
        if (g) (void)hipGraphExecDestroy(g);
    bf_cuda_transfusion_destroy(r->decoder);
    bf_cuda_bev_stage_destroy(r->bev);
    bf_cuda_lss_plan_destroy(r->lss);
    bf_cuda_camera_neck_destroy(r->camera);
    bf_cuda_swin_destroy(r->swin);
    bf_cuda_lidar_backbone_destroy(r->lidar);
    bf_cuda_voxelizer_destroy(r->voxelizer);
    bf_cuda_depth_raster_destroy(r->raster);
    if (r->arena) (void)hipFree(r->arena);
    if (r->fork) (void)hipEventDestroy(r->fork);
    if (r->join) (void)hipEventDestroy(r->join);
    if (r->side) (void)hipStreamDestroy(r->side);
    if (r->stream) (void)hipStreamDestroy(r->stream);
    std::free(r);
}

extern "C" size_t bf_cuda_runtime_resident_bytes(const bf_cuda_runtime *r) {
    return r ? r->resident_bytes : 0;
}

extern "C" int bf_cuda_runtime_create(const char *model_path, size_t point_capacity,
                                      size_t voxel_capacity, size_t sparse_capacity,
                                      bf_cuda_runtime **out, char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!model_path || !out || !point_capacity || !voxel_capacity || !sparse_capacity ||
        voxel_capacity > sparse_capacity || point_capacity > (1u << 30))
        return fail(error, cap, "invalid HIP runtime contract");
    bf_model *model = nullptr;
    if (!bf_model_open(model_path, &model, error, cap)) return 0;
    bf_cuda_runtime *r = (bf_cuda_runtime *)std::calloc(1, sizeof(*r));
    if (!r) {
        bf_model_close(model);
        return fail(error, cap, "HIP runtime allocation failed");
    }
    r->point_capacity = point_capacity;
    r->voxel_capacity = voxel_capacity;
    r->sparse_capacity = sparse_capacity;
    const char *env = std::getenv("BFHIP_RUNTIME_GRAPH");
    r->use_graph = !(env && env[0] == '0');
    // Contracts of cuda_runtime.cu:53-54.
    const bf_voxel_config vcfg = {{-54.0f, -54.0f, -5.0f}, {54.0f, 54.0f, 3.0f},
                                  {0.075f, 0.075f, 0.2f}, 5, 10, voxel_capacity};
    const bf_lss_desc lss = {1, kCams, kBins, kFeatH, kFeatW, kCtx, {-54.0f, -54.0f, -10.0f},
                             {0.3f, 0.3f, 20.0f}, {kFull, kFull, 1}};
    const bf_tensor *fr = bf_model_find(model, "vtransform.frustum");
    // The LiDAR stream gets a hardware queue of its own: HIP spreads ordinary
    // streams over a few shared queues (GPU_MAX_HW_QUEUES), and when both
    // runtime streams land on one queue the branches run back to back (4.3
    // instead of 3.5 ms per frame on MI355X once a caller holds three other
    // streams).  A stream with a CU mask is never shared; the mask names
    // every CU.  Such a stream is a blocking one: work on the null stream
    // waits for it.
    int device = 0, cus = 0;
    int ok = hip_ok(hipGetDevice(&device), error, cap, "query HIP device") &&
             hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                    error, cap, "query HIP CU count");
    std::vector<uint32_t> every_cu(ok ? (size_t)(cus + 31) / 32 : 0, 0u);
    for (int c = 0; c < cus; ++c) every_cu[c / 32] |= 1u << (c % 32);
    ok = ok && cus > 0 &&
             hip_ok(hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking), error, cap,
                    "create HIP runtime stream") &&
             hip_ok(hipExtStreamCreateWithCUMask(&r->side, (uint32_t)every_cu.size(),
                                                 every_cu.data()),
                    error, cap, "create HIP runtime LiDAR stream") &&
             hip_ok(hipEventCreateWithFlags(&r->fork, hipEventDisableTiming), error, cap,
                    "create HIP runtime events") &&
             hip_ok(hipEventCreateWithFlags(&r->join, hipEventDisableTiming), error, cap,
                    "create HIP runtime events") &&
             bf_cuda_depth_raster_create(point_capacity, kCams, kImgH, kImgW, &r->raster, error,
                                         cap) &&
             bf_cuda_voxelizer_create(&vcfg, point_capacity, &r->voxelizer, error, cap) &&
             bf_cuda_lidar_backbone_create(model, 1, 41, 1440, 1440, sparse_capacity, &r->lidar,
                                           error, cap) &&
             bf_cuda_swin_create(model, kCams, kImgH, kImgW, &r->swin, error, cap) &&
             bf_cuda_camera_neck_create(model, kCams, kFeatH, kFeatW, kFull, kFull, &r->camera,
                                        error, cap) &&
             bf_cuda_lss_plan_create(&lss, &r->lss, error, cap) &&
             bf_cuda_bev_stage_create(model, kBev, kBev, &r->bev, error, cap) &&
             bf_cuda_transfusion_create(model, kBev, kBev, kProposals, &r->decoder, error, cap);
    if (ok && (!fr || fr->dtype != BF_DTYPE_F32 || fr->rank != 4 || fr->dims[0] != kBins ||
               fr->dims[1] != kFeatH || fr->dims[2] != kFeatW || fr->dims[3] != 3))
        ok = fail(error, cap, "vtransform.frustum contract mismatch");
    if (ok) {
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t at = off;
            off += (bytes + 255) & ~size_t(255);
            return at;
        };
        const size_t F = sizeof(float);
        const size_t o_images = take((size_t)kCams * 3 * kImgH * kImgW * F);
        const size_t o_points = take(point_capacity * 5 * F);
        const size_t o_aug = take(16 * F), o_l2i = take(96 * F), o_post = take(96 * F);
        const size_t o_calib = take(kCalib * F), o_frustum = take((size_t)fr->nbytes);
        const size_t o_count = take(sizeof(unsigned));
        const size_t o_depth = take((size_t)kCams * kImgH * kImgW * F);
        const size_t o_s0 = take((size_t)kCams * 192 * 32 * 88 * F);
        const size_t o_s1 = take((size_t)kCams * 384 * 16 * 44 * F);
        const size_t o_s2 = take((size_t)kCams * 768 * 8 * 22 * F);
        const size_t o_logits = take((size_t)kCams * kBins * kFeatH * kFeatW * F);
        const size_t o_ctx = take((size_t)kCams * kCtx * kFeatH * kFeatW * F);
        const size_t o_full = take((size_t)kCtx * kFull * kFull * F);
        const size_t o_fusion = take(336 * kPlane * F);
        const size_t o_spatial = take(512 * kPlane * F), o_shared = take(128 * kPlane * F);
        const size_t o_heat = take(10 * kPlane * F);
        const size_t o_vc = take(voxel_capacity * sizeof(bf_coord4));
        const size_t o_vf = take(voxel_capacity * 5 * F), o_vn = take(sizeof(unsigned));
        const size_t o_raw = take((size_t)kProposals * (2 + 1 + 3 + 2 + 2 + 10 + 10) * F);
        const size_t o_lab = take((size_t)kProposals * 2 * sizeof(int64_t));
        ok = hip_ok(hipMalloc((void **)&r->arena, off), error, cap, "allocate HIP runtime buffers");
        if (ok) {
            unsigned char *a = r->arena;
            r->images = (float *)(a + o_images);
            r->points = (float *)(a + o_points);
            r->lidar_aug = (float *)(a + o_aug);
            r->lidar_to_image = (float *)(a + o_l2i);
            r->image_aug = (float *)(a + o_post);
            r->calib = (float *)(a + o_calib);
            r->frustum = (float *)(a + o_frustum);
            r->point_count = (unsigned *)(a + o_count);
            r->dense_depth = (float *)(a + o_depth);
            r->swin0 = (float *)(a + o_s0);
            r->swin1 = (float *)(a + o_s1);
            r->swin2 = (float *)(a + o_s2);
            r->depth_logits = (float *)(a + o_logits);
            r->context = (float *)(a + o_ctx);
            r->full_image_bev = (float *)(a + o_full);
            r->fusion = (float *)(a + o_fusion);
            r->image_bev = r->fusion;
            r->lidar_bev = r->fusion + (size_t)kCtx * kPlane;
            r->spatial = (float *)(a + o_spatial);
            r->shared = (float *)(a + o_shared);
            r->heatmap = (float *)(a + o_heat);
            r->voxel_coords = (bf_coord4 *)(a + o_vc);
            r->voxel_features = (float *)(a + o_vf);
            r->voxel_count = (unsigned *)(a + o_vn);
            float *o = (float *)(a + o_raw);
            r->raw.center_b2p = o;
            r->raw.height_b1p = o + 2 * kProposals;
            r->raw.dimension_log_b3p = o + 3 * kProposals;
            r->raw.rotation_sincos_b2p = o + 6 * kProposals;
            r->raw.velocity_b2p = o + 8 * kProposals;
            r->raw.heatmap_logits_b10p = o + 10 * kProposals;
            r->raw.query_heatmap_scores_b10p = o + 20 * kProposals;
            r->raw.query_labels_bp = (int64_t *)(a + o_lab);
            r->raw.query_indices_bp = r->raw.query_labels_bp + kProposals;
            r->resident_bytes = off;
            ok = hip_ok(hipMemcpy(r->frustum, fr->data, (size_t)fr->nbytes, hipMemcpyHostToDevice),
                        error, cap, "upload HIP frustum");
        }
    }
    bf_model_close(model);
    if (!ok) {
        bf_cuda_runtime_destroy(r);
        return 0;
    }
    r->resident_bytes += bf_cuda_depth_raster_resident_bytes(r->raster) +
                         bf_cuda_voxelizer_resident_bytes(r->voxelizer) +
                         bf_cuda_lidar_backbone_resident_bytes(r->lidar) +
                         bf_cuda_swin_resident_bytes(r->swin) +
                         bf_cuda_camera_neck_resident_bytes(r->camera) +
                         bf_cuda_lss_plan_resident_bytes(r->lss) +
                         bf_cuda_bev_stage_resident_bytes(r->bev) +
                         bf_cuda_transfusion_resident_bytes(r->decoder);
    *out = r;
    return 1;
}

extern "C" int bf_cuda_runtime_infer(bf_cuda_runtime *r, const bf_frame_input *f,
                                     bf_detections *detections, char *error, size_t cap) {
    if (!r || !f || !detections || !f->camera_images || !f->points ||
        !f->camera_intrinsics_6x16 || !f->camera_to_lidar_6x16 || !f->image_augmentation_6x16 ||
        !f->lidar_augmentation_16 || !f->lidar_to_image_6x16 || !f->point_count ||
        f->point_count > r->point_capacity)
        return fail(error, cap, "invalid HIP runtime frame");
    // Calibration as uploaded: camera rotation/translation, intrinsics,
    // post rotation/translation, extra rotation/translation.
    float key[kCalib], unused[18];
    float *rot = key, *trans = rot + 54, *intr = trans + 18, *post_rot = intr + 54;
    float *post_trans = post_rot + 54, *extra_rot = post_trans + 18, *extra_trans = extra_rot + 9;
    extract(f->camera_to_lidar_6x16, rot, trans, kCams);
    extract(f->camera_intrinsics_6x16, intr, unused, kCams);
    extract(f->image_augmentation_6x16, post_rot, post_trans, kCams);
    extract(f->lidar_augmentation_16, extra_rot, extra_trans, 1);
    if (!invertible(extra_rot)) return fail(error, cap, "singular HIP lidar augmentation");
    for (int c = 0; c < kCams; ++c)
        if (!invertible(intr + 9 * c) || !invertible(post_rot + 9 * c))
            return fail(error, cap, "singular HIP camera calibration %d", c);
    const hipStream_t s = r->stream;
    const unsigned count = (unsigned)f->point_count;
    const size_t F = sizeof(float);
    // Once anything is enqueued, a failure drains both streams before
    // returning: copies still read `count` and `key` from this frame, and the
    // next call rewrites the buffers the LiDAR stream may still be reading.
    auto drain = [&]() {
        (void)hipStreamSynchronize(r->side);
        (void)hipStreamSynchronize(s);
        return 0;
    };
    // Points and matrices first: the LiDAR branch needs nothing else.
    if (!hip_ok(hipMemcpyAsync(r->points, f->points, f->point_count * 5 * F,
                               hipMemcpyHostToDevice, s), error, cap, "upload HIP points") ||
        !hip_ok(hipMemcpyAsync(r->point_count, &count, sizeof(count), hipMemcpyHostToDevice, s),
                error, cap, "upload HIP point count") ||
        !hip_ok(hipMemcpyAsync(r->lidar_aug, f->lidar_augmentation_16, 16 * F,
                               hipMemcpyHostToDevice, s), error, cap, "upload HIP lidar aug") ||
        !hip_ok(hipMemcpyAsync(r->lidar_to_image, f->lidar_to_image_6x16, 96 * F,
                               hipMemcpyHostToDevice, s), error, cap, "upload HIP lidar-to-image") ||
        !hip_ok(hipMemcpyAsync(r->image_aug, f->image_augmentation_6x16, 96 * F,
                               hipMemcpyHostToDevice, s), error, cap, "upload HIP image aug") ||
        !hip_ok(hipEventRecord(r->fork, s), error, cap, "fork LiDAR branch") ||
        !hip_ok(hipStreamWaitEvent(r->side, r->fork, 0), error, cap, "fork LiDAR branch") ||
        !run_part(r, 0, enqueue_lidar, r->side, error, cap) ||
        !hip_ok(hipEventRecord(r->join, r->side), error, cap, "join LiDAR branch") ||
        !hip_ok(hipMemcpyAsync(r->images, f->camera_images, (size_t)kCams * 3 * kImgH * kImgW * F,
                               hipMemcpyHostToDevice, s), error, cap, "upload HIP images") ||
        !hip_ok(hipMemcpyAsync(r->calib, key, sizeof(key), hipMemcpyHostToDevice, s), error, cap,
                "upload HIP calibration"))
        return drain();
    if (!r->calib_valid || std::memcmp(key, r->calib_key, sizeof(key)) != 0) {
        // The cell lists are rebuilt in place: until the rebuild is queued
        // they match no calibration, so a failure here leaves the cache
        // invalid and the next frame rebuilds them again.
        r->calib_valid = false;
        if (!bf_cuda_lss_plan_prepare_calibration_f32(r->lss, r->frustum, r->calib, r->calib + 54,
                                                      r->calib + 72, r->calib + 126, r->calib + 180,
                                                      r->calib + 198, r->calib + 207, s, error, cap))
            return drain();
        // Queued: the lists now hold this calibration whatever fails later
        // (every failure path drains the stream, which completes the rebuild).
        std::memcpy(r->calib_key, key, sizeof(key));
        r->calib_valid = true;
    }
    if (r->inject_failure) {  // debug hook: fail after the rebuild is queued
        r->inject_failure = false;
        fail(error, cap, "injected HIP runtime failure after the calibration upload");
        return drain();
    }
    if (!run_part(r, 1, enqueue_camera, s, error, cap) ||
        !hip_ok(hipStreamWaitEvent(s, r->join, 0), error, cap, "join LiDAR branch") ||
        !run_part(r, 2, enqueue_tail, s, error, cap))
        return drain();
    if (!hip_ok(hipMemcpyAsync(detections, r->detections, sizeof(*detections),
                               hipMemcpyDeviceToHost, s), error, cap, "copy HIP detections") ||
        !hip_ok(hipStreamSynchronize(s), error, cap, "synchronize HIP runtime"))
        return drain();
    if (detections->count < 0 || detections->count > BF_MAX_PROPOSALS)
        return fail(error, cap, "HIP runtime detection count out of range");
    return 1;
}

extern "C" int bf_cuda_runtime_debug_bev_stats(const bf_cuda_runtime *r, float stats[4],
                                               char *error, size_t cap) {
    if (!r || !stats) return fail(error, cap, "invalid HIP BEV stats contract");
    constexpr int kParts = 1024;
    void *tmp = nullptr;
    if (!hip_ok(hipMalloc(&tmp, kParts * (sizeof(double) + sizeof(float)) + 4 * sizeof(float)),
                error, cap, "allocate HIP BEV stats"))
        return 0;
    double *sums = (double *)tmp;
    float *maxima = (float *)(sums + kParts), *dev = maxima + kParts;
    const hipStream_t s = r->stream;
    const float *src[2] = {r->image_bev, r->lidar_bev};
    const size_t n[2] = {(size_t)kCtx * kPlane, 256 * kPlane};
    for (int i = 0; i < 2; ++i) {
        stats_partial_kernel<<<kParts, 256, 0, s>>>(src[i], n[i], sums, maxima);
        stats_final_kernel<<<1, 64, 0, s>>>(sums, maxima, kParts, dev + 2 * i);
    }
    const int ok = launch_ok(error, cap, "launch HIP BEV stats") &&
                   hip_ok(hipMemcpyAsync(stats, dev, 4 * sizeof(float), hipMemcpyDeviceToHost, s),
                          error, cap, "copy HIP BEV stats") &&
                   hip_ok(hipStreamSynchronize(s), error, cap, "synchronize HIP BEV stats");
    (void)hipFree(tmp);
    return ok;
}

extern "C" int bf_cuda_runtime_debug_hashes(const bf_cuda_runtime *r, unsigned long long hashes[11],
                                            char *error, size_t cap) {
    if (!r || !hashes) return fail(error, cap, "invalid HIP hash contract");
    constexpr int kParts = 1024;
    unsigned long long *tmp = nullptr;
    if (!hip_ok(hipMalloc((void **)&tmp, (kParts + 11) * sizeof(*tmp)), error, cap,
                "allocate HIP hashes"))
        return 0;
    const float *data[11] = {r->dense_depth, r->swin0,   r->swin1,          r->swin2,
                             r->depth_logits, r->context, r->full_image_bev, r->image_bev,
                             r->lidar_bev,    r->shared,  r->heatmap};
    const size_t n[11] = {(size_t)kCams * kImgH * kImgW,   (size_t)kCams * 192 * 32 * 88,
                          (size_t)kCams * 384 * 16 * 44,   (size_t)kCams * 768 * 8 * 22,
                          (size_t)kCams * kBins * 32 * 88, (size_t)kCams * kCtx * 32 * 88,
                          (size_t)kCtx * kFull * kFull,    (size_t)kCtx * kPlane,
                          256 * kPlane,                    128 * kPlane,
                          10 * kPlane};
    const hipStream_t s = r->stream;
    for (int i = 0; i < 11; ++i) {
        hash_partial_kernel<<<kParts, 256, 0, s>>>(data[i], n[i], tmp);
        hash_final_kernel<<<1, 64, 0, s>>>(tmp, kParts, tmp + kParts + i);
    }
    const int ok = launch_ok(error, cap, "launch HIP tensor hashes") &&
                   hip_ok(hipMemcpyAsync(hashes, tmp + kParts, 11 * sizeof(*hashes),
                                         hipMemcpyDeviceToHost, s),
                          error, cap, "copy HIP tensor hashes") &&
                   hip_ok(hipStreamSynchronize(s), error, cap, "synchronize HIP tensor hashes");
    (void)hipFree(tmp);
    return ok;
}

extern "C" int bfhip_debug_runtime_fail_next(bf_cuda_runtime *r, char *error, size_t cap) {
    if (!r) return fail(error, cap, "invalid HIP runtime failure hook");
    r->inject_failure = true;
    return 1;
}
