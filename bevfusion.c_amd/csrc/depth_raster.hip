// LiDAR-to-image depth raster (drop-in for reference src/cuda_depth_raster.cu).
//
// One thread per (point, camera) projects the point exactly as the reference
// CPU raster does (depth_raster.c:49-105: un-augment with the inverse lidar
// rotation, project, clamp the depth, divide, augment), with products and
// sums kept unfused in the CPU's order, so pixel choices and depths are
// bit-identical to it.  "Later points win" becomes an integer atomic max of
// (point index + 1) per pixel, which is order-independent; a second pass
// reads the winner's depth and clears the owner word for the next call.
#include "bf_cuda_depth_raster.h"
#include "hip_common.h"
#include "internal.h"

#include <cfloat>
#include <climits>
#include <cstdint>
#include <cstdlib>

using namespace bfhip;

namespace {

// Cofactor inverse of the lidar augmentation's rotation (depth_raster.c:14-35).
__global__ void inverse_kernel(const float *__restrict__ m, float *__restrict__ inv,
                               int *__restrict__ valid) {
#pragma clang fp contract(off)
    if (threadIdx.x || blockIdx.x) return;
    const float a00 = m[0], a01 = m[1], a02 = m[2];
    const float a10 = m[4], a11 = m[5], a12 = m[6];
    const float a20 = m[8], a21 = m[9], a22 = m[10];
    const float c00 = a11 * a22 - a12 * a21, c01 = a02 * a21 - a01 * a22,
                c02 = a01 * a12 - a02 * a11;
    const float c10 = a12 * a20 - a10 * a22, c11 = a00 * a22 - a02 * a20,
                c12 = a02 * a10 - a00 * a12;
    const float c20 = a10 * a21 - a11 * a20, c21 = a01 * a20 - a00 * a21,
                c22 = a00 * a11 - a01 * a10;
    const float det = a00 * c00 + a01 * c10 + a02 * c20;
    if (!isfinite(det) || fabsf(det) <= FLT_MIN) {
        *valid = 0;
        return;
    }
    const float s = 1.0f / det;
    const float r[9] = {c00 * s, c01 * s, c02 * s, c10 * s, c11 * s, c12 * s,
                        c20 * s, c21 * s, c22 * s};
    for (int i = 0; i < 9; ++i) inv[i] = r[i];
    *valid = 1;
}

__global__ __launch_bounds__(256) void project_kernel(
    const float *__restrict__ points, const unsigned *__restrict__ count_device, unsigned count,
    int cameras, int height, int width,
    const float *__restrict__ aug, const float *__restrict__ inv, const int *__restrict__ valid,
    const float *__restrict__ l2i, const float *__restrict__ post, unsigned *__restrict__ owners,
    float *__restrict__ distances) {
#pragma clang fp contract(off)
    const size_t item = (size_t)blockIdx.x * 256 + threadIdx.x;
    const unsigned n = count_device ? min(*count_device, count) : count;
    if (item >= (size_t)n * cameras || !*valid) return;
    const unsigned p = (unsigned)(item / cameras);
    const int cam = (int)(item % cameras);
    const float *pt = points + (size_t)p * 5;
    const float c0 = pt[0] - aug[3], c1 = pt[1] - aug[7], c2 = pt[2] - aug[11];
    if (!isfinite(c0) || !isfinite(c1) || !isfinite(c2)) return;
    const float u0 = inv[0] * c0 + inv[1] * c1 + inv[2] * c2;
    const float u1 = inv[3] * c0 + inv[4] * c1 + inv[5] * c2;
    const float u2 = inv[6] * c0 + inv[7] * c1 + inv[8] * c2;
    const float *pr = l2i + cam * 16, *pa = post + cam * 16;
    float q0 = pr[0] * u0 + pr[1] * u1 + pr[2] * u2;
    float q1 = pr[4] * u0 + pr[5] * u1 + pr[6] * u2;
    float q2 = pr[8] * u0 + pr[9] * u1 + pr[10] * u2;
    q0 += pr[3];
    q1 += pr[7];
    q2 += pr[11];
    if (!isfinite(q0) || !isfinite(q1) || !isfinite(q2)) return;
    float dist = q2;
    if (dist < 1e-5f) dist = 1e-5f;
    if (dist > 1e5f) dist = 1e5f;
    const float n0 = q0 / dist, n1 = q1 / dist, n2 = dist;
    float ax = pa[0] * n0 + pa[1] * n1 + pa[2] * n2;
    float ay = pa[4] * n0 + pa[5] * n1 + pa[6] * n2;
    ax += pa[3];
    ay += pa[7];
    if (!isfinite(ax) || !isfinite(ay) || ax < 0.0f || ax >= (float)width || ay < 0.0f ||
        ay >= (float)height)
        return;
    const size_t pixel = ((size_t)cam * height + (size_t)ay) * width + (size_t)ax;
    distances[item] = dist;
    atomicMax(owners + pixel, p + 1u);
}

__global__ __launch_bounds__(256) void materialize_kernel(unsigned *__restrict__ owners,
                                                          const float *__restrict__ distances,
                                                          int cameras, size_t plane,
                                                          float *__restrict__ depth) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= plane * cameras) return;
    const unsigned owner = owners[i];
    const size_t cam = i / plane;
    depth[i] = owner ? distances[(size_t)(owner - 1) * cameras + cam] : 0.0f;
    owners[i] = 0u;  // ready for the next call
}

}  // namespace

struct bf_cuda_depth_raster {
    size_t max_points, cameras, height, width, resident_bytes;
    unsigned *owners;
    float *distances, *inverse;
    int *valid;
};

extern "C" void bf_cuda_depth_raster_destroy(bf_cuda_depth_raster *r) {
    if (!r) return;
    (void)hipFree(r->owners);
    (void)hipFree(r->distances);
    (void)hipFree(r->inverse);
    (void)hipFree(r->valid);
    std::free(r);
}

extern "C" size_t bf_cuda_depth_raster_resident_bytes(const bf_cuda_depth_raster *r) {
    return r ? r->resident_bytes : 0;
}

extern "C" int bf_cuda_depth_raster_create(size_t max_points, size_t cameras, size_t height,
                                           size_t width, bf_cuda_depth_raster **out, char *error,
                                           size_t cap) {
    if (out) *out = nullptr;
    if (!out || !max_points || max_points > UINT_MAX || !cameras || !height || !width ||
        cameras > SIZE_MAX / height || cameras * height > SIZE_MAX / width ||
        max_points > SIZE_MAX / cameras || cameras > INT_MAX || height > INT_MAX ||
        width > INT_MAX)
        return fail(error, cap, "invalid HIP depth raster contract");
    bf_cuda_depth_raster *r = (bf_cuda_depth_raster *)std::calloc(1, sizeof(*r));
    if (!r) return fail(error, cap, "HIP depth raster host allocation failed");
    r->max_points = max_points;
    r->cameras = cameras;
    r->height = height;
    r->width = width;
    const size_t owner_bytes = cameras * height * width * sizeof(unsigned);
    const size_t dist_bytes = max_points * cameras * sizeof(float);
    if (!hip_ok(hipMalloc((void **)&r->owners, owner_bytes), error, cap, "allocate depth owners") ||
        !hip_ok(hipMemset(r->owners, 0, owner_bytes), error, cap, "clear depth owners") ||
        !hip_ok(hipMalloc((void **)&r->distances, dist_bytes), error, cap,
                "allocate depth distances") ||
        !hip_ok(hipMalloc((void **)&r->inverse, 9 * sizeof(float)), error, cap,
                "allocate lidar inverse") ||
        !hip_ok(hipMalloc((void **)&r->valid, sizeof(int)), error, cap, "allocate inverse flag")) {
        bf_cuda_depth_raster_destroy(r);
        return 0;
    }
    r->resident_bytes = owner_bytes + dist_bytes + 9 * sizeof(float) + sizeof(int);
    *out = r;
    return 1;
}

namespace {

// point_count is the exact count, or with count_device the bound of *count_device.
int rasterize(bf_cuda_depth_raster *r, const float *points, const unsigned *count_device,
              size_t point_count, const float *lidar_aug, const float *lidar_to_image,
              const float *image_aug, float *depth, void *stream_value, char *error, size_t cap) {
    if (!r || (!points && point_count) || point_count > r->max_points || !lidar_aug ||
        !lidar_to_image || !image_aug || !depth)
        return fail(error, cap, "invalid HIP depth raster buffers");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    inverse_kernel<<<1, 1, 0, s>>>(lidar_aug, r->inverse, r->valid);
    const size_t items = point_count * r->cameras;
    if (items)
        project_kernel<<<(unsigned)((items + 255) / 256), 256, 0, s>>>(
            points, count_device, (unsigned)point_count, (int)r->cameras, (int)r->height,
            (int)r->width, lidar_aug, r->inverse, r->valid, lidar_to_image, image_aug, r->owners,
            r->distances);
    const size_t plane = r->height * r->width, pixels = plane * r->cameras;
    materialize_kernel<<<(unsigned)((pixels + 255) / 256), 256, 0, s>>>(
        r->owners, r->distances, (int)r->cameras, plane, depth);
    return launch_ok(error, cap, "HIP depth raster launch");
}

}  // namespace

extern "C" int bf_cuda_depth_rasterize_f32(bf_cuda_depth_raster *r, const float *points,
                                           size_t point_count, const float *lidar_aug,
                                           const float *lidar_to_image, const float *image_aug,
                                           float *depth, void *stream, char *error, size_t cap) {
    return rasterize(r, points, nullptr, point_count, lidar_aug, lidar_to_image, image_aug, depth,
                     stream, error, cap);
}

int bfhip::depth_rasterize_count_device(bf_cuda_depth_raster *r, const float *points,
                                        const unsigned *count_device, size_t bound,
                                        const float *lidar_aug, const float *lidar_to_image,
                                        const float *image_aug, float *depth, void *stream,
                                        char *error, size_t cap) {
    if (!count_device || !points) return fail(error, cap, "invalid HIP depth raster buffers");
    return rasterize(r, points, count_device, bound, lidar_aug, lidar_to_image, image_aug, depth,
                     stream, error, cap);
}
