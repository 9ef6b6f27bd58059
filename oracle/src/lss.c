/*
 * Oracle lift-splat pooling: restates reference src/lss.c:8-241.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * geometry:  frustum point (u, v, d) -> undo the image augmentation
 *            (post_rotation^-1 (p - post_translation)), un-project
 *            (u*d, v*d, d), camera -> lidar (R K^-1 q + t), then the optional
 *            lidar augmentation (R_e q + t_e).  Singular post-rotation or
 *            intrinsics fail the call.
 * lift:      softmax over depth bins per pixel (max-shifted, sum in double)
 *            times the context vector.
 * pool:      every sample adds its lifted vector to the BEV cell
 *            trunc((p - min) / step) when that cell is inside the grid.
 * Per-element floating-point operation order matches the reference, so the
 * scalar build is bit-identical to it.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

/* 3x3 inverse by cofactors (lss.c:8-25); fails on a non-finite or tiny
 * determinant. */
static int inverse3(const float *m, float *r) {
    const float a = m[4] * m[8] - m[5] * m[7], b = m[2] * m[7] - m[1] * m[8];
    const float c = m[1] * m[5] - m[2] * m[4], d = m[5] * m[6] - m[3] * m[8];
    const float e = m[0] * m[8] - m[2] * m[6], f = m[2] * m[3] - m[0] * m[5];
    const float g = m[3] * m[7] - m[4] * m[6], h = m[1] * m[6] - m[0] * m[7];
    const float k = m[0] * m[4] - m[1] * m[3];
    const float det = m[0] * a + m[1] * d + m[2] * g;
    if (!isfinite(det) || fabsf(det) <= FLT_MIN) return 0;
    const float s = 1.0f / det;
    const float cof[9] = {a, b, c, d, e, f, g, h, k};
    for (int i = 0; i < 9; ++i) r[i] = cof[i] * s;
    return 1;
}

/* r = m v, each row summed left to right (lss.c:36-41). */
static void apply3(const float *m, const float *v, float *r) {
    for (int i = 0; i < 3; ++i) r[i] = m[3 * i] * v[0] + m[3 * i + 1] * v[1] + m[3 * i + 2] * v[2];
}

/* r = a b (lss.c:27-34): each entry accumulated from 0 over k. */
static void product3(const float *a, const float *b, float *r) {
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < 3; ++k) acc += a[3 * i + k] * b[3 * k + j];
            r[3 * i + j] = acc;
        }
}

static int checked_mul(size_t a, size_t b, size_t *r) {
    if (a && b > SIZE_MAX / a) return 0;
    *r = a * b;
    return 1;
}

/* Contract and sizes (lss.c:49-70). */
static int lss_sizes(const bf_lss_desc *d, size_t *samples, size_t *lifted, size_t *bev) {
    if (!d || !d->batches || !d->cameras || !d->depth_bins || !d->feature_height ||
        !d->feature_width || !d->channels)
        return 0;
    for (int a = 0; a < 3; ++a)
        if (!isfinite(d->grid_minimum[a]) || !isfinite(d->grid_step[a]) ||
            !(d->grid_step[a] > 0.0f) || !d->grid_cells[a] || d->grid_cells[a] > INT32_MAX)
            return 0;
    size_t n;
    if (!checked_mul(d->batches, d->cameras, &n) || !checked_mul(n, d->depth_bins, &n) ||
        !checked_mul(n, d->feature_height, &n) || !checked_mul(n, d->feature_width, samples) ||
        !checked_mul(*samples, d->channels, lifted))
        return 0;
    if (!checked_mul(d->batches, d->channels, &n) || !checked_mul(n, d->grid_cells[2], &n) ||
        !checked_mul(n, d->grid_cells[0], &n) || !checked_mul(n, d->grid_cells[1], bev))
        return 0;
    return 1;
}

int bf_lss_geometry_f32_ref(const float *frustum, const float *cam_rot, const float *cam_trans,
                            const float *intrinsics, const float *post_rot,
                            const float *post_trans, const float *extra_rot,
                            const float *extra_trans, float *geometry, size_t batches,
                            size_t cameras, size_t depth_bins, size_t height, size_t width) {
    if (!frustum || !cam_rot || !cam_trans || !intrinsics || !post_rot || !post_trans ||
        !geometry || !batches || !cameras || !depth_bins || !height || !width)
        return 0;
    const size_t per_camera = depth_bins * height * width;
    for (size_t b = 0; b < batches; ++b) {
        const float *er = extra_rot ? extra_rot + 9 * b : NULL;
        const float *et = extra_trans ? extra_trans + 3 * b : NULL;
        for (size_t n = 0; n < cameras; ++n) {
            const size_t cam = b * cameras + n;
            float post_inv[9], k_inv[9], to_lidar[9];
            if (!inverse3(post_rot + 9 * cam, post_inv) || !inverse3(intrinsics + 9 * cam, k_inv))
                return 0;
            product3(cam_rot + 9 * cam, k_inv, to_lidar);
            const float *pt = post_trans + 3 * cam, *ct = cam_trans + 3 * cam;
            float *out = geometry + 3 * per_camera * cam;
            for (size_t s = 0; s < per_camera; ++s) {
                const float *f = frustum + 3 * s;
                const float p[3] = {f[0] - pt[0], f[1] - pt[1], f[2] - pt[2]};
                float u[3], q[3], l[3];
                apply3(post_inv, p, u);
                q[0] = u[0] * u[2];
                q[1] = u[1] * u[2];
                q[2] = u[2];
                apply3(to_lidar, q, l);
                for (int i = 0; i < 3; ++i) l[i] += ct[i];
                float r[3] = {l[0], l[1], l[2]};
                if (er) apply3(er, l, r);
                if (et)
                    for (int i = 0; i < 3; ++i) r[i] += et[i];
                memcpy(out + 3 * s, r, sizeof r);
            }
        }
    }
    return 1;
}

/* Max-shifted softmax statistics of one pixel's depth column (lss.c:144-158):
 * fails on a non-finite logit. */
static int depth_stats(const float *col, size_t stride, size_t depths, float *maxv, float *inv) {
    float m = -FLT_MAX;
    for (size_t k = 0; k < depths; ++k) {
        const float v = col[k * stride];
        if (!isfinite(v)) return 0;
        if (v > m) m = v;
    }
    double total = 0.0;
    for (size_t k = 0; k < depths; ++k) total += expf(col[k * stride] - m);
    *maxv = m;
    *inv = (float)(1.0 / total);
    return isfinite(*inv);
}

int bf_lss_lift_f32_ref(const float *logits, const float *context, float *lifted,
                        const bf_lss_desc *d) {
    size_t samples, lifted_count, bev_count;
    if (!logits || !context || !lifted || !lss_sizes(d, &samples, &lifted_count, &bev_count))
        return 0;
    const size_t hw = d->feature_height * d->feature_width, C = d->channels, D = d->depth_bins;
    for (size_t cam = 0; cam < d->batches * d->cameras; ++cam)
        for (size_t p = 0; p < hw; ++p) {
            const float *col = logits + cam * D * hw + p;
            float m, inv;
            if (!depth_stats(col, hw, D, &m, &inv)) return 0;
            for (size_t k = 0; k < D; ++k) {
                const float prob = expf(col[k * hw] - m) * inv;
                float *row = lifted + ((cam * D + k) * hw + p) * C;
                for (size_t c = 0; c < C; ++c) row[c] = prob * context[(cam * C + c) * hw + p];
            }
        }
    return 1;
}

/* BEV cell of a metric point (lss.c:182-191): trunc((p - min) / step) per
 * axis, inside [0, cells). */
static int bev_cell(const float *p, const bf_lss_desc *d, int32_t cell[3]) {
    for (int a = 0; a < 3; ++a) {
        const float t = (p[a] - d->grid_minimum[a]) / d->grid_step[a];
        if (!isfinite(t) || t < (float)INT32_MIN || t > (float)INT32_MAX) return 0;
        cell[a] = (int32_t)t;
        if (cell[a] < 0 || (size_t)cell[a] >= d->grid_cells[a]) return 0;
    }
    return 1;
}

/* Offset of (batch, channel, cell) in [B, C*Z, X, Y] (lss.c:193-198). */
static size_t bev_offset(const bf_lss_desc *d, size_t b, size_t c, const int32_t cell[3]) {
    const size_t Z = d->grid_cells[2], X = d->grid_cells[0], Y = d->grid_cells[1];
    return ((b * (d->channels * Z) + c * Z + (size_t)cell[2]) * X + (size_t)cell[0]) * Y +
           (size_t)cell[1];
}

/* Test helper with no reference counterpart: every sample's cell rank within
 * its batch, (z * X + x) * Y + y, -1 outside the grid (the cell rule of
 * lss.c:182-191 in the rank order of cuda_lss.cu:244-253). */
int bf_oracle_lss_ranks(const float *geometry, int32_t *ranks, const bf_lss_desc *d) {
    size_t samples, lifted_count, bev_count;
    if (!geometry || !ranks || !lss_sizes(d, &samples, &lifted_count, &bev_count)) return 0;
    const int64_t X = (int64_t)d->grid_cells[0], Y = (int64_t)d->grid_cells[1];
    for (size_t s = 0; s < samples; ++s) {
        int32_t cell[3];
        ranks[s] = bev_cell(geometry + 3 * s, d, cell)
                       ? (int32_t)(((int64_t)cell[2] * X + cell[0]) * Y + cell[1])
                       : -1;
    }
    return 1;
}

int bf_lss_bev_pool_f32_ref(const float *lifted, const float *geometry, float *bev,
                            const bf_lss_desc *d) {
    size_t samples, lifted_count, bev_count;
    if (!lifted || !geometry || !bev || !lss_sizes(d, &samples, &lifted_count, &bev_count))
        return 0;
    memset(bev, 0, bev_count * sizeof *bev);
    const size_t per_batch = samples / d->batches;
    for (size_t s = 0; s < samples; ++s) {
        int32_t cell[3];
        if (!bev_cell(geometry + 3 * s, d, cell)) continue;
        for (size_t c = 0; c < d->channels; ++c)
            bev[bev_offset(d, s / per_batch, c, cell)] += lifted[s * d->channels + c];
    }
    return 1;
}

int bf_lss_lift_pool_f32_ref(const float *logits, const float *context, const float *geometry,
                             float *bev, const bf_lss_desc *d) {
    size_t samples, lifted_count, bev_count;
    if (!logits || !context || !geometry || !bev ||
        !lss_sizes(d, &samples, &lifted_count, &bev_count))
        return 0;
    memset(bev, 0, bev_count * sizeof *bev);
    const size_t hw = d->feature_height * d->feature_width, C = d->channels, D = d->depth_bins;
    for (size_t b = 0; b < d->batches; ++b)
        for (size_t n = 0; n < d->cameras; ++n) {
            const size_t cam = b * d->cameras + n;
            for (size_t p = 0; p < hw; ++p) {
                const float *col = logits + cam * D * hw + p;
                float m, inv;
                if (!depth_stats(col, hw, D, &m, &inv)) return 0;
                for (size_t k = 0; k < D; ++k) {
                    const size_t s = (cam * D + k) * hw + p;
                    int32_t cell[3];
                    if (!bev_cell(geometry + 3 * s, d, cell)) continue;
                    const float prob = expf(logits[s] - m) * inv;
                    for (size_t c = 0; c < C; ++c)
                        bev[bev_offset(d, b, c, cell)] += prob * context[(cam * C + c) * hw + p];
                }
            }
        }
    return 1;
}
