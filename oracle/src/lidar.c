/*
 * Oracle LiDAR side: restates reference src/depth_raster.c:14-105 (point
 * projection into the six dense depth images), src/voxel.c:13-151
 * (voxelisation in first-encounter order), src/kernels_ref.c:477-490
 * (MeanVFE) and 516-772 (sparse 3-D convolution), and
 * src/lidar_backbone.c:86-273 (the SECOND sparse encoder).  TEST
 * INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Per-element floating-point operation order follows the reference, so the
 * scalar build is bit-identical to the reference's C compiled here.  The
 * coordinate tables differ in method only: output sites are found through a
 * sorted key array and binary search instead of an open-addressing hash; the
 * sites and their order (ascending (batch, z, y, x)) are the same.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================= depth raster (depth_raster.c) =================== */
/* Inverse of the upper-left 3x3 of a row-major 4x4 by cofactors
 * (depth_raster.c:14-35). */
static int lr_inverse3(const float *m, float *out) {
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
    if (!isfinite(det) || fabsf(det) <= FLT_MIN) return 0;
    const float s = 1.0f / det;
    out[0] = c00 * s; out[1] = c01 * s; out[2] = c02 * s;
    out[3] = c10 * s; out[4] = c11 * s; out[5] = c12 * s;
    out[6] = c20 * s; out[7] = c21 * s; out[8] = c22 * s;
    return 1;
}

/* depth_raster.c:49-105: points [P, stride] = (batch, x, y, z, ...); later
 * points overwrite earlier ones at a shared pixel. */
int bf_depth_rasterize_f32_ref(const float *points, size_t point_count, size_t stride,
                               const float *lidar_aug, const float *lidar_to_image,
                               const float *image_aug, float *depth, size_t batches,
                               size_t cameras, size_t height, size_t width) {
    size_t count;
    if ((!points && point_count) || stride < 4 || !lidar_aug || !lidar_to_image ||
        !image_aug || !depth || !batches || !cameras || !height || !width ||
        !bf_oracle_mul(batches, cameras, &count) || !bf_oracle_mul(count, height, &count) ||
        !bf_oracle_mul(count, width, &count))
        return 0;
    memset(depth, 0, count * sizeof(float));
    for (size_t b = 0; b < batches; ++b) {
        const float *aug = lidar_aug + b * 16;
        float inv[9];
        if (!lr_inverse3(aug, inv)) return 0;
        for (size_t p = 0; p < point_count; ++p) {
            const float *pt = points + p * stride;
            if (!isfinite(pt[0]) || pt[0] != (float)b) continue;
            const float c0 = pt[1] - aug[3], c1 = pt[2] - aug[7], c2 = pt[3] - aug[11];
            if (!isfinite(c0) || !isfinite(c1) || !isfinite(c2)) continue;
            const float u0 = inv[0] * c0 + inv[1] * c1 + inv[2] * c2;
            const float u1 = inv[3] * c0 + inv[4] * c1 + inv[5] * c2;
            const float u2 = inv[6] * c0 + inv[7] * c1 + inv[8] * c2;
            for (size_t cam = 0; cam < cameras; ++cam) {
                const size_t ci = b * cameras + cam;
                const float *pr = lidar_to_image + ci * 16, *post = image_aug + ci * 16;
                float q0 = pr[0] * u0 + pr[1] * u1 + pr[2] * u2;
                float q1 = pr[4] * u0 + pr[5] * u1 + pr[6] * u2;
                float q2 = pr[8] * u0 + pr[9] * u1 + pr[10] * u2;
                q0 += pr[3];
                q1 += pr[7];
                q2 += pr[11];
                if (!isfinite(q0) || !isfinite(q1) || !isfinite(q2)) continue;
                float dist = q2;
                if (dist < 1e-5f) dist = 1e-5f;
                if (dist > 1e5f) dist = 1e5f;
                const float n0 = q0 / dist, n1 = q1 / dist, n2 = dist;
                float ax = post[0] * n0 + post[1] * n1 + post[2] * n2;
                float ay = post[4] * n0 + post[5] * n1 + post[6] * n2;
                ax += post[3];
                ay += post[7];
                if (!isfinite(ax) || !isfinite(ay) || ax < 0.0f || ax >= (float)width ||
                    ay < 0.0f || ay >= (float)height)
                    continue;
                depth[(ci * height + (size_t)ay) * width + (size_t)ax] = dist;
            }
        }
    }
    return 1;
}

/* ======================= voxeliser (voxel.c) ============================= */
static uint64_t lr_mix64(uint64_t v) {
    v ^= v >> 30;
    v *= 0xbf58476d1ce4e5b9ull;
    v ^= v >> 27;
    v *= 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

static size_t lr_table_capacity(size_t n) {
    if (!n || n > SIZE_MAX / 2) return 0;
    size_t c = 2;
    while (c < n * 2) {
        if (c > SIZE_MAX / 2) return 0;
        c <<= 1;
    }
    return c;
}

/* voxel.c:31-49: cells per axis = round(extent / size), within 1e-4. */
int bf_voxel_grid_shape(const bf_voxel_config *cfg, size_t grid[3]) {
    if (!cfg || !grid || !cfg->point_features || !cfg->max_points_per_voxel || !cfg->max_voxels)
        return 0;
    for (int a = 0; a < 3; ++a) {
        const float extent = cfg->maximum[a] - cfg->minimum[a], size = cfg->voxel_size[a];
        if (!isfinite(extent) || !isfinite(size) || extent <= 0.0f || size <= 0.0f) return 0;
        const double cells = (double)extent / size;
        const long long r = llround(cells);
        if (r <= 0 || (double)r > (double)SIZE_MAX || fabs(cells - (double)r) > 1e-4 * fmax(1.0, cells))
            return 0;
        grid[a] = (size_t)r;
    }
    return 1;
}

typedef struct { uint64_t key; size_t value; } lr_slot;

size_t bf_voxelize_workspace_bytes(const bf_voxel_config *cfg) {
    const size_t c = cfg ? lr_table_capacity(cfg->max_voxels) : 0;
    return c && c <= SIZE_MAX / sizeof(lr_slot) ? c * sizeof(lr_slot) : 0;
}

/* voxel.c:57-138: points in input order; a voxel is created at its first
 * point (until max_voxels exist), keeps its first max_points_per_voxel points. */
int bf_voxelize_f32_workspace_ref(const float *points, size_t point_count, size_t stride,
                                  int32_t batch, const bf_voxel_config *cfg, float *voxels,
                                  bf_coord4 *coords, int64_t *counts, size_t *voxel_count,
                                  bf_voxel_stats *stats, void *workspace, size_t workspace_bytes) {
    if (voxel_count) *voxel_count = 0;
    if (stats) memset(stats, 0, sizeof(*stats));
    size_t grid[3];
    if (!points || !cfg || !voxels || !coords || !counts || !voxel_count || !stats || !workspace ||
        batch < 0 || stride < cfg->point_features || cfg->point_features < 3 ||
        !bf_voxel_grid_shape(cfg, grid))
        return 0;
    const size_t cap = lr_table_capacity(cfg->max_voxels), need = bf_voxelize_workspace_bytes(cfg);
    if (!cap || !need || workspace_bytes < need) return 0;
    lr_slot *table = workspace;
    memset(table, 0, need);
    stats->input_points = point_count;
    const size_t F = cfg->point_features, M = cfg->max_points_per_voxel;
    size_t live = 0;
    for (size_t p = 0; p < point_count; ++p) {
        const float *pt = points + p * stride;
        int finite = 1;
        for (size_t f = 0; f < F; ++f) finite &= isfinite(pt[f]);
        if (!finite) {
            ++stats->rejected_nonfinite;
            continue;
        }
        int32_t cell[3];
        int inside = 1;
        for (int a = 0; a < 3 && inside; ++a) {
            if (pt[a] < cfg->minimum[a] || pt[a] >= cfg->maximum[a]) {
                inside = 0;
                break;
            }
            cell[a] = (int32_t)floorf((pt[a] - cfg->minimum[a]) / cfg->voxel_size[a]);
            if (cell[a] < 0 || (size_t)cell[a] >= grid[a]) inside = 0;
        }
        if (!inside) {
            ++stats->rejected_out_of_range;
            continue;
        }
        const uint64_t key = ((uint64_t)(uint32_t)cell[2] * grid[1] + (uint32_t)cell[1]) * grid[0] +
                             (uint32_t)cell[0] + 1;
        size_t slot = (size_t)lr_mix64(key) & (cap - 1);
        while (table[slot].key && table[slot].key != key) slot = (slot + 1) & (cap - 1);
        size_t v;
        if (!table[slot].key) {
            if (live == cfg->max_voxels) {
                ++stats->dropped_voxel_capacity;
                continue;
            }
            v = live++;
            table[slot].key = key;
            table[slot].value = v;
            coords[v] = (bf_coord4){batch, cell[2], cell[1], cell[0]};
            counts[v] = 0;
            memset(voxels + v * M * F, 0, M * F * sizeof(float));
        } else {
            v = table[slot].value;
        }
        if ((size_t)counts[v] == M) {
            ++stats->dropped_point_capacity;
            continue;
        }
        memcpy(voxels + (v * M + (size_t)counts[v]) * F, pt, F * sizeof(float));
        ++counts[v];
        ++stats->accepted_points;
    }
    *voxel_count = live;
    return 1;
}

/* kernels_ref.c:477-490: mean of each voxel's first min(count, max) points. */
void bf_mean_vfe_f32_ref(const float *points, const int64_t *counts, float *out, size_t voxels,
                         size_t max_points, size_t channels) {
    for (size_t v = 0; v < voxels; ++v) {
        size_t live = counts[v] <= 0 ? 0 : (size_t)counts[v];
        if (live > max_points) live = max_points;
        for (size_t c = 0; c < channels; ++c) {
            float sum = 0.0f;
            for (size_t p = 0; p < live; ++p) sum += points[(v * max_points + p) * channels + c];
            out[v * channels + c] = live ? sum / (float)live : 0.0f;
        }
    }
}

/* ======================= sparse 3-D convolution ========================== */
/* Linear site key (kernels_ref.c:536-552): ((b D + z) H + y) W + x + 1. */
static int lr_key(bf_coord4 c, size_t b, size_t d, size_t h, size_t w, uint64_t *key) {
    if (c.batch < 0 || c.z < 0 || c.y < 0 || c.x < 0 || (size_t)c.batch >= b ||
        (size_t)c.z >= d || (size_t)c.y >= h || (size_t)c.x >= w)
        return 0;
    *key = (((uint64_t)c.batch * d + (uint32_t)c.z) * h + (uint32_t)c.y) * w + (uint32_t)c.x + 1;
    return 1;
}

static int lr_axis(size_t in, size_t k, size_t s, size_t p, size_t dil, size_t *out) {
    if (!in || !k || !s || !dil) return 0;
    const size_t eff = dil * (k - 1) + 1, padded = in + 2 * p;
    if (eff > padded) return 0;
    *out = (padded - eff) / s + 1;
    return *out != 0;
}

/* kernels_ref.c:596-622 */
int bf_sparse_conv3d_output_shape(const bf_sparse_conv3d_desc *d, size_t *od, size_t *oh,
                                  size_t *ow) {
    if (!d || !od || !oh || !ow || !d->batches || !d->in_channels || !d->out_channels ||
        d->batches > INT32_MAX || d->in_depth > INT32_MAX || d->in_height > INT32_MAX ||
        d->in_width > INT32_MAX)
        return 0;
    if (d->submanifold) {
        if (d->stride_depth != 1 || d->stride_height != 1 || d->stride_width != 1) return 0;
        *od = d->in_depth;
        *oh = d->in_height;
        *ow = d->in_width;
        return *od && *oh && *ow;
    }
    return lr_axis(d->in_depth, d->kernel_depth, d->stride_depth, d->pad_depth,
                   d->dilation_depth, od) &&
           lr_axis(d->in_height, d->kernel_height, d->stride_height, d->pad_height,
                   d->dilation_height, oh) &&
           lr_axis(d->in_width, d->kernel_width, d->stride_width, d->pad_width,
                   d->dilation_width, ow);
}

typedef struct { uint64_t key; size_t index; } lr_site;

static int lr_site_order(const void *l, const void *r) {
    const lr_site *a = l, *b = r;
    return (a->key > b->key) - (a->key < b->key);
}

/* Index of `key` in a key-sorted site array, or SIZE_MAX. */
static size_t lr_find(const lr_site *s, size_t n, uint64_t key) {
    size_t lo = 0, hi = n;
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (s[mid].key < key) lo = mid + 1;
        else hi = mid;
    }
    return lo < n && s[lo].key == key ? s[lo].index : SIZE_MAX;
}

/* One output axis candidate: (in + pad - k dil) / stride when exact and in
 * range (kernels_ref.c:632-644). */
static int lr_candidate(int32_t in, size_t k, size_t pad, size_t dil, size_t s, size_t lim,
                        int32_t *out) {
    const int64_t num = (int64_t)in + (int64_t)pad - (int64_t)k * (int64_t)dil;
    if (num < 0 || num % (int64_t)s) return 0;
    const int64_t v = num / (int64_t)s;
    if (v >= (int64_t)lim) return 0;
    *out = (int32_t)v;
    return 1;
}

size_t bf_sparse_conv3d_workspace_bytes(size_t in_cap, size_t out_cap) {
    size_t n, bytes;
    if (!in_cap || !out_cap || in_cap > SIZE_MAX - out_cap) return 0;
    n = in_cap + out_cap;
    return bf_oracle_mul(n, sizeof(lr_site), &bytes) ? bytes : 0;
}

/* kernels_ref.c:655-756.  Output sites: the input sites (submanifold) or
 * every exact strided image of an input site under each kernel tap, unique,
 * in ascending key order; more than out_cap sites fail.  Each output channel
 * starts at the bias and adds, tap by tap (kz, ky, kx) and then input channel
 * by input channel, source feature x weight[tap][ci][co]. */
int bf_sparse_conv3d_f32_workspace_ref(const bf_coord4 *in_coords, const float *in_features,
                                       size_t in_count, const float *weight, const float *bias,
                                       bf_coord4 *out_coords, float *out_features, size_t out_cap,
                                       size_t *out_count, const bf_sparse_conv3d_desc *d,
                                       void *workspace, size_t workspace_bytes) {
    if (out_count) *out_count = 0;
    size_t od, oh, ow;
    if (!in_coords || !in_features || !in_count || !weight || !out_coords || !out_features ||
        !out_count || !workspace || !bf_sparse_conv3d_output_shape(d, &od, &oh, &ow))
        return 0;
    const size_t need = bf_sparse_conv3d_workspace_bytes(in_count, out_cap);
    if (!need || workspace_bytes < need) return 0;
    lr_site *in_sites = workspace, *out_sites = in_sites + in_count;
    for (size_t i = 0; i < in_count; ++i) {
        if (!lr_key(in_coords[i], d->batches, d->in_depth, d->in_height, d->in_width,
                    &in_sites[i].key))
            return 0;
        in_sites[i].index = i;
    }
    qsort(in_sites, in_count, sizeof(lr_site), lr_site_order);
    for (size_t i = 1; i < in_count; ++i)
        if (in_sites[i].key == in_sites[i - 1].key) return 0;  /* duplicate input site */
    size_t count = 0;
    if (d->submanifold) {
        if (in_count > out_cap) return 0;
        for (size_t i = 0; i < in_count; ++i) out_sites[count++] = in_sites[i];
    } else {
        /* Candidate keys of every input site and tap, then sort + unique. */
        const size_t taps = d->kernel_depth * d->kernel_height * d->kernel_width;
        size_t cand;
        if (!bf_oracle_mul(in_count, taps, &cand)) return 0;
        uint64_t *keys = malloc((cand ? cand : 1) * sizeof(uint64_t));
        if (!keys) return 0;
        size_t n = 0;
        for (size_t i = 0; i < in_count; ++i)
            for (size_t kz = 0; kz < d->kernel_depth; ++kz)
                for (size_t ky = 0; ky < d->kernel_height; ++ky)
                    for (size_t kx = 0; kx < d->kernel_width; ++kx) {
                        bf_coord4 c = {in_coords[i].batch, 0, 0, 0};
                        if (!lr_candidate(in_coords[i].z, kz, d->pad_depth, d->dilation_depth,
                                          d->stride_depth, od, &c.z) ||
                            !lr_candidate(in_coords[i].y, ky, d->pad_height, d->dilation_height,
                                          d->stride_height, oh, &c.y) ||
                            !lr_candidate(in_coords[i].x, kx, d->pad_width, d->dilation_width,
                                          d->stride_width, ow, &c.x))
                            continue;
                        if (!lr_key(c, d->batches, od, oh, ow, &keys[n])) {
                            free(keys);
                            return 0;
                        }
                        ++n;
                    }
        lr_site *tmp = malloc((n ? n : 1) * sizeof(lr_site));
        if (!tmp) {
            free(keys);
            return 0;
        }
        for (size_t i = 0; i < n; ++i) tmp[i] = (lr_site){keys[i], 0};
        free(keys);
        qsort(tmp, n, sizeof(lr_site), lr_site_order);
        for (size_t i = 0; i < n; ++i) {
            if (count && tmp[i].key == out_sites[count - 1].key) continue;
            if (count == out_cap) {
                free(tmp);
                return 0;
            }
            out_sites[count++] = tmp[i];
        }
        free(tmp);
    }
    /* Output coordinates from the sorted keys. */
    for (size_t o = 0; o < count; ++o) {
        uint64_t k = out_sites[o].key - 1;
        bf_coord4 c;
        c.x = (int32_t)(k % ow);
        k /= ow;
        c.y = (int32_t)(k % oh);
        k /= oh;
        c.z = (int32_t)(k % od);
        c.batch = (int32_t)(k / od);
        out_coords[o] = c;
    }
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static)
#endif
    for (size_t o = 0; o < count; ++o) {
        const bf_coord4 oc = out_coords[o];
        float *dst = out_features + o * d->out_channels;
        for (size_t co = 0; co < d->out_channels; ++co) dst[co] = bias ? bias[co] : 0.0f;
        for (size_t kz = 0; kz < d->kernel_depth; ++kz)
            for (size_t ky = 0; ky < d->kernel_height; ++ky)
                for (size_t kx = 0; kx < d->kernel_width; ++kx) {
                    const int64_t iz = (int64_t)oc.z * (int64_t)d->stride_depth -
                                       (int64_t)d->pad_depth + (int64_t)(kz * d->dilation_depth);
                    const int64_t iy = (int64_t)oc.y * (int64_t)d->stride_height -
                                       (int64_t)d->pad_height + (int64_t)(ky * d->dilation_height);
                    const int64_t ix = (int64_t)oc.x * (int64_t)d->stride_width -
                                       (int64_t)d->pad_width + (int64_t)(kx * d->dilation_width);
                    if (iz < 0 || iy < 0 || ix < 0 || iz >= (int64_t)d->in_depth ||
                        iy >= (int64_t)d->in_height || ix >= (int64_t)d->in_width)
                        continue;
                    uint64_t key;
                    lr_key((bf_coord4){oc.batch, (int32_t)iz, (int32_t)iy, (int32_t)ix},
                           d->batches, d->in_depth, d->in_height, d->in_width, &key);
                    const size_t src = lr_find(in_sites, in_count, key);
                    if (src == SIZE_MAX) continue;
                    const size_t tap = (kz * d->kernel_height + ky) * d->kernel_width + kx;
                    const float *sf = in_features + src * d->in_channels;
                    const float *kw = weight + tap * d->in_channels * d->out_channels;
                    for (size_t co = 0; co < d->out_channels; ++co) {
                        float sum = dst[co];
#if defined(BF_WITH_OPENMP)
#pragma omp simd reduction(+:sum)
#endif
                        for (size_t ci = 0; ci < d->in_channels; ++ci)
                            sum += sf[ci] * kw[ci * d->out_channels + co];
                        dst[co] = sum;
                    }
                }
    }
    *out_count = count;
    return 1;
}

/* ======================= SECOND sparse encoder (lidar_backbone.c) ======== */
typedef struct { const float *scale, *bias, *mean, *var; } lr_bn;
typedef struct {
    const float *weight;
    lr_bn bn;
    size_t ci, co, kd, kh, kw, sd, sh, sw, pd, ph, pw;
    int subm;
} lr_layer;

struct bf_lidar_backbone {
    lr_layer input, residual[4][2][2], down[3], output;
};

static int lr_bind_layer(const bf_model *m, lr_layer *l, const char *wname, const char *bn,
                         size_t ci, size_t co, size_t kd, size_t kh, size_t kw, size_t sd,
                         size_t sh, size_t sw, size_t pd, size_t ph, size_t pw, int subm,
                         char *e, size_t cap) {
    const uint32_t wd[5] = {(uint32_t)kd, (uint32_t)kh, (uint32_t)kw, (uint32_t)ci, (uint32_t)co};
    l->weight = bf_oracle_bind(m, wname, BF_DTYPE_F32, 5, wd, e, cap);
    if (!l->weight) return 0;
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float **slot[4] = {&l->bn.scale, &l->bn.bias, &l->bn.mean, &l->bn.var};
    const uint32_t cd[1] = {(uint32_t)co};
    char name[192];
    for (int i = 0; i < 4; ++i) {
        snprintf(name, sizeof(name), "%s.%s", bn, suffix[i]);
        if (!(*slot[i] = bf_oracle_bind(m, name, BF_DTYPE_F32, 1, cd, e, cap))) return 0;
    }
    *l = (lr_layer){l->weight, l->bn, ci, co, kd, kh, kw, sd, sh, sw, pd, ph, pw, subm};
    return 1;
}

/* lidar_backbone.c:94-133: layer table of the checkpoint. */
int bf_lidar_backbone_create(const bf_model *model, bf_lidar_backbone **out, char *error,
                             size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid lidar backbone arguments");
    bf_lidar_backbone *n = calloc(1, sizeof(*n));
    if (!n) return bf_oracle_fail(error, cap, "lidar backbone allocation failed");
    static const size_t ch[4] = {16, 32, 64, 128};
    char w[160], b[160];
    if (!lr_bind_layer(model, &n->input, "backbone_3d.conv_input.0.weight",
                       "backbone_3d.conv_input.1", 5, 16, 3, 3, 3, 1, 1, 1, 1, 1, 1, 1, error, cap))
        goto fail;
    for (size_t s = 0; s < 4; ++s)
        for (size_t blk = 0; blk < 2; ++blk)
            for (size_t c = 0; c < 2; ++c) {
                snprintf(w, sizeof(w), "backbone_3d.conv%zu.%zu.conv%zu.weight", s + 1,
                         blk + (s ? 1 : 0), c + 1);
                snprintf(b, sizeof(b), "backbone_3d.conv%zu.%zu.bn%zu", s + 1, blk + (s ? 1 : 0),
                         c + 1);
                if (!lr_bind_layer(model, &n->residual[s][blk][c], w, b, ch[s], ch[s], 3, 3, 3, 1,
                                   1, 1, 1, 1, 1, 1, error, cap))
                    goto fail;
            }
    for (size_t t = 0; t < 3; ++t) {
        snprintf(w, sizeof(w), "backbone_3d.conv%zu.0.0.weight", t + 2);
        snprintf(b, sizeof(b), "backbone_3d.conv%zu.0.1", t + 2);
        if (!lr_bind_layer(model, &n->down[t], w, b, ch[t], ch[t + 1], 3, 3, 3, 2, 2, 2,
                           t + 2 == 4 ? 0 : 1, 1, 1, 0, error, cap))
            goto fail;
    }
    if (!lr_bind_layer(model, &n->output, "backbone_3d.conv_out.0.weight",
                       "backbone_3d.conv_out.1", 128, 128, 3, 1, 1, 2, 1, 1, 0, 0, 0, 0, error,
                       cap))
        goto fail;
    *out = n;
    return 1;
fail:
    free(n);
    return 0;
}

void bf_lidar_backbone_destroy(bf_lidar_backbone *n) { free(n); }

/* lidar_backbone.c:137-145 (the sparse workspace is this oracle's own). */
size_t bf_lidar_backbone_workspace_bytes(size_t capacity) {
    size_t f, c, s;
    if (!capacity || !bf_oracle_mul(capacity, 3 * 128 * sizeof(float), &f) ||
        !bf_oracle_mul(capacity, 2 * sizeof(bf_coord4), &c) || f > SIZE_MAX - c)
        return 0;
    s = bf_sparse_conv3d_workspace_bytes(capacity, capacity);
    return s && f + c <= SIZE_MAX - s ? f + c + s : 0;
}

/* lidar_backbone.c:147-162 */
int bf_lidar_backbone_output_shape(size_t d, size_t h, size_t w, size_t *od, size_t *oh,
                                   size_t *ow) {
    if (!d || !h || !w || !od || !oh || !ow) return 0;
    for (size_t s = 0; s < 3; ++s) {
        const size_t pz = s == 2 ? 0 : 1;
        if (d + 2 * pz < 3) return 0;
        d = (d + 2 * pz - 3) / 2 + 1;
        h = (h + 2 - 3) / 2 + 1;
        w = (w + 2 - 3) / 2 + 1;
    }
    if (d < 3) return 0;
    *od = (d - 3) / 2 + 1;
    *oh = h;
    *ow = w;
    return *od && *oh && *ow;
}

/* lidar_backbone.c:164-172: eval BN (epsilon 1e-3), optional ReLU. */
static void lr_bn_relu(float *f, size_t rows, size_t ch, const lr_bn *bn, int relu) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < ch; ++c) {
            const float k = bn->scale[c] / sqrtf(bn->var[c] + 1e-3f);
            const float v = (f[r * ch + c] - bn->mean[c]) * k + bn->bias[c];
            f[r * ch + c] = relu && v < 0.0f ? 0.0f : v;
        }
}

static int lr_run(const lr_layer *l, const bf_coord4 *ic, const float *inf, size_t n,
                  bf_coord4 *oc, float *of, size_t capacity, size_t b, size_t d, size_t h, size_t w,
                  size_t *count, size_t *od, size_t *oh, size_t *ow, int relu, void *ws,
                  size_t wsb) {
    const bf_sparse_conv3d_desc desc = {b, d, h, w, l->ci, l->co, l->kd, l->kh, l->kw,
                                        l->sd, l->sh, l->sw, l->pd, l->ph, l->pw, 1, 1, 1,
                                        l->subm};
    if (!bf_sparse_conv3d_output_shape(&desc, od, oh, ow) ||
        !bf_sparse_conv3d_f32_workspace_ref(ic, inf, n, l->weight, NULL, oc, of, capacity, count,
                                            &desc, ws, wsb))
        return 0;
    lr_bn_relu(of, *count, l->co, &l->bn, relu);
    return 1;
}

/* lidar_backbone.c:191-273: input SubM conv, four stages of two residual
 * SubM blocks (stages 2-4 entered by a strided conv), the (3,1,1)/(2,1,1)
 * output conv, then a dense scatter into [B,128,D,H,W]. */
int bf_lidar_backbone_forward_ref(const bf_lidar_backbone *net, const bf_coord4 *vc,
                                  const float *vf, size_t nv, size_t batches, size_t d, size_t h,
                                  size_t w, size_t capacity, float *dense, void *workspace,
                                  size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_lidar_backbone_workspace_bytes(capacity);
    size_t od, oh, ow;
    if (!net || !vc || !vf || !nv || nv > capacity || !batches || !d || !h || !w || !dense ||
        !workspace || !need || workspace_bytes < need ||
        !bf_lidar_backbone_output_shape(d, h, w, &od, &oh, &ow))
        return bf_oracle_fail(error, cap, "invalid lidar backbone buffers or dimensions");
    bf_coord4 *coords[2] = {workspace, (bf_coord4 *)workspace + capacity};
    float *fb = (float *)(coords[1] + capacity);
    float *feat[3] = {fb, fb + capacity * 128, fb + capacity * 256};
    void *ws = fb + capacity * 384;
    const size_t wsb = need - (size_t)((unsigned char *)ws - (unsigned char *)workspace);
    const bf_coord4 *cc = vc;
    const float *cf = vf;
    size_t cn = nv, cs = 1, fs = 0, nd, nh, nw;
    if (!lr_run(&net->input, cc, cf, cn, coords[0], feat[0], capacity, batches, d, h, w, &cn, &nd,
                &nh, &nw, 1, ws, wsb))
        return bf_oracle_fail(error, cap, "lidar input sparse convolution failed");
    cc = coords[0];
    cf = feat[0];
    cs = 0;
    for (size_t s = 0; s < 4; ++s) {
        if (s) {
            const size_t ncs = cs ^ 1, nfs = (fs + 1) % 3;
            if (!lr_run(&net->down[s - 1], cc, cf, cn, coords[ncs], feat[nfs], capacity, batches,
                        d, h, w, &cn, &nd, &nh, &nw, 1, ws, wsb))
                return bf_oracle_fail(error, cap, "lidar stage %zu downsample failed", s);
            d = nd;
            h = nh;
            w = nw;
            cs = ncs;
            fs = nfs;
            cc = coords[cs];
            cf = feat[fs];
        }
        for (size_t blk = 0; blk < 2; ++blk) {
            const size_t fc = cs ^ 1, f1 = (fs + 1) % 3, f2 = (fs + 2) % 3;
            size_t n1, n2;
            if (!lr_run(&net->residual[s][blk][0], cc, cf, cn, coords[fc], feat[f1], capacity,
                        batches, d, h, w, &n1, &nd, &nh, &nw, 1, ws, wsb) ||
                !lr_run(&net->residual[s][blk][1], coords[fc], feat[f1], n1, coords[cs],
                        feat[f2], capacity, batches, d, h, w, &n2, &nd, &nh, &nw, 0, ws, wsb) ||
                n2 != cn)
                return bf_oracle_fail(error, cap, "lidar stage %zu residual block %zu failed", s,
                                      blk);
            const size_t total = cn * net->residual[s][blk][1].co;
            for (size_t i = 0; i < total; ++i) {
                const float v = feat[f2][i] + cf[i];
                feat[f2][i] = v > 0.0f ? v : 0.0f;
            }
            fs = f2;
            cc = coords[cs];
            cf = feat[fs];
        }
    }
    const size_t fc = cs ^ 1, ff = (fs + 1) % 3;
    size_t fn;
    if (!lr_run(&net->output, cc, cf, cn, coords[fc], feat[ff], capacity, batches, d, h, w, &fn,
                &nd, &nh, &nw, 1, ws, wsb))
        return bf_oracle_fail(error, cap, "lidar output sparse convolution failed");
    size_t dn;
    if (!bf_oracle_mul(batches, 128, &dn) || !bf_oracle_mul(dn, nd, &dn) ||
        !bf_oracle_mul(dn, nh, &dn) || !bf_oracle_mul(dn, nw, &dn))
        return bf_oracle_fail(error, cap, "lidar dense output overflow");
    memset(dense, 0, dn * sizeof(float));
    const size_t sp = nh * nw;
    for (size_t i = 0; i < fn; ++i) {
        const bf_coord4 c = coords[fc][i];
        for (size_t ch = 0; ch < 128; ++ch)
            dense[(((size_t)c.batch * 128 + ch) * nd + (size_t)c.z) * sp + (size_t)c.y * nw +
                  (size_t)c.x] = feat[ff][i * 128 + ch];
    }
    return 1;
}
