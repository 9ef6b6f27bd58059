/*
 * Oracle shifted-window attention: restates reference src/swin.c:10-311.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Semantics (mmdet ShiftWindowMSA): zero-pad H,W to multiples of the window,
 * then read window token (iy,ix) of window (wy,wx) from padded source
 * ((wy*w+iy+shift) mod Hp, (wx*w+ix+shift) mod Wp); padded sources are zero
 * rows, so their q/k/v equal the qkv bias.  Shifted blocks add -100 to scores
 * whose region labels differ (label = 3*region_y + region_x, region
 * 0/1/2 = p < P-w / p < P-shift / otherwise).  Outputs are written back
 * through the same map.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* swin.c:16-74: per-window QKV, per-head exact softmax attention, proj. */
static int window_core(const float *windows, const float *qkv_w, const float *qkv_b,
                       const float *rel_bias, const int64_t *rel_index,
                       const float *mask, size_t mask_windows,
                       const float *proj_w, const float *proj_b, float *output,
                       size_t total, size_t tokens, size_t c, size_t heads,
                       size_t bias_rows, float *qkv, float *score, float *mixed) {
    const size_t hd = c / heads;
    const float scale = 1.0f / sqrtf((float)hd);
    for (size_t win = 0; win < total; ++win) {
        bf_linear_f32(windows + win * tokens * c, qkv_w, qkv_b, qkv, tokens, c, 3 * c);
        memset(mixed, 0, tokens * c * sizeof(*mixed));
        for (size_t h = 0; h < heads; ++h)
            for (size_t q = 0; q < tokens; ++q) {
                const float *qrow = qkv + q * 3 * c + h * hd;
                float *srow = score + q * tokens;
                float best = -FLT_MAX;
                for (size_t k = 0; k < tokens; ++k) {
                    const int64_t r = rel_index[q * tokens + k];
                    if (r < 0 || (uint64_t)r >= bias_rows) return 0;
                    const float *krow = qkv + k * 3 * c + c + h * hd;
                    float s = rel_bias[(size_t)r * heads + h];
#if defined(BF_WITH_OPENMP)
#pragma omp simd reduction(+:s)
#endif
                    for (size_t e = 0; e < hd; ++e) s += qrow[e] * scale * krow[e];
                    if (mask) s += mask[((win % mask_windows) * tokens + q) * tokens + k];
                    srow[k] = s;
                    if (s > best) best = s;
                }
                double denom = 0.0;
                for (size_t k = 0; k < tokens; ++k) {
                    const float e = expf(srow[k] - best);
                    srow[k] = e;
                    denom += e;
                }
                const float inv = (float)(1.0 / denom);
                float *mrow = mixed + q * c + h * hd;
                for (size_t k = 0; k < tokens; ++k) {
                    const float p = srow[k] * inv;
                    const float *vrow = qkv + k * 3 * c + 2 * c + h * hd;
                    for (size_t e = 0; e < hd; ++e) mrow[e] += p * vrow[e];
                }
            }
        bf_linear_f32(mixed, proj_w, proj_b, output + win * tokens * c, tokens, c, c);
    }
    return 1;
}

/* swin.c:76-104 */
int bf_swin_window_attention_f32_ref(
    const float *windows, const float *qkv_w, const float *qkv_b,
    const float *rel_bias, const int64_t *rel_index, const float *mask,
    size_t mask_windows, const float *proj_w, const float *proj_b, float *output,
    size_t total, size_t tokens, size_t c, size_t heads, size_t bias_rows) {
    if (!windows || !qkv_w || !qkv_b || !rel_bias || !rel_index || !proj_w ||
        !proj_b || !output || !total || !tokens || !c || !heads || c % heads ||
        !bias_rows || (mask && !mask_windows))
        return 0;
    size_t nq, ns, nm;
    if (!bf_oracle_mul(tokens, 3 * c, &nq) || !bf_oracle_mul(tokens, tokens, &ns) ||
        !bf_oracle_mul(tokens, c, &nm))
        return 0;
    float *qkv = malloc(nq * sizeof(float)), *score = malloc(ns * sizeof(float));
    float *mixed = malloc(nm * sizeof(float));
    int ok = qkv && score && mixed &&
             window_core(windows, qkv_w, qkv_b, rel_bias, rel_index, mask, mask_windows,
                         proj_w, proj_b, output, total, tokens, c, heads, bias_rows,
                         qkv, score, mixed);
    free(qkv); free(score); free(mixed);
    return ok;
}

/* swin.c:106-110: padded coordinate read by shifted position p. */
static size_t shifted_source(size_t p, size_t extent, size_t shift) {
    return shift ? (p + shift) % extent : p;
}

/* swin.c:106-110 reverse branch: shifted position holding source p. */
static size_t shifted_home(size_t p, size_t extent, size_t shift) {
    return shift ? (p + extent - shift) % extent : p;
}

/* swin.c:112-117 */
static size_t region_of(size_t p, size_t extent, size_t window, size_t shift) {
    return p < extent - window ? 0 : (p < extent - shift ? 1 : 2);
}

static void window_mask(float *mask, size_t wy, size_t wx, size_t hp, size_t wp,
                        size_t window, size_t shift) {
    const size_t tokens = window * window;
    for (size_t a = 0; a < tokens; ++a) {
        const size_t la = region_of(wy * window + a / window, hp, window, shift) * 3 +
                          region_of(wx * window + a % window, wp, window, shift);
        for (size_t b = 0; b < tokens; ++b) {
            const size_t lb = region_of(wy * window + b / window, hp, window, shift) * 3 +
                              region_of(wx * window + b % window, wp, window, shift);
            mask[a * tokens + b] = la == lb ? 0.0f : -100.0f;
        }
    }
}

static int window_geometry(const bf_swin_window_desc *d, size_t *hp, size_t *wp) {
    if (d->height > SIZE_MAX - (d->window_size - 1) ||
        d->width > SIZE_MAX - (d->window_size - 1)) return 0;
    *hp = (d->height + d->window_size - 1) / d->window_size * d->window_size;
    *wp = (d->width + d->window_size - 1) / d->window_size * d->window_size;
    return 1;
}

/* swin.c:119-219: whole-tensor variant (all windows materialised). */
int bf_swin_shifted_window_f32_ref(
    const float *query, const float *qkv_w, const float *qkv_b,
    const float *rel_bias, const int64_t *rel_index, const float *proj_w,
    const float *proj_b, float *output, const bf_swin_window_desc *d) {
    if (!query || !qkv_w || !qkv_b || !rel_bias || !rel_index || !proj_w || !proj_b ||
        !output || !d || !d->batches || !d->height || !d->width || !d->channels ||
        !d->heads || d->channels % d->heads || !d->window_size ||
        d->shift_size >= d->window_size)
        return 0;
    size_t hp, wp;
    if (!window_geometry(d, &hp, &wp)) return 0;
    const size_t w = d->window_size, c = d->channels;
    const size_t ny = hp / w, nx = wp / w;
    size_t per_image, total, tokens, values, mvalues;
    if (!bf_oracle_mul(ny, nx, &per_image) || !bf_oracle_mul(d->batches, per_image, &total) ||
        !bf_oracle_mul(w, w, &tokens) || !bf_oracle_mul(total, tokens, &values) ||
        !bf_oracle_mul(values, c, &values) || !bf_oracle_mul(per_image, tokens, &mvalues) ||
        !bf_oracle_mul(mvalues, tokens, &mvalues))
        return 0;
    float *windows = calloc(values, sizeof(float));
    float *attended = malloc(values * sizeof(float));
    float *mask = d->shift_size ? malloc(mvalues * sizeof(float)) : NULL;
    if (!windows || !attended || (d->shift_size && !mask)) {
        free(windows); free(attended); free(mask);
        return 0;
    }
    for (size_t b = 0; b < d->batches; ++b)
        for (size_t wy = 0; wy < ny; ++wy)
            for (size_t wx = 0; wx < nx; ++wx)
                for (size_t t = 0; t < tokens; ++t) {
                    size_t sy = shifted_source(wy * w + t / w, hp, d->shift_size);
                    size_t sx = shifted_source(wx * w + t % w, wp, d->shift_size);
                    if (sy >= d->height || sx >= d->width) continue;
                    memcpy(windows + (((b * ny + wy) * nx + wx) * tokens + t) * c,
                           query + ((b * d->height + sy) * d->width + sx) * c, c * sizeof(float));
                }
    if (mask)
        for (size_t wy = 0; wy < ny; ++wy)
            for (size_t wx = 0; wx < nx; ++wx)
                window_mask(mask + (wy * nx + wx) * tokens * tokens, wy, wx, hp, wp, w,
                            d->shift_size);
    size_t side = 2 * w - 1, rows;
    int ok = bf_oracle_mul(side, side, &rows) &&
             bf_swin_window_attention_f32_ref(windows, qkv_w, qkv_b, rel_bias, rel_index,
                                              mask, mask ? per_image : 0, proj_w, proj_b,
                                              attended, total, tokens, c, d->heads, rows);
    if (ok)
        for (size_t b = 0; b < d->batches; ++b)
            for (size_t y = 0; y < d->height; ++y)
                for (size_t x = 0; x < d->width; ++x) {
                    size_t py = shifted_home(y, hp, d->shift_size);
                    size_t px = shifted_home(x, wp, d->shift_size);
                    size_t win = (b * ny + py / w) * nx + px / w;
                    size_t t = (py % w) * w + px % w;
                    memcpy(output + ((b * d->height + y) * d->width + x) * c,
                           attended + (win * tokens + t) * c, c * sizeof(float));
                }
    free(windows); free(attended); free(mask);
    return ok;
}

/* swin.c:221-230 */
size_t bf_swin_shifted_window_workspace_bytes(const bf_swin_window_desc *d) {
    if (!d || !d->channels || !d->window_size) return 0;
    size_t tokens, tc, tt;
    if (!bf_oracle_mul(d->window_size, d->window_size, &tokens) ||
        !bf_oracle_mul(tokens, d->channels, &tc) || tc > SIZE_MAX / 6 ||
        !bf_oracle_mul(tokens, tokens, &tt) || tt > SIZE_MAX / 2 ||
        6 * tc > SIZE_MAX - 2 * tt || 6 * tc + 2 * tt > SIZE_MAX / sizeof(float))
        return 0;
    return (6 * tc + 2 * tt) * sizeof(float);
}

/* swin.c:232-311: streamed one window at a time in a caller workspace laid
 * out as [window | attended | qkv(3) | scores | mixed | mask]. */
int bf_swin_shifted_window_f32_workspace_ref(
    const float *query, const float *qkv_w, const float *qkv_b,
    const float *rel_bias, const int64_t *rel_index, const float *proj_w,
    const float *proj_b, float *output, const bf_swin_window_desc *d,
    void *workspace, size_t workspace_bytes) {
    const size_t need = bf_swin_shifted_window_workspace_bytes(d);
    if (!query || !qkv_w || !qkv_b || !rel_bias || !rel_index || !proj_w || !proj_b ||
        !output || !d || !workspace || workspace_bytes < need || !d->batches ||
        !d->height || !d->width || !d->heads || d->channels % d->heads ||
        d->shift_size >= d->window_size)
        return 0;
    size_t hp, wp;
    if (!window_geometry(d, &hp, &wp)) return 0;
    const size_t w = d->window_size, c = d->channels, tokens = w * w, tc = tokens * c;
    const size_t ny = hp / w, nx = wp / w, rows = (2 * w - 1) * (2 * w - 1);
    float *win = (float *)workspace, *attended = win + tc, *qkv = attended + tc;
    float *score = qkv + 3 * tc, *mixed = score + tokens * tokens, *mask = mixed + tc;
    for (size_t b = 0; b < d->batches; ++b)
        for (size_t wy = 0; wy < ny; ++wy)
            for (size_t wx = 0; wx < nx; ++wx) {
                memset(win, 0, tc * sizeof(float));
                for (size_t t = 0; t < tokens; ++t) {
                    size_t sy = shifted_source(wy * w + t / w, hp, d->shift_size);
                    size_t sx = shifted_source(wx * w + t % w, wp, d->shift_size);
                    if (sy < d->height && sx < d->width)
                        memcpy(win + t * c, query + ((b * d->height + sy) * d->width + sx) * c,
                               c * sizeof(float));
                }
                if (d->shift_size) window_mask(mask, wy, wx, hp, wp, w, d->shift_size);
                if (!window_core(win, qkv_w, qkv_b, rel_bias, rel_index,
                                 d->shift_size ? mask : NULL, d->shift_size ? 1 : 0,
                                 proj_w, proj_b, attended, 1, tokens, c, d->heads, rows,
                                 qkv, score, mixed))
                    return 0;
                for (size_t t = 0; t < tokens; ++t) {
                    size_t sy = shifted_source(wy * w + t / w, hp, d->shift_size);
                    size_t sx = shifted_source(wx * w + t % w, wp, d->shift_size);
                    if (sy < d->height && sx < d->width)
                        memcpy(output + ((b * d->height + sy) * d->width + sx) * c,
                               attended + t * c, c * sizeof(float));
                }
            }
    return 1;
}
