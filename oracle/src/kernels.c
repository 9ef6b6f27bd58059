/*
 * Oracle operator library: restates reference src/kernels_ref.c:16-475.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Dispatch mirrors the reference: BF_CPU_SCALAR (non-empty, not "0") forces
 * the scalar *_ref routines; otherwise convolutions take the OpenMP spatial
 * sweep and linear layers an OpenMP row x column split.  No CBLAS is linked
 * (the image has none), so the backend reports "openmp" / "scalar".
 */
#include "oracle.h"

#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int bf_oracle_fail(char *error, size_t cap, const char *fmt, ...) {
    if (error && cap) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(error, cap, fmt, ap);
        va_end(ap);
    }
    return 0;
}

int bf_oracle_mul(size_t a, size_t b, size_t *out) {
    if (a && b > SIZE_MAX / a) return 0;
    *out = a * b;
    return 1;
}

/* Tensor binding with the dtype/rank/dims contract of the reference modules
 * (e.g. src/swin_backbone.c:58-77). */
const void *bf_oracle_bind(const bf_model *model, const char *name, uint32_t dtype,
                           uint32_t rank, const uint32_t *dims,
                           char *error, size_t cap) {
    const bf_tensor *t = bf_model_find(model, name);
    if (!t) { bf_oracle_fail(error, cap, "missing tensor %s", name); return NULL; }
    if (t->dtype != dtype || t->rank != rank) {
        bf_oracle_fail(error, cap, "%s: dtype/rank mismatch", name);
        return NULL;
    }
    for (uint32_t i = 0; i < rank; ++i)
        if (t->dims[i] != dims[i]) {
            bf_oracle_fail(error, cap, "%s: dimension %u is %u, expected %u",
                           name, i, t->dims[i], dims[i]);
            return NULL;
        }
    return t->data;
}

/* kernels_ref.c:16-19 */
static int scalar_forced(void) {
    const char *v = getenv("BF_CPU_SCALAR");
    return v && v[0] && strcmp(v, "0") != 0;
}

/* kernels_ref.c:21-36 (CBLAS/Accelerate branches absent in this build). */
const char *bf_cpu_kernel_backend(void) {
    if (scalar_forced()) return "scalar-forced";
#if defined(BF_WITH_OPENMP)
    return "openmp";
#else
    return "scalar";
#endif
}

/* kernels_ref.c:38-61: standard output extent with dilation and groups. */
int bf_conv2d_output_shape(const bf_conv2d_desc *d, size_t *oh, size_t *ow) {
    if (!d || !oh || !ow || !d->n || !d->in_channels || !d->in_height ||
        !d->in_width || !d->out_channels || !d->kernel_height ||
        !d->kernel_width || !d->stride_height || !d->stride_width ||
        !d->dilation_height || !d->dilation_width || !d->groups ||
        d->in_channels % d->groups || d->out_channels % d->groups)
        return 0;
    if (d->kernel_height > (SIZE_MAX - 1) / d->dilation_height + 1 ||
        d->kernel_width > (SIZE_MAX - 1) / d->dilation_width + 1)
        return 0;
    size_t span_h = d->dilation_height * (d->kernel_height - 1) + 1;
    size_t span_w = d->dilation_width * (d->kernel_width - 1) + 1;
    if (d->pad_height > (SIZE_MAX - d->in_height) / 2 ||
        d->pad_width > (SIZE_MAX - d->in_width) / 2)
        return 0;
    size_t ph = d->in_height + 2 * d->pad_height, pw = d->in_width + 2 * d->pad_width;
    if (span_h > ph || span_w > pw) return 0;
    *oh = (ph - span_h) / d->stride_height + 1;
    *ow = (pw - span_w) / d->stride_width + 1;
    return *oh && *ow;
}

/* kernels_ref.c:63-102: direct convolution.  Per output element the sum
 * starts at the bias and accumulates taps in (ci, ky, kx) order, skipping
 * taps that fall into the zero padding. */
int bf_conv2d_f32_ref(const float *input, const float *weight, const float *bias,
                      float *output, const bf_conv2d_desc *d) {
    size_t oh, ow;
    if (!input || !weight || !output || !bf_conv2d_output_shape(d, &oh, &ow)) return 0;
    const size_t cig = d->in_channels / d->groups, cog = d->out_channels / d->groups;
    const size_t ihw = d->in_height * d->in_width;
    for (size_t n = 0; n < d->n; ++n)
        for (size_t co = 0; co < d->out_channels; ++co) {
            const size_t c0 = (co / cog) * cig;
            const float *wco = weight + co * cig * d->kernel_height * d->kernel_width;
            float *dst = output + (n * d->out_channels + co) * oh * ow;
            for (size_t y = 0; y < oh; ++y)
                for (size_t x = 0; x < ow; ++x) {
                    float acc = bias ? bias[co] : 0.0f;
                    for (size_t c = 0; c < cig; ++c) {
                        const float *plane = input + (n * d->in_channels + c0 + c) * ihw;
                        const float *wc = wco + c * d->kernel_height * d->kernel_width;
                        for (size_t ky = 0; ky < d->kernel_height; ++ky) {
                            size_t py = y * d->stride_height + ky * d->dilation_height;
                            if (py < d->pad_height || py - d->pad_height >= d->in_height) continue;
                            const float *row = plane + (py - d->pad_height) * d->in_width;
                            for (size_t kx = 0; kx < d->kernel_width; ++kx) {
                                size_t px = x * d->stride_width + kx * d->dilation_width;
                                if (px < d->pad_width || px - d->pad_width >= d->in_width) continue;
                                acc += row[px - d->pad_width] * wc[ky * d->kernel_width + kx];
                            }
                        }
                    }
                    dst[y * ow + x] = acc;
                }
        }
    return 1;
}

/* kernels_ref.c:104-121: [begin,end) of outputs whose tap at kernel offset
 * `off` lands inside the unpadded input. */
static void tap_range(size_t outputs, size_t input, size_t stride, size_t pad,
                      size_t off, size_t *begin, size_t *end) {
    size_t lo = 0, hi = 0;
    if (off < pad) lo = (pad - off + stride - 1) / stride;
    if (off < pad + input) hi = (pad + input - off + stride - 1) / stride;
    if (lo > outputs) lo = outputs;
    if (hi > outputs) hi = outputs;
    *begin = lo;
    *end = hi < lo ? lo : hi;
}

/* kernels_ref.c:123-179: OpenMP spatial sweep.  One task per (n, co) plane;
 * taps are visited in (ci, ky, kx) order, so every element receives exactly
 * the same sequence of additions as the direct routine above. */
static int conv2d_sweep(const float *input, const float *weight, const float *bias,
                        float *output, const bf_conv2d_desc *d, size_t oh, size_t ow) {
    const size_t cig = d->in_channels / d->groups, cog = d->out_channels / d->groups;
    const size_t tasks = d->n * d->out_channels;
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static)
#endif
    for (size_t task = 0; task < tasks; ++task) {
        const size_t n = task / d->out_channels, co = task % d->out_channels;
        const size_t c0 = (co / cog) * cig;
        float *dst = output + task * oh * ow;
        const float start = bias ? bias[co] : 0.0f;
        for (size_t i = 0; i < oh * ow; ++i) dst[i] = start;
        for (size_t c = 0; c < cig; ++c) {
            const float *plane = input + (n * d->in_channels + c0 + c) * d->in_height * d->in_width;
            for (size_t ky = 0; ky < d->kernel_height; ++ky) {
                size_t y0, y1;
                const size_t oy = ky * d->dilation_height;
                tap_range(oh, d->in_height, d->stride_height, d->pad_height, oy, &y0, &y1);
                for (size_t kx = 0; kx < d->kernel_width; ++kx) {
                    const float w = weight[((co * cig + c) * d->kernel_height + ky) *
                                           d->kernel_width + kx];
                    size_t x0, x1;
                    const size_t ox = kx * d->dilation_width;
                    tap_range(ow, d->in_width, d->stride_width, d->pad_width, ox, &x0, &x1);
                    for (size_t y = y0; y < y1; ++y) {
                        const float *src = plane + (y * d->stride_height + oy - d->pad_height) * d->in_width;
                        float *out = dst + y * ow;
#if defined(BF_WITH_OPENMP)
#pragma omp simd
#endif
                        for (size_t x = x0; x < x1; ++x)
                            out[x] += src[x * d->stride_width + ox - d->pad_width] * w;
                    }
                }
            }
        }
    }
    return 1;
}

/* kernels_ref.c:181-212 without the CBLAS 1x1 branch (no CBLAS here). */
int bf_conv2d_f32(const float *input, const float *weight, const float *bias,
                  float *output, const bf_conv2d_desc *d) {
    size_t oh, ow;
    if (!input || !weight || !output || !bf_conv2d_output_shape(d, &oh, &ow)) return 0;
    if (scalar_forced()) return bf_conv2d_f32_ref(input, weight, bias, output, d);
    return conv2d_sweep(input, weight, bias, output, d, oh, ow);
}

/* kernels_ref.c:214-227: extent of one transposed-convolution axis. */
static int tconv_extent(size_t in, size_t k, size_t stride, size_t pad,
                        size_t opad, size_t dil, size_t *out) {
    if (!in || !k || !stride || !dil || opad >= stride || k > (SIZE_MAX - 1) / dil + 1)
        return 0;
    size_t span = dil * (k - 1) + 1;
    if (span > SIZE_MAX - opad) return 0;
    size_t tail = span + opad;
    if (in - 1 > (SIZE_MAX - tail) / stride) return 0;
    size_t full = (in - 1) * stride + tail;
    if (pad > full / 2 || full - 2 * pad == 0) return 0;
    *out = full - 2 * pad;
    return 1;
}

int bf_conv_transpose2d_output_shape(const bf_conv_transpose2d_desc *d,
                                     size_t *oh, size_t *ow) {
    if (!d || !oh || !ow || !d->n || !d->in_channels || !d->out_channels ||
        !d->groups || d->in_channels % d->groups || d->out_channels % d->groups)
        return 0;
    return tconv_extent(d->in_height, d->kernel_height, d->stride_height, d->pad_height,
                        d->output_pad_height, d->dilation_height, oh) &&
           tconv_extent(d->in_width, d->kernel_width, d->stride_width, d->pad_width,
                        d->output_pad_width, d->dilation_width, ow);
}

/* kernels_ref.c:242-290: scatter form, IOHW weights. */
int bf_conv_transpose2d_f32_ref(const float *input, const float *weight,
                                const float *bias, float *output,
                                const bf_conv_transpose2d_desc *d) {
    size_t oh, ow;
    if (!input || !weight || !output || !bf_conv_transpose2d_output_shape(d, &oh, &ow))
        return 0;
    if (oh > SIZE_MAX / ow) return 0;
    const size_t ohw = oh * ow;
    if (d->n > SIZE_MAX / d->out_channels || d->n * d->out_channels > SIZE_MAX / ohw) return 0;
    for (size_t n = 0; n < d->n; ++n)
        for (size_t co = 0; co < d->out_channels; ++co) {
            float *dst = output + (n * d->out_channels + co) * ohw;
            for (size_t i = 0; i < ohw; ++i) dst[i] = bias ? bias[co] : 0.0f;
        }
    const size_t cig = d->in_channels / d->groups, cog = d->out_channels / d->groups;
    const size_t khw = d->kernel_height * d->kernel_width;
    for (size_t n = 0; n < d->n; ++n)
        for (size_t ci = 0; ci < d->in_channels; ++ci) {
            const size_t g = ci / cig;
            for (size_t iy = 0; iy < d->in_height; ++iy)
                for (size_t ix = 0; ix < d->in_width; ++ix) {
                    const float v = input[((n * d->in_channels + ci) * d->in_height + iy) * d->in_width + ix];
                    for (size_t cl = 0; cl < cog; ++cl) {
                        const size_t co = g * cog + cl;
                        const float *w = weight + (ci * cog + cl) * khw;
                        float *dst = output + (n * d->out_channels + co) * ohw;
                        for (size_t ky = 0; ky < d->kernel_height; ++ky) {
                            size_t py = iy * d->stride_height + ky * d->dilation_height;
                            if (py < d->pad_height || py - d->pad_height >= oh) continue;
                            for (size_t kx = 0; kx < d->kernel_width; ++kx) {
                                size_t px = ix * d->stride_width + kx * d->dilation_width;
                                if (px < d->pad_width || px - d->pad_width >= ow) continue;
                                dst[(py - d->pad_height) * ow + (px - d->pad_width)] +=
                                    v * w[ky * d->kernel_width + kx];
                            }
                        }
                    }
                }
        }
    return 1;
}

/* kernels_ref.c:292-302: y = x W^T + b, W is [out, in]. */
void bf_linear_f32_ref(const float *x, const float *w, const float *b, float *y,
                       size_t rows, size_t in_f, size_t out_f) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * in_f;
        for (size_t o = 0; o < out_f; ++o) {
            const float *wo = w + o * in_f;
            float acc = b ? b[o] : 0.0f;
            for (size_t i = 0; i < in_f; ++i) acc += xr[i] * wo[i];
            y[r * out_f + o] = acc;
        }
    }
}

/* kernels_ref.c:304-339 without the CBLAS branch. */
void bf_linear_f32(const float *x, const float *w, const float *b, float *y,
                   size_t rows, size_t in_f, size_t out_f) {
    if (scalar_forced()) {
        bf_linear_f32_ref(x, w, b, y, rows, in_f, out_f);
        return;
    }
#if defined(BF_WITH_OPENMP)
    const size_t tasks = rows * out_f;
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < tasks; ++t) {
        const size_t r = t / out_f, o = t % out_f;
        const float *xr = x + r * in_f, *wo = w + o * in_f;
        float acc = b ? b[o] : 0.0f;
#pragma omp simd reduction(+:acc)
        for (size_t i = 0; i < in_f; ++i) acc += xr[i] * wo[i];
        y[t] = acc;
    }
#else
    bf_linear_f32_ref(x, w, b, y, rows, in_f, out_f);
#endif
}

/* kernels_ref.c:341-355: eval-mode batch norm, per-channel affine. */
void bf_batch_norm_2d_f32_ref(const float *in, const float *scale, const float *bias,
                              const float *mean, const float *var, float eps,
                              float *out, size_t n, size_t c, size_t h, size_t w) {
    const size_t hw = h * w;
    for (size_t b = 0; b < n; ++b)
        for (size_t ch = 0; ch < c; ++ch) {
            const float f = scale[ch] / sqrtf(var[ch] + eps);
            const float o = bias[ch] - mean[ch] * f;
            const size_t base = (b * c + ch) * hw;
            for (size_t i = 0; i < hw; ++i) out[base + i] = in[base + i] * f + o;
        }
}

/* kernels_ref.c:357-380 */
void bf_batch_norm_2d_f32(const float *in, const float *scale, const float *bias,
                          const float *mean, const float *var, float eps,
                          float *out, size_t n, size_t c, size_t h, size_t w) {
    if (scalar_forced()) {
        bf_batch_norm_2d_f32_ref(in, scale, bias, mean, var, eps, out, n, c, h, w);
        return;
    }
    const size_t hw = h * w, tasks = n * c;
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static) if(tasks * hw >= 4096)
#endif
    for (size_t t = 0; t < tasks; ++t) {
        const size_t ch = t % c;
        const float f = scale[ch] / sqrtf(var[ch] + eps);
        const float o = bias[ch] - mean[ch] * f;
        for (size_t i = 0; i < hw; ++i) out[t * hw + i] = in[t * hw + i] * f + o;
    }
}

/* kernels_ref.c:382-400: two-pass statistics in double, applied in float. */
static void layer_norm_row(const float *src, const float *scale, const float *bias,
                           float eps, float *dst, size_t c) {
    double s = 0.0;
    for (size_t i = 0; i < c; ++i) s += src[i];
    const float mean = (float)(s / (double)c);
    double ss = 0.0;
    for (size_t i = 0; i < c; ++i) {
        const double dv = (double)src[i] - mean;
        ss += dv * dv;
    }
    const float inv = 1.0f / sqrtf((float)(ss / (double)c) + eps);
    for (size_t i = 0; i < c; ++i) dst[i] = (src[i] - mean) * inv * scale[i] + bias[i];
}

void bf_layer_norm_f32_ref(const float *in, const float *scale, const float *bias,
                           float eps, float *out, size_t rows, size_t c) {
    for (size_t r = 0; r < rows; ++r)
        layer_norm_row(in + r * c, scale, bias, eps, out + r * c, c);
}

/* kernels_ref.c:402-428 */
void bf_layer_norm_f32(const float *in, const float *scale, const float *bias,
                       float eps, float *out, size_t rows, size_t c) {
    if (scalar_forced()) {
        bf_layer_norm_f32_ref(in, scale, bias, eps, out, rows, c);
        return;
    }
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static) if(rows * c >= 4096)
#endif
    for (size_t r = 0; r < rows; ++r)
        layer_norm_row(in + r * c, scale, bias, eps, out + r * c, c);
}

/* kernels_ref.c:430-446: max-shifted softmax, double denominator. */
void bf_softmax_f32_ref(const float *in, float *out, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float *s = in + r * cols;
        float *d = out + r * cols;
        float m = -FLT_MAX;
        for (size_t i = 0; i < cols; ++i) m = s[i] > m ? s[i] : m;
        double sum = 0.0;
        for (size_t i = 0; i < cols; ++i) {
            d[i] = expf(s[i] - m);
            sum += d[i];
        }
        const float inv = (float)(1.0 / sum);
        for (size_t i = 0; i < cols; ++i) d[i] *= inv;
    }
}

/* kernels_ref.c:448-462: exact-erf GELU. */
static const float kInvSqrt2 = 0.7071067811865475244f;

void bf_gelu_f32_ref(const float *in, float *out, size_t count) {
    for (size_t i = 0; i < count; ++i)
        out[i] = 0.5f * in[i] * (1.0f + erff(in[i] * kInvSqrt2));
}

void bf_gelu_f32(const float *in, float *out, size_t count) {
    if (scalar_forced()) { bf_gelu_f32_ref(in, out, count); return; }
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static) if(count >= 4096)
#endif
    for (size_t i = 0; i < count; ++i)
        out[i] = 0.5f * in[i] * (1.0f + erff(in[i] * kInvSqrt2));
}

/* kernels_ref.c:464-475 */
void bf_relu_f32_ref(const float *in, float *out, size_t count) {
    for (size_t i = 0; i < count; ++i) out[i] = in[i] > 0.0f ? in[i] : 0.0f;
}

void bf_relu_f32(const float *in, float *out, size_t count) {
    if (scalar_forced()) { bf_relu_f32_ref(in, out, count); return; }
#if defined(BF_WITH_OPENMP)
#pragma omp parallel for schedule(static) if(count >= 4096)
#endif
    for (size_t i = 0; i < count; ++i) out[i] = in[i] > 0.0f ? in[i] : 0.0f;
}
