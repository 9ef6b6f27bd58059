/*
 * Oracle camera neck: restates reference src/image_fpn.c:10-197,
 * src/depth_head.c:10-190 and src/lss_downsample.c:10-148.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Every convolution goes through bf_conv2d_f32 followed by eval-mode
 * BatchNorm and ReLU as separate passes, exactly as the reference CPU modules
 * do (the GPU contexts fold BN into the weights instead).
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { const float *scale, *bias, *mean, *var; } bound_bn;

static int bind_bn(const bf_model *m, const char *prefix, size_t c, bound_bn *bn,
                   char *e, size_t cap) {
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float **slot[4] = {&bn->scale, &bn->bias, &bn->mean, &bn->var};
    const uint32_t dims[1] = {(uint32_t)c};
    char name[160];
    for (int i = 0; i < 4; ++i) {
        snprintf(name, sizeof(name), "%s.%s", prefix, suffix[i]);
        *slot[i] = (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, 1, dims, e, cap);
        if (!*slot[i]) return 0;
    }
    return 1;
}

static void bn_relu(float *v, const bound_bn *bn, size_t c, size_t h, size_t w) {
    bf_batch_norm_2d_f32(v, bn->scale, bn->bias, bn->mean, bn->var, 1e-5f, v, 1, c, h, w);
    bf_relu_f32(v, v, c * h * w);
}

/* ===================== GeneralizedLSSFPN (image_fpn.c) =================== */
struct bf_image_fpn {
    const float *lateral_w[2], *output_w[2];
    bound_bn lateral_bn[2], output_bn[2];
};

/* image_fpn.c:73-100 */
int bf_image_fpn_create(const bf_model *model, bf_image_fpn **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid image FPN arguments");
    bf_image_fpn *f = calloc(1, sizeof(*f));
    if (!f) return bf_oracle_fail(error, cap, "image FPN allocation failed");
    static const uint32_t lateral_in[2] = {448, 1152};
    char name[160];
    for (int l = 0; l < 2; ++l) {
        const uint32_t ld[4] = {256, lateral_in[l], 1, 1}, od[4] = {256, 256, 3, 3};
        snprintf(name, sizeof(name), "neck.lateral_convs.%d.conv.weight", l);
        f->lateral_w[l] = (const float *)bf_oracle_bind(model, name, BF_DTYPE_F32, 4, ld, error, cap);
        if (!f->lateral_w[l]) goto fail;
        snprintf(name, sizeof(name), "neck.lateral_convs.%d.bn", l);
        if (!bind_bn(model, name, 256, &f->lateral_bn[l], error, cap)) goto fail;
        snprintf(name, sizeof(name), "neck.fpn_convs.%d.conv.weight", l);
        f->output_w[l] = (const float *)bf_oracle_bind(model, name, BF_DTYPE_F32, 4, od, error, cap);
        if (!f->output_w[l]) goto fail;
        snprintf(name, sizeof(name), "neck.fpn_convs.%d.bn", l);
        if (!bind_bn(model, name, 256, &f->output_bn[l], error, cap)) goto fail;
    }
    *out = f;
    return 1;
fail:
    free(f);
    return 0;
}

void bf_image_fpn_destroy(bf_image_fpn *f) { free(f); }

/* image_fpn.c:104-114: concat buffer (max of both levels) + one 256-ch level-0 map. */
size_t bf_image_fpn_workspace_bytes(size_t h, size_t w) {
    if (!h || !w || h > SIZE_MAX - 3 || w > SIZE_MAX - 3) return 0;
    size_t l0, l1, t;
    if (!bf_oracle_mul(h, w, &l0) || !bf_oracle_mul(l0, 448, &l0) ||
        !bf_oracle_mul((h + 1) / 2, (w + 1) / 2, &l1) || !bf_oracle_mul(l1, 1152, &l1))
        return 0;
    size_t concat = l0 > l1 ? l0 : l1;
    if (!bf_oracle_mul(h, w, &t) || !bf_oracle_mul(t, 256, &t) || concat > SIZE_MAX - t ||
        !bf_oracle_mul(concat + t, sizeof(float), &concat))
        return 0;
    return concat;
}

/* image_fpn.c:123-142: bilinear resize, align_corners=False, source
 * coordinate (o+0.5)*in/out-0.5 clamped at 0, upper neighbour clamped to
 * the last row/column. */
static void bilinear(const float *in, size_t ih, size_t iw, float *out, size_t oh, size_t ow) {
    for (size_t y = 0; y < oh; ++y) {
        float sy = ((float)y + 0.5f) * (float)ih / (float)oh - 0.5f;
        if (sy < 0.0f) sy = 0.0f;
        const size_t y0 = (size_t)floorf(sy), y1 = y0 + 1 < ih ? y0 + 1 : y0;
        const float fy = sy - (float)y0;
        for (size_t x = 0; x < ow; ++x) {
            float sx = ((float)x + 0.5f) * (float)iw / (float)ow - 0.5f;
            if (sx < 0.0f) sx = 0.0f;
            const size_t x0 = (size_t)floorf(sx), x1 = x0 + 1 < iw ? x0 + 1 : x0;
            const float fx = sx - (float)x0;
            const float top = in[y0 * iw + x0] * (1.0f - fx) + in[y0 * iw + x1] * fx;
            const float bot = in[y1 * iw + x0] * (1.0f - fx) + in[y1 * iw + x1] * fx;
            out[y * ow + x] = top * (1.0f - fy) + bot * fy;
        }
    }
}

/* image_fpn.c:144-168: concat(lower, up(upper)) -> 1x1 -> BN/ReLU -> 3x3 -> BN/ReLU. */
static int fuse_level(const bf_image_fpn *f, int level, const float *lower, size_t cl,
                      size_t oh, size_t ow, const float *upper, size_t cu, size_t ih,
                      size_t iw, float *out, float *concat, float *tmp) {
    const size_t ohw = oh * ow, ihw = ih * iw;
    memcpy(concat, lower, cl * ohw * sizeof(float));
    for (size_t c = 0; c < cu; ++c)
        bilinear(upper + c * ihw, ih, iw, concat + (cl + c) * ohw, oh, ow);
    const bf_conv2d_desc lat = {1, cl + cu, oh, ow, 256, 1, 1, 1, 1, 0, 0, 1, 1, 1};
    if (!bf_conv2d_f32(concat, f->lateral_w[level], NULL, tmp, &lat)) return 0;
    bn_relu(tmp, &f->lateral_bn[level], 256, oh, ow);
    const bf_conv2d_desc fin = {1, 256, oh, ow, 256, 3, 3, 1, 1, 1, 1, 1, 1, 1};
    if (!bf_conv2d_f32(tmp, f->output_w[level], NULL, out, &fin)) return 0;
    bn_relu(out, &f->output_bn[level], 256, oh, ow);
    return 1;
}

/* image_fpn.c:170-197 */
int bf_image_fpn_forward_ref(const bf_image_fpn *f, const float *in0, const float *in1,
                             const float *in2, size_t batches, size_t h0, size_t w0,
                             float *out0, float *out1, void *workspace,
                             size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_image_fpn_workspace_bytes(h0, w0);
    if (!f || !in0 || !in1 || !in2 || !batches || !h0 || !w0 || !out0 || !out1 ||
        !workspace || !need || workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid image FPN buffers or dimensions");
    const size_t h1 = (h0 + 1) / 2, w1 = (w0 + 1) / 2, h2 = (h1 + 1) / 2, w2 = (w1 + 1) / 2;
    const size_t c0 = 448 * h0 * w0, c1 = 1152 * h1 * w1;
    float *concat = (float *)workspace, *tmp = concat + (c0 > c1 ? c0 : c1);
    for (size_t b = 0; b < batches; ++b) {
        float *o1 = out1 + b * 256 * h1 * w1;
        if (!fuse_level(f, 1, in1 + b * 384 * h1 * w1, 384, h1, w1, in2 + b * 768 * h2 * w2,
                        768, h2, w2, o1, concat, tmp))
            return bf_oracle_fail(error, cap, "image FPN level 1 failed");
        if (!fuse_level(f, 0, in0 + b * 192 * h0 * w0, 192, h0, w0, o1, 256, h1, w1,
                        out0 + b * 256 * h0 * w0, concat, tmp))
            return bf_oracle_fail(error, cap, "image FPN level 0 failed");
    }
    return 1;
}

/* ========================= DepthLSS head (depth_head.c) ================= */
typedef struct { const float *weight, *bias; bound_bn bn; } bound_conv;

struct bf_depth_head {
    bound_conv dtransform[3], trunk[2];
    const float *out_w, *out_b;
};

static int bind_conv(const bf_model *m, const char *base, int conv, int bn, size_t co,
                     size_t ci, size_t k, bound_conv *out, char *e, size_t cap) {
    char name[160];
    const uint32_t wd[4] = {(uint32_t)co, (uint32_t)ci, (uint32_t)k, (uint32_t)k};
    const uint32_t bd[1] = {(uint32_t)co};
    snprintf(name, sizeof(name), "%s.%d.weight", base, conv);
    out->weight = (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, 4, wd, e, cap);
    snprintf(name, sizeof(name), "%s.%d.bias", base, conv);
    out->bias = (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, 1, bd, e, cap);
    snprintf(name, sizeof(name), "%s.%d", base, bn);
    return out->weight && out->bias && bind_bn(m, name, co, &out->bn, e, cap);
}

/* depth_head.c:96-123 */
int bf_depth_head_create(const bf_model *model, bf_depth_head **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid depth-head arguments");
    bf_depth_head *d = calloc(1, sizeof(*d));
    if (!d) return bf_oracle_fail(error, cap, "depth-head allocation failed");
    const uint32_t wd[4] = {198, 256, 1, 1}, bd[1] = {198};
    if (!bind_conv(model, "vtransform.dtransform", 0, 1, 8, 1, 1, &d->dtransform[0], error, cap) ||
        !bind_conv(model, "vtransform.dtransform", 3, 4, 32, 8, 5, &d->dtransform[1], error, cap) ||
        !bind_conv(model, "vtransform.dtransform", 6, 7, 64, 32, 5, &d->dtransform[2], error, cap) ||
        !bind_conv(model, "vtransform.depthnet", 0, 1, 256, 320, 3, &d->trunk[0], error, cap) ||
        !bind_conv(model, "vtransform.depthnet", 3, 4, 256, 256, 3, &d->trunk[1], error, cap))
        goto fail;
    d->out_w = (const float *)bf_oracle_bind(model, "vtransform.depthnet.6.weight",
                                             BF_DTYPE_F32, 4, wd, error, cap);
    d->out_b = (const float *)bf_oracle_bind(model, "vtransform.depthnet.6.bias",
                                             BF_DTYPE_F32, 1, bd, error, cap);
    if (!d->out_w || !d->out_b) goto fail;
    *out = d;
    return 1;
fail:
    free(d);
    return 0;
}

void bf_depth_head_destroy(bf_depth_head *d) { free(d); }

/* depth_head.c:127-133: two 384-channel buffers at feature resolution
 * (the reference bounds each by 512*H*W and 256*H*W floats). */
size_t bf_depth_head_workspace_bytes(size_t h, size_t w) {
    if (!h || !w || h > SIZE_MAX / 8 || w > SIZE_MAX / 8) return 0;
    size_t hw, v;
    if (!bf_oracle_mul(h, w, &hw) || !bf_oracle_mul(hw, 768, &v) ||
        !bf_oracle_mul(v, sizeof(float), &v))
        return 0;
    return v;
}

static int conv_bn_relu(const float *in, const bound_conv *c, float *out, size_t ci,
                        size_t co, size_t h, size_t w, size_t k, size_t stride, size_t pad) {
    const bf_conv2d_desc d = {1, ci, h, w, co, k, k, stride, stride, pad, pad, 1, 1, 1};
    size_t oh, ow;
    if (!bf_conv2d_f32(in, c->weight, c->bias, out, &d) || !bf_conv2d_output_shape(&d, &oh, &ow))
        return 0;
    bn_relu(out, &c->bn, co, oh, ow);
    return 1;
}

/* depth_head.c:155-190 */
int bf_depth_head_forward_ref(const bf_depth_head *d, const float *features,
                              const float *depth, size_t batches, size_t h, size_t w,
                              float *logits, float *context, void *workspace,
                              size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_depth_head_workspace_bytes(h, w);
    if (!d || !features || !depth || !batches || !h || !w || !logits || !context ||
        !workspace || !need || workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid depth-head buffers or dimensions");
    const size_t hw = h * w, ih = 8 * h, iw = 8 * w;
    float *a = (float *)workspace, *b = a + 512 * hw;
    for (size_t n = 0; n < batches; ++n) {
        if (!conv_bn_relu(depth + n * ih * iw, &d->dtransform[0], a, 1, 8, ih, iw, 1, 1, 0) ||
            !conv_bn_relu(a, &d->dtransform[1], b, 8, 32, ih, iw, 5, 4, 2) ||
            !conv_bn_relu(b, &d->dtransform[2], a, 32, 64, 2 * h, 2 * w, 5, 2, 2))
            return bf_oracle_fail(error, cap, "depth image encoder failed at camera %zu", n);
        memmove(a + 64 * hw, features + n * 256 * hw, 256 * hw * sizeof(float));
        if (!conv_bn_relu(a, &d->trunk[0], b, 320, 256, h, w, 3, 1, 1) ||
            !conv_bn_relu(b, &d->trunk[1], a, 256, 256, h, w, 3, 1, 1))
            return bf_oracle_fail(error, cap, "depth prediction trunk failed at camera %zu", n);
        const bf_conv2d_desc fin = {1, 256, h, w, 198, 1, 1, 1, 1, 0, 0, 1, 1, 1};
        if (!bf_conv2d_f32(a, d->out_w, d->out_b, b, &fin))
            return bf_oracle_fail(error, cap, "depth prediction output failed at camera %zu", n);
        memcpy(logits + n * 118 * hw, b, 118 * hw * sizeof(float));
        memcpy(context + n * 80 * hw, b + 118 * hw, 80 * hw * sizeof(float));
    }
    return 1;
}

/* ===================== post-LSS downsample (lss_downsample.c) ============ */
struct bf_lss_downsample {
    const float *weight[3];
    bound_bn bn[3];
};

/* lss_downsample.c:70-90 */
int bf_lss_downsample_create(const bf_model *model, bf_lss_downsample **out,
                             char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid LSS downsample arguments");
    bf_lss_downsample *s = calloc(1, sizeof(*s));
    if (!s) return bf_oracle_fail(error, cap, "LSS downsample allocation failed");
    static const int conv_idx[3] = {0, 3, 6}, bn_idx[3] = {1, 4, 7};
    const uint32_t wd[4] = {80, 80, 3, 3};
    char name[160];
    for (int l = 0; l < 3; ++l) {
        snprintf(name, sizeof(name), "vtransform.downsample.%d.weight", conv_idx[l]);
        s->weight[l] = (const float *)bf_oracle_bind(model, name, BF_DTYPE_F32, 4, wd, error, cap);
        snprintf(name, sizeof(name), "vtransform.downsample.%d", bn_idx[l]);
        if (!s->weight[l] || !bind_bn(model, name, 80, &s->bn[l], error, cap)) {
            free(s);
            return 0;
        }
    }
    *out = s;
    return 1;
}

void bf_lss_downsample_destroy(bf_lss_downsample *s) { free(s); }

/* lss_downsample.c:117-126 (workspace: full-res 80-ch map + half-res map). */
size_t bf_lss_downsample_workspace_bytes(size_t h, size_t w) {
    if (!h || !w || (h & 1) || (w & 1)) return 0;
    size_t full, half;
    if (!bf_oracle_mul(h, w, &full) || !bf_oracle_mul(full, 80, &full) ||
        !bf_oracle_mul(h / 2, w / 2, &half) || !bf_oracle_mul(half, 80, &half) ||
        full > SIZE_MAX - half || !bf_oracle_mul(full + half, sizeof(float), &full))
        return 0;
    return full;
}

static int conv80(const float *in, const float *w, float *out, size_t h, size_t wd, size_t s) {
    const bf_conv2d_desc d = {1, 80, h, wd, 80, 3, 3, s, s, 1, 1, 1, 1, 1};
    return bf_conv2d_f32(in, w, NULL, out, &d);
}

/* lss_downsample.c:117-148: conv s1 -> conv s2 -> conv s1, each BN+ReLU,
 * then out[c][x][y] = result[c][y][x] on the half-resolution map. */
int bf_lss_downsample_forward_ref(const bf_lss_downsample *s, const float *input,
                                  size_t batches, size_t h, size_t w, float *output,
                                  void *workspace, size_t workspace_bytes, char *error,
                                  size_t cap) {
    const size_t need = bf_lss_downsample_workspace_bytes(h, w);
    if (!s || !input || !batches || !h || !w || !output || !workspace || !need ||
        workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid LSS downsample buffers or dimensions");
    const size_t hh = h / 2, hw = w / 2;
    float *full = (float *)workspace, *half = full + 80 * h * w;
    for (size_t n = 0; n < batches; ++n) {
        if (!conv80(input + n * 80 * h * w, s->weight[0], full, h, w, 1))
            return bf_oracle_fail(error, cap, "LSS downsample convolution 0 failed");
        bn_relu(full, &s->bn[0], 80, h, w);
        if (!conv80(full, s->weight[1], half, h, w, 2))
            return bf_oracle_fail(error, cap, "LSS downsample convolution 1 failed");
        bn_relu(half, &s->bn[1], 80, hh, hw);
        if (!conv80(half, s->weight[2], full, hh, hw, 1))
            return bf_oracle_fail(error, cap, "LSS downsample convolution 2 failed");
        bn_relu(full, &s->bn[2], 80, hh, hw);
        float *dst = output + n * 80 * hh * hw;
        for (size_t c = 0; c < 80; ++c)
            for (size_t y = 0; y < hh; ++y)
                for (size_t x = 0; x < hw; ++x)
                    dst[(c * hw + x) * hh + y] = full[(c * hh + y) * hw + x];
    }
    return 1;
}
