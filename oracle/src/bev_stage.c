/*
 * Oracle BEV stage: restates reference src/bev_stage.c:16-227 (fuser, SECOND
 * backbone with two deblocks, TransFusion shared conv and heatmap head).
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Every convolution goes through bf_conv2d_f32 (the deblock.1 transposed
 * 2x2/s2 conv through bf_conv_transpose2d_f32_ref), followed by eval-mode
 * BatchNorm (epsilon 1e-3) and ReLU as separate passes, in the reference's
 * order; shared and heatmap-output convs carry their own bias and no BN.
 */
#include "oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { const float *scale, *bias, *mean, *var; } bev_bn;

struct bf_bev_stage {
    const float *fuser_w;
    bev_bn fuser_bn;
    const float *block_w[2][6];
    bev_bn block_bn[2][6];
    const float *deblock_w[2];
    bev_bn deblock_bn[2];
    const float *shared_w, *shared_b;
    const float *mid_w;
    bev_bn mid_bn;
    const float *out_w, *out_b;
};

static int bind_bev_bn(const bf_model *m, const char *prefix, size_t c, bev_bn *bn, char *e,
                       size_t cap) {
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

static const float *bind_w(const bf_model *m, const char *name, uint32_t d0, uint32_t d1,
                           uint32_t k, char *e, size_t cap) {
    const uint32_t dims[4] = {d0, d1, k, k};
    return (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, 4, dims, e, cap);
}

static const float *bind_b(const bf_model *m, const char *name, uint32_t c, char *e, size_t cap) {
    const uint32_t dims[1] = {c};
    return (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, 1, dims, e, cap);
}

/* bev_stage.c:84-131; layer indices of the SECOND blocks are the
 * nn.Sequential positions of conv (1, 4, ..., 16) and BN (2, 5, ..., 17). */
int bf_bev_stage_create(const bf_model *model, bf_bev_stage **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid BEV stage arguments");
    bf_bev_stage *s = calloc(1, sizeof(*s));
    if (!s) return bf_oracle_fail(error, cap, "BEV stage allocation failed");
    char name[160];
    s->fuser_w = bind_w(model, "fuser.conv.0.weight", 256, 336, 3, error, cap);
    if (!s->fuser_w || !bind_bev_bn(model, "fuser.conv.1", 256, &s->fuser_bn, error, cap))
        goto fail;
    for (int b = 0; b < 2; ++b) {
        const uint32_t ch = b ? 256 : 128, first = b ? 128 : 256;
        for (int l = 0; l < 6; ++l) {
            snprintf(name, sizeof(name), "backbone_2d.blocks.%d.%d.weight", b, 3 * l + 1);
            s->block_w[b][l] = bind_w(model, name, ch, l ? ch : first, 3, error, cap);
            if (!s->block_w[b][l]) goto fail;
            snprintf(name, sizeof(name), "backbone_2d.blocks.%d.%d", b, 3 * l + 2);
            if (!bind_bev_bn(model, name, ch, &s->block_bn[b][l], error, cap)) goto fail;
        }
    }
    s->deblock_w[0] = bind_w(model, "backbone_2d.deblocks.0.0.weight", 256, 128, 1, error, cap);
    /* ConvTranspose2d weights are [in, out, kH, kW]. */
    s->deblock_w[1] = bind_w(model, "backbone_2d.deblocks.1.0.weight", 256, 256, 2, error, cap);
    if (!s->deblock_w[0] || !s->deblock_w[1] ||
        !bind_bev_bn(model, "backbone_2d.deblocks.0.1", 256, &s->deblock_bn[0], error, cap) ||
        !bind_bev_bn(model, "backbone_2d.deblocks.1.1", 256, &s->deblock_bn[1], error, cap))
        goto fail;
    s->shared_w = bind_w(model, "dense_head.shared_conv.weight", 128, 512, 3, error, cap);
    s->shared_b = bind_b(model, "dense_head.shared_conv.bias", 128, error, cap);
    s->mid_w = bind_w(model, "dense_head.heatmap_head.0.conv.weight", 128, 128, 3, error, cap);
    if (!s->shared_w || !s->shared_b || !s->mid_w ||
        !bind_bev_bn(model, "dense_head.heatmap_head.0.bn", 128, &s->mid_bn, error, cap))
        goto fail;
    s->out_w = bind_w(model, "dense_head.heatmap_head.1.weight", 10, 128, 3, error, cap);
    s->out_b = bind_b(model, "dense_head.heatmap_head.1.bias", 10, error, cap);
    if (!s->out_w || !s->out_b) goto fail;
    *out = s;
    return 1;
fail:
    free(s);
    return 0;
}

void bf_bev_stage_destroy(bf_bev_stage *s) { free(s); }

/* bev_stage.c:135-140: two 256-channel full-resolution maps. */
size_t bf_bev_stage_workspace_bytes(size_t h, size_t w) {
    size_t hw, bytes;
    if (!h || !w || !bf_oracle_mul(h, w, &hw) || !bf_oracle_mul(hw, 2 * 256 * sizeof(float), &bytes))
        return 0;
    return bytes;
}

/* 3x3 (or caller-sized) convolution with unit dilation and one group
 * (bev_stage.c:142-148). */
static int bev_conv(const float *in, const float *w, const float *b, float *out, size_t ci,
                    size_t co, size_t k, size_t h, size_t wd, size_t stride, size_t pad) {
    const bf_conv2d_desc d = {1, ci, h, wd, co, k, k, stride, stride, pad, pad, 1, 1, 1};
    return bf_conv2d_f32(in, w, b, out, &d);
}

static void bev_bn_relu(float *v, const bev_bn *bn, size_t c, size_t h, size_t w) {
    bf_batch_norm_2d_f32(v, bn->scale, bn->bias, bn->mean, bn->var, 1e-3f, v, 1, c, h, w);
    bf_relu_f32(v, v, c * h * w);
}

/* bev_stage.c:157-227 */
int bf_bev_stage_forward_ref(const bf_bev_stage *s, const float *input, size_t batches,
                             size_t h, size_t w, float *spatial, float *shared, float *heatmap,
                             void *workspace, size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_bev_stage_workspace_bytes(h, w);
    if (!s || !input || !batches || !h || !w || (h & 1) || (w & 1) || !spatial || !shared ||
        !heatmap || !workspace || !need || workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid BEV stage buffers or dimensions");
    const size_t hw = h * w, hh = h / 2, hw2 = w / 2;
    float *buf_a = (float *)workspace, *buf_b = buf_a + 256 * hw;
    for (size_t n = 0; n < batches; ++n) {
        const float *x = input + n * 336 * hw;
        float *sp = spatial + n * 512 * hw, *sh = shared + n * 128 * hw;
        float *hm = heatmap + n * 10 * hw;
        if (!bev_conv(x, s->fuser_w, NULL, buf_a, 336, 256, 3, h, w, 1, 1))
            return bf_oracle_fail(error, cap, "fuser convolution failed");
        bev_bn_relu(buf_a, &s->fuser_bn, 256, h, w);
        const float *cur = buf_a;
        float *next = buf_b;
        for (int l = 0; l < 6; ++l) {
            if (!bev_conv(cur, s->block_w[0][l], NULL, next, l ? 128 : 256, 128, 3, h, w, 1, 1))
                return bf_oracle_fail(error, cap, "BEV block 0 convolution %d failed", l);
            bev_bn_relu(next, &s->block_bn[0][l], 128, h, w);
            cur = next;
            next = next == buf_a ? buf_b : buf_a;
        }
        if (!bev_conv(cur, s->deblock_w[0], NULL, sp, 128, 256, 1, h, w, 1, 0))
            return bf_oracle_fail(error, cap, "BEV deblock 0 failed");
        bev_bn_relu(sp, &s->deblock_bn[0], 256, h, w);
        next = cur == buf_a ? buf_b : buf_a;
        for (int l = 0; l < 6; ++l) {
            if (!bev_conv(cur, s->block_w[1][l], NULL, next, l ? 256 : 128, 256, 3, l ? hh : h,
                          l ? hw2 : w, l ? 1 : 2, 1))
                return bf_oracle_fail(error, cap, "BEV block 1 convolution %d failed", l);
            bev_bn_relu(next, &s->block_bn[1][l], 256, hh, hw2);
            cur = next;
            next = next == buf_a ? buf_b : buf_a;
        }
        const bf_conv_transpose2d_desc up = {1, 256, hh, hw2, 256, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 1};
        if (!bf_conv_transpose2d_f32_ref(cur, s->deblock_w[1], NULL, sp + 256 * hw, &up))
            return bf_oracle_fail(error, cap, "BEV deblock 1 failed");
        bev_bn_relu(sp + 256 * hw, &s->deblock_bn[1], 256, h, w);
        if (!bev_conv(sp, s->shared_w, s->shared_b, sh, 512, 128, 3, h, w, 1, 1))
            return bf_oracle_fail(error, cap, "TransFusion shared convolution failed");
        if (!bev_conv(sh, s->mid_w, NULL, buf_a, 128, 128, 3, h, w, 1, 1))
            return bf_oracle_fail(error, cap, "TransFusion heatmap middle convolution failed");
        bev_bn_relu(buf_a, &s->mid_bn, 128, h, w);
        if (!bev_conv(buf_a, s->out_w, s->out_b, hm, 128, 10, 3, h, w, 1, 1))
            return bf_oracle_fail(error, cap, "TransFusion heatmap output convolution failed");
    }
    return 1;
}
