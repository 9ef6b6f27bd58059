/*
 * Oracle Swin-T image backbone: restates reference src/swin_backbone.c:11-352.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Graph: 4x4/s4 patch conv 3->96 (scalar), LN; stages of (2,2,6,2) blocks at
 * C=(96,192,384,768), heads=(3,6,12,24), window 7, shift 3 on odd blocks;
 * after stages 1..3 an output LN stored NHWC->NCHW; between stages a 2x2
 * patch merge in nn.Unfold order (element c*4 + ky*2 + kx, zero past odd
 * edges) -> LN(4C) -> bias-free reduction to 2C.
 */
#include "oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const size_t kC[4] = {96, 192, 384, 768};
static const size_t kHeads[4] = {3, 6, 12, 24};
static const size_t kDepth[4] = {2, 2, 6, 2};

typedef struct {
    const float *n1s, *n1b, *rel_bias;
    const int64_t *rel_index;
    const float *qkv_w, *qkv_b, *proj_w, *proj_b;
    const float *n2s, *n2b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} swin_block;

struct bf_swin_backbone {
    const float *patch_w, *patch_b, *patch_ns, *patch_nb;
    swin_block blocks[4][6];
    const float *merge_s[3], *merge_b[3], *merge_w[3];
    const float *out_s[3], *out_b[3];
};

static const float *bind_f(const bf_model *m, const char *name, uint32_t rank,
                           const uint32_t *dims, char *e, size_t cap) {
    return (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, rank, dims, e, cap);
}

/* swin_backbone.c:107-188: bind every tensor, checking dtype/rank/dims. */
int bf_swin_backbone_create(const bf_model *model, bf_swin_backbone **out,
                            char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid Swin backbone arguments");
    bf_swin_backbone *net = calloc(1, sizeof(*net));
    if (!net) return bf_oracle_fail(error, cap, "Swin backbone allocation failed");
    char name[192];
    const uint32_t pd[4] = {96, 3, 4, 4}, d96[1] = {96};
    net->patch_w = bind_f(model, "image_backbone.patch_embed.projection.weight", 4, pd, error, cap);
    net->patch_b = bind_f(model, "image_backbone.patch_embed.projection.bias", 1, d96, error, cap);
    net->patch_ns = bind_f(model, "image_backbone.patch_embed.norm.weight", 1, d96, error, cap);
    net->patch_nb = bind_f(model, "image_backbone.patch_embed.norm.bias", 1, d96, error, cap);
    if (!net->patch_w || !net->patch_b || !net->patch_ns || !net->patch_nb) goto fail;
    for (size_t s = 0; s < 4; ++s) {
        const uint32_t c = (uint32_t)kC[s], h = (uint32_t)kHeads[s];
        const uint32_t dc[1] = {c}, d3c[1] = {3 * c}, d4c[1] = {4 * c};
        const uint32_t qkv[2] = {3 * c, c}, sq[2] = {c, c}, rel[2] = {169, h};
        const uint32_t idx[2] = {49, 49}, f1[2] = {4 * c, c}, f2[2] = {c, 4 * c};
        for (size_t b = 0; b < kDepth[s]; ++b) {
            swin_block *k = &net->blocks[s][b];
#define BIND(field, suffix, rank, dims)                                                  \
    do {                                                                                 \
        snprintf(name, sizeof(name), "image_backbone.stages.%zu.blocks.%zu.%s", s, b, suffix); \
        k->field = bind_f(model, name, rank, dims, error, cap);                          \
        if (!k->field) goto fail;                                                        \
    } while (0)
            BIND(n1s, "norm1.weight", 1, dc);
            BIND(n1b, "norm1.bias", 1, dc);
            BIND(rel_bias, "attn.w_msa.relative_position_bias_table", 2, rel);
            snprintf(name, sizeof(name),
                     "image_backbone.stages.%zu.blocks.%zu.attn.w_msa.relative_position_index", s, b);
            k->rel_index = (const int64_t *)bf_oracle_bind(model, name, BF_DTYPE_I64, 2, idx,
                                                           error, cap);
            if (!k->rel_index) goto fail;
            BIND(qkv_w, "attn.w_msa.qkv.weight", 2, qkv);
            BIND(qkv_b, "attn.w_msa.qkv.bias", 1, d3c);
            BIND(proj_w, "attn.w_msa.proj.weight", 2, sq);
            BIND(proj_b, "attn.w_msa.proj.bias", 1, dc);
            BIND(n2s, "norm2.weight", 1, dc);
            BIND(n2b, "norm2.bias", 1, dc);
            BIND(fc1_w, "ffn.layers.0.0.weight", 2, f1);
            BIND(fc1_b, "ffn.layers.0.0.bias", 1, d4c);
            BIND(fc2_w, "ffn.layers.1.weight", 2, f2);
            BIND(fc2_b, "ffn.layers.1.bias", 1, dc);
#undef BIND
        }
        if (s < 3) {
            const uint32_t red[2] = {2 * c, 4 * c};
            snprintf(name, sizeof(name), "image_backbone.stages.%zu.downsample.norm.weight", s);
            net->merge_s[s] = bind_f(model, name, 1, d4c, error, cap);
            snprintf(name, sizeof(name), "image_backbone.stages.%zu.downsample.norm.bias", s);
            net->merge_b[s] = bind_f(model, name, 1, d4c, error, cap);
            snprintf(name, sizeof(name), "image_backbone.stages.%zu.downsample.reduction.weight", s);
            net->merge_w[s] = bind_f(model, name, 2, red, error, cap);
            if (!net->merge_s[s] || !net->merge_b[s] || !net->merge_w[s]) goto fail;
        }
    }
    for (size_t o = 0; o < 3; ++o) {
        const uint32_t dc[1] = {(uint32_t)kC[o + 1]};
        snprintf(name, sizeof(name), "image_backbone.norm%zu.weight", o + 1);
        net->out_s[o] = bind_f(model, name, 1, dc, error, cap);
        snprintf(name, sizeof(name), "image_backbone.norm%zu.bias", o + 1);
        net->out_b[o] = bind_f(model, name, 1, dc, error, cap);
        if (!net->out_s[o] || !net->out_b[o]) goto fail;
    }
    *out = net;
    return 1;
fail:
    free(net);
    return 0;
}

void bf_swin_backbone_destroy(bf_swin_backbone *net) { free(net); }

/* swin_backbone.c:192-203 */
int bf_swin_backbone_output_shapes(size_t ih, size_t iw, bf_swin_backbone_shapes *s) {
    if (!ih || !iw || !s || ih > SIZE_MAX - 31 || iw > SIZE_MAX - 31) return 0;
    for (size_t i = 0; i < 3; ++i) {
        const size_t div = (size_t)8 << i;
        s->height[i] = (ih + div - 1) / div;
        s->width[i] = (iw + div - 1) / div;
        s->channels[i] = kC[i + 1];
    }
    return 1;
}

/* swin_backbone.c:205-216: 6 stage-0 token buffers + one window workspace
 * sized for the largest block (C=768, 24 heads). */
size_t bf_swin_backbone_workspace_bytes(size_t batches, size_t ih, size_t iw) {
    if (!batches || !ih || !iw || ih > SIZE_MAX - 3 || iw > SIZE_MAX - 3) return 0;
    size_t v;
    if (!bf_oracle_mul(batches, (ih + 3) / 4, &v) || !bf_oracle_mul(v, (iw + 3) / 4, &v) ||
        !bf_oracle_mul(v, 96, &v) || !bf_oracle_mul(v, 6, &v) ||
        !bf_oracle_mul(v, sizeof(float), &v))
        return 0;
    const bf_swin_window_desc largest = {1, 1, 1, 768, 24, 7, 3};
    const size_t attn = bf_swin_shifted_window_workspace_bytes(&largest);
    return attn && v <= SIZE_MAX - attn ? v + attn : 0;
}

/* swin_backbone.c:218-237: scalar 4x4/s4 patch conv, NHWC output. */
static void patch_embed(const bf_swin_backbone *net, const float *in, float *out,
                        size_t batches, size_t ih, size_t iw, size_t oh, size_t ow) {
    for (size_t b = 0; b < batches; ++b)
        for (size_t y = 0; y < oh; ++y)
            for (size_t x = 0; x < ow; ++x)
                for (size_t co = 0; co < 96; ++co) {
                    float acc = net->patch_b[co];
                    for (size_t ci = 0; ci < 3; ++ci)
                        for (size_t ky = 0; ky < 4; ++ky)
                            for (size_t kx = 0; kx < 4; ++kx) {
                                const size_t sy = 4 * y + ky, sx = 4 * x + kx;
                                if (sy < ih && sx < iw)
                                    acc += in[((b * 3 + ci) * ih + sy) * iw + sx] *
                                           net->patch_w[((co * 3 + ci) * 4 + ky) * 4 + kx];
                            }
                    out[((b * oh + y) * ow + x) * 96 + co] = acc;
                }
}

/* swin_backbone.c:239-263: x += W-MSA(LN1 x); x += MLP(LN2 x). */
static int run_block(const swin_block *k, float *x, float *normal, float *hidden,
                     size_t batches, size_t h, size_t w, size_t c, size_t heads,
                     size_t shift, void *ws, size_t ws_bytes) {
    const size_t rows = batches * h * w, count = rows * c;
    bf_layer_norm_f32(x, k->n1s, k->n1b, 1e-5f, normal, rows, c);
    const bf_swin_window_desc d = {batches, h, w, c, heads, 7, shift};
    if (!bf_swin_shifted_window_f32_workspace_ref(normal, k->qkv_w, k->qkv_b, k->rel_bias,
                                                  k->rel_index, k->proj_w, k->proj_b,
                                                  hidden, &d, ws, ws_bytes))
        return 0;
    for (size_t i = 0; i < count; ++i) x[i] += hidden[i];
    bf_layer_norm_f32(x, k->n2s, k->n2b, 1e-5f, normal, rows, c);
    bf_linear_f32(normal, k->fc1_w, k->fc1_b, hidden, rows, c, 4 * c);
    bf_gelu_f32(hidden, hidden, rows * 4 * c);
    bf_linear_f32(hidden, k->fc2_w, k->fc2_b, normal, rows, 4 * c, c);
    for (size_t i = 0; i < count; ++i) x[i] += normal[i];
    return 1;
}

/* swin_backbone.c:265-276 */
static void store_output(const float *x, float *out, const float *s, const float *b,
                         float *normal, size_t batches, size_t h, size_t w, size_t c) {
    const size_t hw = h * w;
    bf_layer_norm_f32(x, s, b, 1e-5f, normal, batches * hw, c);
    for (size_t n = 0; n < batches; ++n)
        for (size_t ch = 0; ch < c; ++ch)
            for (size_t p = 0; p < hw; ++p)
                out[(n * c + ch) * hw + p] = normal[(n * hw + p) * c + ch];
}

/* swin_backbone.c:278-302 */
static void patch_merge(const float *ms, const float *mb, const float *mw,
                        const float *x, float *unfolded, float *out,
                        size_t batches, size_t h, size_t w, size_t c) {
    const size_t oh = (h + 1) / 2, ow = (w + 1) / 2, rows = batches * oh * ow;
    for (size_t n = 0; n < batches; ++n)
        for (size_t y = 0; y < oh; ++y)
            for (size_t xx = 0; xx < ow; ++xx) {
                float *row = unfolded + ((n * oh + y) * ow + xx) * 4 * c;
                for (size_t ch = 0; ch < c; ++ch)
                    for (size_t q = 0; q < 4; ++q) {
                        const size_t sy = 2 * y + q / 2, sx = 2 * xx + q % 2;
                        row[ch * 4 + q] = sy < h && sx < w ? x[((n * h + sy) * w + sx) * c + ch] : 0.0f;
                    }
            }
    bf_layer_norm_f32(unfolded, ms, mb, 1e-5f, unfolded, rows, 4 * c);
    bf_linear_f32(unfolded, mw, NULL, out, rows, 4 * c, 2 * c);
}

/* swin_backbone.c:304-352 */
int bf_swin_backbone_forward_ref(const bf_swin_backbone *net, const float *input,
                                 size_t batches, size_t ih, size_t iw, float *out1,
                                 float *out2, float *out3, void *workspace,
                                 size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_swin_backbone_workspace_bytes(batches, ih, iw);
    if (!net || !input || !batches || !ih || !iw || !out1 || !out2 || !out3 ||
        !workspace || !need || workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid Swin backbone buffers or dimensions");
    size_t h = (ih + 3) / 4, w = (iw + 3) / 4, tokens;
    if (!bf_oracle_mul(h, w, &tokens) || !bf_oracle_mul(batches, tokens, &tokens) ||
        !bf_oracle_mul(tokens, 96, &tokens))
        return bf_oracle_fail(error, cap, "Swin backbone shape overflow");
    float *a = (float *)workspace, *b = a + tokens, *hidden = b + tokens;
    void *ws = a + 6 * tokens;
    const size_t ws_bytes = need - 6 * tokens * sizeof(float);
    patch_embed(net, input, a, batches, ih, iw, h, w);
    bf_layer_norm_f32(a, net->patch_ns, net->patch_nb, 1e-5f, a, batches * h * w, 96);
    float *x = a, *other = b, *outs[3] = {out1, out2, out3};
    for (size_t s = 0; s < 4; ++s) {
        for (size_t k = 0; k < kDepth[s]; ++k)
            if (!run_block(&net->blocks[s][k], x, other, hidden, batches, h, w, kC[s],
                           kHeads[s], (k & 1) ? 3 : 0, ws, ws_bytes))
                return bf_oracle_fail(error, cap, "Swin stage %zu block %zu failed", s, k);
        if (s > 0)
            store_output(x, outs[s - 1], net->out_s[s - 1], net->out_b[s - 1], other,
                         batches, h, w, kC[s]);
        if (s < 3) {
            patch_merge(net->merge_s[s], net->merge_b[s], net->merge_w[s], x, hidden, other,
                        batches, h, w, kC[s]);
            float *t = x;
            x = other;
            other = t;
            h = (h + 1) / 2;
            w = (w + 1) / 2;
        }
    }
    return 1;
}
