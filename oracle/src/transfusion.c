/*
 * Oracle TransFusion head: restates reference src/transfusion.c:8-193
 * (heatmap NMS + top-k proposals, raw-output decoding, detection filtering)
 * and src/transfusion_decoder.c:23-456 (query initialisation, position
 * embeddings, self and cross multi-head attention, FFN, LayerNorms and the
 * six prediction heads).  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Per-element floating-point operation order follows the reference, so the
 * scalar build is bit-identical to the reference's C compiled here.  The
 * top-k differs in method only: every candidate is ordered by (score
 * descending, flat index ascending), a total order, so any exact selection
 * returns the reference heap's result.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#if defined(BF_WITH_OPENMP)
#include <omp.h>
#endif

#define TF_C 128u
#define TF_HEADS 8u
#define TF_HEAD_C (TF_C / TF_HEADS)
#define TF_SLOTS 16u

/* Two-branch logistic (transfusion.c:8-16). */
static float tf_sigmoid(float v) {
    if (v >= 0.0f) {
        const float e = expf(-v);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(v);
    return e / (1.0f + e);
}

typedef struct {
    float score;
    size_t flat;
} tf_candidate;

/* Higher score first; equal scores by smaller flat index (transfusion.c:24-32). */
static int tf_order(const void *l, const void *r) {
    const tf_candidate *a = l, *b = r;
    if (a->score != b->score) return a->score > b->score ? -1 : 1;
    return (a->flat > b->flat) - (a->flat < b->flat);
}

/* transfusion.c:75-132 */
int bf_transfusion_select_proposals_f32_ref(const float *logits, float *suppressed,
                                            float *top_scores, int64_t *top_classes,
                                            int64_t *top_indices, size_t batches,
                                            size_t classes, size_t height, size_t width,
                                            size_t proposals, size_t kernel) {
    if (!logits || !suppressed || !top_scores || !top_classes || !top_indices || !batches ||
        !classes || !height || !width || !proposals || proposals > BF_MAX_PROPOSALS ||
        proposals > classes * height * width || !kernel || !(kernel & 1))
        return 0;
    const size_t spatial = height * width, pad = kernel / 2, n = classes * spatial;
    tf_candidate *all = malloc(n * sizeof(*all));
    if (!all) return 0;
    for (size_t b = 0; b < batches; ++b) {
        for (size_t cls = 0; cls < classes; ++cls) {
            const int bypass = classes == 10 && (cls == 8 || cls == 9);
            const float *plane = logits + (b * classes + cls) * spatial;
            float *out = suppressed + (b * classes + cls) * spatial;
            for (size_t y = 0; y < height; ++y)
                for (size_t x = 0; x < width; ++x) {
                    const float v = tf_sigmoid(plane[y * width + x]);
                    int keep = bypass;
                    if (!bypass && y >= pad && x >= pad && y + pad < height && x + pad < width) {
                        float m = -FLT_MAX;
                        for (size_t ky = 0; ky < kernel; ++ky)
                            for (size_t kx = 0; kx < kernel; ++kx) {
                                const float q =
                                    tf_sigmoid(plane[(y + ky - pad) * width + x + kx - pad]);
                                if (q > m) m = q;
                            }
                        keep = v == m;
                    }
                    out[y * width + x] = keep ? v : 0.0f;
                }
        }
        for (size_t f = 0; f < n; ++f) {
            all[f].score = suppressed[b * n + f];
            all[f].flat = f;
        }
        qsort(all, n, sizeof(*all), tf_order);
        for (size_t r = 0; r < proposals; ++r) {
            top_scores[b * proposals + r] = all[r].score;
            top_classes[b * proposals + r] = (int64_t)(all[r].flat / spatial);
            top_indices[b * proposals + r] = (int64_t)(all[r].flat % spatial);
        }
    }
    free(all);
    return 1;
}

/* transfusion.c:134-167 */
int bf_transfusion_decode_raw_f32_ref(const float *heatmap, const float *query_scores,
                                      const int64_t *query_labels, const float *center,
                                      const float *height, const float *dimension_log,
                                      const float *rotation, const float *velocity, float *boxes,
                                      float *scores, int64_t *labels, size_t batches,
                                      size_t classes, size_t proposals, float feature_stride,
                                      const float voxel_size[2], const float minimum[2]) {
    if (!heatmap || !query_scores || !query_labels || !center || !height || !dimension_log ||
        !rotation || !boxes || !scores || !labels || !batches || !classes || !proposals ||
        !isfinite(feature_stride) || feature_stride <= 0.0f || !voxel_size || !minimum ||
        voxel_size[0] <= 0.0f || voxel_size[1] <= 0.0f)
        return 0;
    for (size_t b = 0; b < batches; ++b)
        for (size_t p = 0; p < proposals; ++p) {
            const int64_t cls = query_labels[b * proposals + p];
            if (cls < 0 || (uint64_t)cls >= classes) return 0;
            const size_t co = (b * classes + (size_t)cls) * proposals + p;
            scores[b * proposals + p] = tf_sigmoid(heatmap[co]) * query_scores[co];
            labels[b * proposals + p] = cls;
            float *box = boxes + (b * proposals + p) * 9;
            box[0] = center[(b * 2) * proposals + p] * feature_stride * voxel_size[0] + minimum[0];
            box[1] = center[(b * 2 + 1) * proposals + p] * feature_stride * voxel_size[1] +
                     minimum[1];
            box[2] = height[b * proposals + p];
            for (size_t a = 0; a < 3; ++a) box[3 + a] = expf(dimension_log[(b * 3 + a) * proposals + p]);
            box[6] = atan2f(rotation[(b * 2) * proposals + p], rotation[(b * 2 + 1) * proposals + p]);
            box[7] = velocity ? velocity[(b * 2) * proposals + p] : 0.0f;
            box[8] = velocity ? velocity[(b * 2 + 1) * proposals + p] : 0.0f;
        }
    return 1;
}

/* transfusion.c:169-193 */
int bf_transfusion_filter_detections(const float *boxes, const float *scores,
                                     const int64_t *labels, size_t batches, size_t proposals,
                                     float threshold, const float range[6],
                                     bf_detections *output) {
    if (!boxes || !scores || !labels || !batches || !proposals || proposals > BF_MAX_PROPOSALS ||
        !isfinite(threshold) || !range || !output)
        return 0;
    for (size_t b = 0; b < batches; ++b) {
        output[b].count = 0;
        for (size_t p = 0; p < proposals; ++p) {
            const float *box = boxes + (b * proposals + p) * 9;
            const float score = scores[b * proposals + p];
            int keep = isfinite(score) && score > threshold;
            for (size_t a = 0; a < 3; ++a)
                keep &= isfinite(box[a]) && box[a] >= range[a] && box[a] <= range[a + 3];
            if (!keep) continue;
            bf_detection *d = &output[b].items[output[b].count++];
            d->x = box[0]; d->y = box[1]; d->z = box[2];
            d->width = box[3]; d->length = box[4]; d->height = box[5];
            d->yaw = box[6]; d->velocity_x = box[7]; d->velocity_y = box[8];
            d->score = score;
            d->class_id = (int)labels[b * proposals + p];
        }
    }
    return 1;
}

/* ======================= decoder (transfusion_decoder.c) ================= */
typedef struct { const float *scale, *bias, *mean, *var; } tf_bn;
typedef struct {
    const float *w1, *b1;
    tf_bn bn;
    const float *w2, *b2;
} tf_position;
typedef struct {
    const float *hidden_w;
    tf_bn bn;
    const float *out_w, *out_b;
    size_t channels;
} tf_head;

struct bf_transfusion_decoder {
    const float *class_w, *class_b;
    const float *self_in_w, *self_in_b, *self_out_w, *self_out_b;
    const float *cross_in_w, *cross_in_b, *cross_out_w, *cross_out_b;
    const float *lin1_w, *lin1_b, *lin2_w, *lin2_b;
    const float *norm_w[3], *norm_b[3];
    tf_position self_pos, cross_pos;
    tf_head heads[6];
};

static const float *tf_bind(const bf_model *m, const char *name, uint32_t rank, uint32_t d0,
                            uint32_t d1, uint32_t d2, char *e, size_t cap) {
    const uint32_t dims[3] = {d0, d1, d2};
    return (const float *)bf_oracle_bind(m, name, BF_DTYPE_F32, rank, dims, e, cap);
}

static int tf_bind_bn(const bf_model *m, const char *prefix, uint32_t c, tf_bn *bn, char *e,
                      size_t cap) {
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float **slot[4] = {&bn->scale, &bn->bias, &bn->mean, &bn->var};
    char name[192];
    for (int i = 0; i < 4; ++i) {
        snprintf(name, sizeof(name), "%s.%s", prefix, suffix[i]);
        if (!(*slot[i] = tf_bind(m, name, 1, c, 0, 0, e, cap))) return 0;
    }
    return 1;
}

/* transfusion_decoder.c:121-139 */
static int tf_bind_position(const bf_model *m, const char *base, tf_position *p, char *e,
                            size_t cap) {
    char name[192];
    snprintf(name, sizeof(name), "%s.position_embedding_head.0.weight", base);
    p->w1 = tf_bind(m, name, 3, TF_C, 2, 1, e, cap);
    snprintf(name, sizeof(name), "%s.position_embedding_head.0.bias", base);
    p->b1 = tf_bind(m, name, 1, TF_C, 0, 0, e, cap);
    if (!p->w1 || !p->b1) return 0;
    snprintf(name, sizeof(name), "%s.position_embedding_head.1", base);
    if (!tf_bind_bn(m, name, TF_C, &p->bn, e, cap)) return 0;
    snprintf(name, sizeof(name), "%s.position_embedding_head.3.weight", base);
    p->w2 = tf_bind(m, name, 3, TF_C, TF_C, 1, e, cap);
    snprintf(name, sizeof(name), "%s.position_embedding_head.3.bias", base);
    p->b2 = tf_bind(m, name, 1, TF_C, 0, 0, e, cap);
    return p->w2 && p->b2;
}

/* transfusion_decoder.c:141-163 */
static int tf_bind_head(const bf_model *m, const char *head, uint32_t channels, tf_head *h,
                        char *e, size_t cap) {
    char name[192];
    snprintf(name, sizeof(name), "dense_head.prediction_head.%s.0.0.weight", head);
    h->hidden_w = tf_bind(m, name, 3, 64, TF_C, 1, e, cap);
    if (!h->hidden_w) return 0;
    snprintf(name, sizeof(name), "dense_head.prediction_head.%s.0.1", head);
    if (!tf_bind_bn(m, name, 64, &h->bn, e, cap)) return 0;
    snprintf(name, sizeof(name), "dense_head.prediction_head.%s.1.weight", head);
    h->out_w = tf_bind(m, name, 3, channels, 64, 1, e, cap);
    snprintf(name, sizeof(name), "dense_head.prediction_head.%s.1.bias", head);
    h->out_b = tf_bind(m, name, 1, channels, 0, 0, e, cap);
    h->channels = channels;
    return h->out_w && h->out_b;
}

/* transfusion_decoder.c:165-208 */
int bf_transfusion_decoder_create(const bf_model *model, bf_transfusion_decoder **out,
                                  char *error, size_t cap) {
    if (out) *out = NULL;
    if (!model || !out) return bf_oracle_fail(error, cap, "invalid TransFusion arguments");
    bf_transfusion_decoder *d = calloc(1, sizeof(*d));
    if (!d) return bf_oracle_fail(error, cap, "TransFusion allocation failed");
    const char *p = "dense_head.decoder.";
    char n[192];
#define TFB(field, rank, a, b, c, fmt, ...)                        \
    do {                                                          \
        snprintf(n, sizeof(n), fmt, __VA_ARGS__);                 \
        if (!(d->field = tf_bind(model, n, rank, a, b, c, error, cap))) goto fail; \
    } while (0)
    TFB(class_w, 3, TF_C, 10, 1, "%s", "dense_head.class_encoding.weight");
    TFB(class_b, 1, TF_C, 0, 0, "%s", "dense_head.class_encoding.bias");
    TFB(self_in_w, 2, 3 * TF_C, TF_C, 0, "%sself_attn.in_proj_weight", p);
    TFB(self_in_b, 1, 3 * TF_C, 0, 0, "%sself_attn.in_proj_bias", p);
    TFB(self_out_w, 2, TF_C, TF_C, 0, "%sself_attn.out_proj.weight", p);
    TFB(self_out_b, 1, TF_C, 0, 0, "%sself_attn.out_proj.bias", p);
    TFB(cross_in_w, 2, 3 * TF_C, TF_C, 0, "%smultihead_attn.in_proj_weight", p);
    TFB(cross_in_b, 1, 3 * TF_C, 0, 0, "%smultihead_attn.in_proj_bias", p);
    TFB(cross_out_w, 2, TF_C, TF_C, 0, "%smultihead_attn.out_proj.weight", p);
    TFB(cross_out_b, 1, TF_C, 0, 0, "%smultihead_attn.out_proj.bias", p);
    TFB(lin1_w, 2, 256, TF_C, 0, "%slinear1.weight", p);
    TFB(lin1_b, 1, 256, 0, 0, "%slinear1.bias", p);
    TFB(lin2_w, 2, TF_C, 256, 0, "%slinear2.weight", p);
    TFB(lin2_b, 1, TF_C, 0, 0, "%slinear2.bias", p);
    for (int i = 0; i < 3; ++i) {
        TFB(norm_w[i], 1, TF_C, 0, 0, "%snorm%d.weight", p, i + 1);
        TFB(norm_b[i], 1, TF_C, 0, 0, "%snorm%d.bias", p, i + 1);
    }
#undef TFB
    if (!tf_bind_position(model, "dense_head.decoder.self_posembed", &d->self_pos, error, cap) ||
        !tf_bind_position(model, "dense_head.decoder.cross_posembed", &d->cross_pos, error, cap))
        goto fail;
    static const char *names[6] = {"center", "height", "dim", "rot", "vel", "heatmap"};
    static const uint32_t channels[6] = {2, 1, 3, 2, 2, 10};
    for (int i = 0; i < 6; ++i)
        if (!tf_bind_head(model, names[i], channels[i], &d->heads[i], error, cap)) goto fail;
    *out = d;
    return 1;
fail:
    free(d);
    return 0;
}

void bf_transfusion_decoder_destroy(bf_transfusion_decoder *d) { free(d); }

/* transfusion_decoder.c:212-224, with one deliberate difference: the
 * projection and score-slot regions hold max(keys, proposals) rows.  The
 * reference sizes them by keys alone (transfusion_decoder.c:219, 354-357),
 * but self attention also runs its P-row K/V projections and P-wide score
 * rows through them, so for proposals > H * W (allowed by its contract,
 * proposals <= 10 * H * W) its self attention overruns into the suppressed
 * map and the query rows.  For proposals <= H * W both layouts give the same
 * results. */
size_t bf_transfusion_decoder_workspace_bytes(size_t height, size_t width, size_t proposals) {
    size_t keys, rows, key_floats, row_floats, proposal_floats, bytes;
    if (!height || !width || !proposals || proposals > 200 || !bf_oracle_mul(height, width, &keys) ||
        proposals > 10 * keys)
        return 0;
    rows = keys > proposals ? keys : proposals;
    if (!bf_oracle_mul(keys, TF_C + 10, &key_floats) ||
        !bf_oracle_mul(rows, 2 * TF_C + TF_SLOTS, &row_floats) ||
        key_floats > SIZE_MAX - row_floats ||
        !bf_oracle_mul(proposals, 8 * TF_C + 1, &proposal_floats) ||
        key_floats + row_floats > SIZE_MAX - proposal_floats ||
        !bf_oracle_mul(key_floats + row_floats + proposal_floats, sizeof(float), &bytes))
        return 0;
    return bytes;
}

/* transfusion_decoder.c:226-234: eval BatchNorm (epsilon 1e-5) + ReLU per row. */
static void tf_bn_relu(float *v, size_t rows, size_t c, const tf_bn *bn) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < c; ++i) {
            const float f = bn->scale[i] / sqrtf(bn->var[i] + 1e-5f);
            const float y = (v[r * c + i] - bn->mean[i]) * f + bn->bias[i];
            v[r * c + i] = y > 0.0f ? y : 0.0f;
        }
}

/* transfusion_decoder.c:236-250: cell centre (x + 0.5, y + 0.5) -> 1x1 conv ->
 * BN + ReLU -> 1x1 conv. */
static void tf_position_embed(const tf_position *p, const int64_t *indices, size_t count,
                              size_t width, float *hidden, float *out) {
    for (size_t r = 0; r < count; ++r) {
        const size_t cell = indices ? (size_t)indices[r] : r;
        const float x = (float)(cell % width) + 0.5f, y = (float)(cell / width) + 0.5f;
        for (size_t c = 0; c < TF_C; ++c)
            hidden[r * TF_C + c] = p->b1[c] + p->w1[c * 2] * x + p->w1[c * 2 + 1] * y;
    }
    tf_bn_relu(hidden, count, TF_C, &p->bn);
    bf_linear_f32(hidden, p->w2, p->b2, out, count, TF_C, TF_C);
}

/* transfusion_decoder.c:259-313: nn.MultiheadAttention (8 heads of 16),
 * scores scaled by 1/sqrt(16), max-shifted softmax with a double sum. */
static void tf_attention(const float *query, size_t nq, const float *kv, size_t nk,
                         const float *in_w, const float *in_b, const float *out_w,
                         const float *out_b, float *qp, float *kp, float *vp, float *slots,
                         float *heads, float *out) {
    bf_linear_f32(query, in_w, in_b, qp, nq, TF_C, TF_C);
    bf_linear_f32(kv, in_w + TF_C * TF_C, in_b + TF_C, kp, nk, TF_C, TF_C);
    bf_linear_f32(kv, in_w + 2 * TF_C * TF_C, in_b + 2 * TF_C, vp, nk, TF_C, TF_C);
    const float scale = 1.0f / sqrtf((float)TF_HEAD_C);
#if defined(BF_WITH_OPENMP)
    int threads = omp_get_max_threads();
    if (threads > (int)TF_SLOTS) threads = (int)TF_SLOTS;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (size_t q = 0; q < nq; ++q) {
        size_t slot = 0;
#if defined(BF_WITH_OPENMP)
        slot = (size_t)omp_get_thread_num();
#endif
        float *s = slots + slot * nk;
        for (size_t c = 0; c < TF_C; ++c) heads[q * TF_C + c] = 0.0f;
        for (size_t h = 0; h < TF_HEADS; ++h) {
            float m = -FLT_MAX;
            for (size_t k = 0; k < nk; ++k) {
                float dot = 0.0f;
#if defined(BF_WITH_OPENMP)
#pragma omp simd reduction(+:dot)
#endif
                for (size_t l = 0; l < TF_HEAD_C; ++l)
                    dot += qp[q * TF_C + h * TF_HEAD_C + l] * kp[k * TF_C + h * TF_HEAD_C + l];
                dot *= scale;
                s[k] = dot;
                if (dot > m) m = dot;
            }
            double sum = 0.0;
            for (size_t k = 0; k < nk; ++k) {
                s[k] = expf(s[k] - m);
                sum += s[k];
            }
            const float inv = (float)(1.0 / sum);
            for (size_t k = 0; k < nk; ++k) {
                const float prob = s[k] * inv;
                for (size_t l = 0; l < TF_HEAD_C; ++l)
                    heads[q * TF_C + h * TF_HEAD_C + l] += prob * vp[k * TF_C + h * TF_HEAD_C + l];
            }
        }
    }
    bf_linear_f32(heads, out_w, out_b, out, nq, TF_C, TF_C);
}

/* transfusion_decoder.c:315-327: conv1d 128->64 (no bias) -> BN + ReLU ->
 * conv1d 64->C (+bias), stored channel-major [C][P]. */
static void tf_head_forward(const tf_head *h, const float *query, size_t np, float *hidden,
                            float *out) {
    bf_linear_f32(query, h->hidden_w, NULL, hidden, np, TF_C, 64);
    tf_bn_relu(hidden, np, 64, &h->bn);
    float *rows = hidden + np * 64;
    bf_linear_f32(hidden, h->out_w, h->out_b, rows, np, 64, h->channels);
    for (size_t p = 0; p < np; ++p)
        for (size_t c = 0; c < h->channels; ++c) out[c * np + p] = rows[p * h->channels + c];
}

static void tf_residual_norm(float *query, const float *update, const float *w, const float *b,
                             size_t np) {
    for (size_t i = 0; i < np * TF_C; ++i) query[i] += update[i];
    bf_layer_norm_f32(query, w, b, 1e-5f, query, np, TF_C);
}

/* transfusion_decoder.c:329-456 */
int bf_transfusion_decoder_forward_ref(const bf_transfusion_decoder *d, const float *shared,
                                       const float *dense_heatmap, size_t batches, size_t height,
                                       size_t width, size_t proposals,
                                       bf_transfusion_raw_outputs *out, void *workspace,
                                       size_t workspace_bytes, char *error, size_t cap) {
    const size_t need = bf_transfusion_decoder_workspace_bytes(height, width, proposals);
    if (!d || !shared || !dense_heatmap || !batches || !out || !out->center_b2p ||
        !out->height_b1p || !out->dimension_log_b3p || !out->rotation_sincos_b2p ||
        !out->velocity_b2p || !out->heatmap_logits_b10p || !out->query_heatmap_scores_b10p ||
        !out->query_labels_bp || !out->query_indices_bp || !workspace || !need ||
        workspace_bytes < need)
        return bf_oracle_fail(error, cap, "invalid TransFusion buffers or dimensions");
    const size_t keys = height * width, P = proposals;
    float *w = (float *)workspace;
    const size_t rows = keys > P ? keys : P;
    float *key_value = w; w += keys * TF_C;
    float *key_proj = w; w += rows * TF_C;
    float *value_proj = w; w += rows * TF_C;
    float *suppressed = w; w += keys * 10;
    float *slots = w; w += rows * TF_SLOTS;
    float *query = w; w += P * TF_C;
    float *query_pos = w; w += P * TF_C;
    float *tmp = w; w += P * TF_C;
    float *attn = w; w += P * TF_C;
    float *q_proj = w; w += P * TF_C;
    float *ffn = w; w += P * 256;
    float *head_hidden = w; w += P * TF_C;
    float *top_scores = w;
    for (size_t b = 0; b < batches; ++b) {
        const float *sh = shared + b * TF_C * keys;
        int64_t *labels = out->query_labels_bp + b * P, *indices = out->query_indices_bp + b * P;
        if (!bf_transfusion_select_proposals_f32_ref(dense_heatmap + b * 10 * keys, suppressed,
                                                     top_scores, labels, indices, 1, 10, height,
                                                     width, P, 3))
            return bf_oracle_fail(error, cap, "TransFusion proposal selection failed");
        for (size_t p = 0; p < P; ++p) {
            const size_t idx = (size_t)indices[p], cls = (size_t)labels[p];
            for (size_t c = 0; c < TF_C; ++c)
                query[p * TF_C + c] = sh[c * keys + idx] + d->class_b[c] + d->class_w[c * 10 + cls];
        }
        tf_position_embed(&d->self_pos, indices, P, width, tmp, query_pos);
        tf_position_embed(&d->cross_pos, NULL, keys, width, key_proj, key_value);
        for (size_t k = 0; k < keys; ++k)
            for (size_t c = 0; c < TF_C; ++c) key_value[k * TF_C + c] += sh[c * keys + k];
        for (size_t i = 0; i < P * TF_C; ++i) tmp[i] = query[i] + query_pos[i];
        tf_attention(tmp, P, tmp, P, d->self_in_w, d->self_in_b, d->self_out_w, d->self_out_b,
                     q_proj, key_proj, value_proj, slots, attn, tmp);
        tf_residual_norm(query, tmp, d->norm_w[0], d->norm_b[0], P);
        for (size_t i = 0; i < P * TF_C; ++i) tmp[i] = query[i] + query_pos[i];
        tf_attention(tmp, P, key_value, keys, d->cross_in_w, d->cross_in_b, d->cross_out_w,
                     d->cross_out_b, q_proj, key_proj, value_proj, slots, attn, tmp);
        tf_residual_norm(query, tmp, d->norm_w[1], d->norm_b[1], P);
        bf_linear_f32(query, d->lin1_w, d->lin1_b, ffn, P, TF_C, 256);
        bf_relu_f32(ffn, ffn, P * 256);
        bf_linear_f32(ffn, d->lin2_w, d->lin2_b, tmp, P, 256, TF_C);
        tf_residual_norm(query, tmp, d->norm_w[2], d->norm_b[2], P);
        float *heads[6] = {out->center_b2p + b * 2 * P, out->height_b1p + b * P,
                           out->dimension_log_b3p + b * 3 * P, out->rotation_sincos_b2p + b * 2 * P,
                           out->velocity_b2p + b * 2 * P, out->heatmap_logits_b10p + b * 10 * P};
        for (int h = 0; h < 6; ++h) tf_head_forward(&d->heads[h], query, P, head_hidden, heads[h]);
        for (size_t p = 0; p < P; ++p) {
            const size_t idx = (size_t)indices[p];
            out->center_b2p[(b * 2) * P + p] += (float)(idx % width) + 0.5f;
            out->center_b2p[(b * 2 + 1) * P + p] += (float)(idx / width) + 0.5f;
            for (size_t c = 0; c < 10; ++c)
                out->query_heatmap_scores_b10p[(b * 10 + c) * P + p] = suppressed[c * keys + idx];
        }
    }
    return 1;
}
