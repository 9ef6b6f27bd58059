// TransFusion decoder context (drop-in for reference src/cuda_transfusion.cu):
// proposal selection, query initialisation, self and cross multi-head
// attention with their position embeddings, FFN, three LayerNorms and the six
// prediction heads for one BEV map, plus the GPU detection decode.
//
// Work split by shape (P <= 200 proposals, K = H * W keys, C = 128 channels,
// 8 heads of 16):
//   suppress_kernel   sigmoid + 3x3 NMS over the 10 x K heatmap; writes the
//                     suppressed scores and one unique 64-bit sort key per
//                     candidate (score bits << 32 | ~flat), so descending key
//                     order is the reference's (score desc, flat asc) order.
//   topk_kernel       exact top-256 of each 8192-candidate chunk by an LDS
//                     bitonic sort, repeated over the chunk winners until one
//                     chunk remains: deterministic, no atomics, no memsets.
//   key_kernel        the K-row side on the matrix cores, one 64-key tile per
//                     workgroup: cell-centre position head (2 -> 128, BN,
//                     ReLU, 128 -> 128) + shared -> key_value, then the K and
//                     V projections; fp16 operands, fp32 accumulation; K is
//                     stored head-major [8][K][16], V channel-major [128][K]
//                     (the layouts the attention's MFMA operands read).
//   cross_attention   split-key flash attention on the matrix cores: a
//                     workgroup owns one head and one key split, each wave
//                     all 208 (padded) queries over its 64-key steps; scores
//                     S^T = K Q^T (16x16x16), probabilities fed straight
//                     back as the B operand of O^T = V^T P^T (16x16x32);
//                     online softmax in base 2 with Q pre-scaled by
//                     0.25 * log2(e); waves and splits merge in fixed order.
//   query/self/tail   one workgroup per proposal in fp32: query gather,
//                     self position head, QKV, self attention, out
//                     projection, LayerNorms, cross Q, split merge, FFN and
//                     the six heads (weights transposed at create so lanes
//                     read them coalesced).
#include "bf_cuda_transfusion.h"
#include "host_util.h"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <new>
#include <vector>

using namespace bfhip;

namespace {

constexpr int kC = 128, kHeads = 8, kHeadC = 16, kClasses = 10;
constexpr int kQTiles = 13, kPPad = kQTiles * 16;  // >= BF_MAX_PROPOSALS
constexpr int kTopSlots = 256, kChunk = 8192;
constexpr int kKeyTile = 64, kLdsRow = kC + 8;      // fp16 LDS row: 272 B, conflict-free
constexpr int kStepKeys = 64, kWaves = 4;
constexpr int kMaxSplits = 128;
constexpr int kHeadOutputs = 20;                    // 2 + 1 + 3 + 2 + 2 + 10
constexpr float kBnEps = 1e-5f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_16x16x16(h4 a, h4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x32(h8 a, h8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Device parameter views (one allocation).  "_t" matrices are stored
// transposed, [in][out], for the per-proposal kernels.
struct Params {
    const float *class_w, *class_b;      // [128][10], [128]
    const float *self_pos;               // [6][128]: w_x, w_y, b, mean, factor, beta
    const float *self_pos_w2t, *self_pos_b2;
    const float *self_in_t, *self_in_b;  // [128][384], [384]
    const float *self_out_t, *self_out_b;
    const float *cross_pos;              // [6][128]
    const _Float16 *cross_pos_w2;        // [128 out][128 in]
    const float *cross_pos_b2;
    const float *cross_q_t, *cross_q_b;  // [128][128], [128]
    const _Float16 *cross_kv;            // [256 out][128 in]: K rows then V rows
    const float *cross_kv_b;             // [256]
    const float *cross_out_t, *cross_out_b;
    const float *norm_w[3], *norm_b[3];
    const float *ffn1_t, *ffn1_b;        // [128][256], [256]
    const float *ffn2_t, *ffn2_b;        // [256][128], [128]
    const float *head_t;                 // [128][384]: six 64-wide hidden layers
    const float *head_bn;                // [3][384]: mean, factor, beta
    const float *head_out, *head_out_b;  // [20][64], [20]
};

// Logistic in the reference's two-branch form (transfusion.c:8-16).  exp is
// evaluated in double and rounded once, which is the correctly rounded expf,
// so scores (and hence the selected proposals) match a host built on a
// correctly rounded libm bit for bit.
__device__ __forceinline__ float logistic(float v) {
    if (v >= 0.0f) {
        const float e = (float)exp(-(double)v);
        return 1.0f / (1.0f + e);
    }
    const float e = (float)exp((double)v);
    return e / (1.0f + e);
}

// Reference transfusion.c:75-132 / cuda_transfusion.cu:164-170: classes 8 and
// 9 bypass NMS, border cells of the other classes are suppressed.
__global__ __launch_bounds__(256) void suppress_kernel(const float *__restrict__ logits,
                                                       float *__restrict__ suppressed,
                                                       uint64_t *__restrict__ sort_keys, int h,
                                                       int w, unsigned keys) {
    const unsigned f = blockIdx.x * 256u + threadIdx.x;
    if (f >= 10u * keys) return;
    const unsigned cls = f / keys, pos = f - cls * keys;
    const int y = (int)(pos / (unsigned)w), x = (int)pos - y * w;
    const float v = logistic(logits[f]);
    bool keep = cls == 8 || cls == 9;
    if (!keep && y > 0 && x > 0 && y + 1 < h && x + 1 < w) {
        const float *plane = logits + (size_t)cls * keys;
        float m = -FLT_MAX;
        for (int ky = -1; ky <= 1; ++ky)
            for (int kx = -1; kx <= 1; ++kx) {
                const float q = logistic(plane[(y + ky) * w + x + kx]);
                if (q > m) m = q;
            }
        keep = v == m;
    }
    const float out = keep ? v : 0.0f;
    suppressed[f] = out;
    const uint32_t bits = out != out ? 0x7fc00000u : __float_as_uint(out);
    sort_keys[f] = ((uint64_t)bits << 32) | (uint32_t)(0xffffffffu - f);
}

// Top 256 keys (descending) of each kChunk-key chunk: LDS bitonic sort of
// `sort_n` (a power of two, 256..8192) slots, zero-padded (zero is below
// every real key, whose low word ~flat is never 0 for flat < 2^32 - 1).
__global__ __launch_bounds__(1024) void topk_kernel(const uint64_t *__restrict__ in, int n,
                                                    int sort_n, uint64_t *__restrict__ out) {
    __shared__ uint64_t s[kChunk];
    const int t = threadIdx.x;
    const int base = blockIdx.x * kChunk, count = min(kChunk, n - base);
    for (int i = t; i < sort_n; i += 1024) s[i] = i < count ? in[base + i] : 0ull;
    __syncthreads();
    for (int k = 2; k <= sort_n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = t; i < sort_n / 2; i += 1024) {
                const int a = ((i & ~(j - 1)) << 1) | (i & (j - 1)), b = a + j;
                const bool desc = (a & k) == 0;
                const uint64_t x = s[a], y = s[b];
                if ((x < y) == desc) {
                    s[a] = y;
                    s[b] = x;
                }
            }
            __syncthreads();
        }
    for (int i = t; i < kTopSlots; i += 1024) out[blockIdx.x * kTopSlots + i] = s[i];
}

// ------------------------------------------------ per-proposal fp32 helpers
// y[n] = b[n] + sum_k x[k] wt[k][n] for one row; x in LDS, wt [K][N].  N = 128
// splits K over the two halves of the 256 threads; results land in y (LDS)
// and are visible after the caller's barrier.
template <int K, int N>
__device__ __forceinline__ void row_linear(const float *x, const float *__restrict__ wt,
                                           const float *__restrict__ b, float *y, float *red) {
    const int t = threadIdx.x;
    if constexpr (N == 128) {
        const int n = t & 127, k0 = (t >> 7) * (K / 2);
        float a = 0.0f;
#pragma unroll 8
        for (int k = 0; k < K / 2; ++k) a = fmaf(x[k0 + k], wt[(size_t)(k0 + k) * N + n], a);
        red[t] = a;
        __syncthreads();
        if (t < 128) y[t] = (b ? b[t] : 0.0f) + red[t] + red[t + 128];
    } else {
        for (int n = t; n < N; n += 256) {
            float a = 0.0f;
#pragma unroll 8
            for (int k = 0; k < K; ++k) a = fmaf(x[k], wt[(size_t)k * N + n], a);
            y[n] = (b ? b[n] : 0.0f) + a;
        }
    }
}

// LayerNorm over 128 channels held one per thread (t < 128), epsilon 1e-5
// (transfusion_decoder.c LayerNorm, kernels_ref.c:339-351): two-pass mean and
// variance.  Every thread must call it.
__device__ __forceinline__ float layer_norm128(float v, const float *__restrict__ w,
                                               const float *__restrict__ b, float *stat) {
    const int t = threadIdx.x;
    float s = group_sum<64>(t < 128 ? v : 0.0f);
    if ((t & 63) == 0 && t < 128) stat[t >> 6] = s;
    __syncthreads();
    const float mean = (stat[0] + stat[1]) * (1.0f / kC);
    const float d = t < 128 ? v - mean : 0.0f;
    const float q = group_sum<64>(d * d);
    if ((t & 63) == 0 && t < 128) stat[2 + (t >> 6)] = q;
    __syncthreads();
    const float inv = 1.0f / sqrtf((stat[2] + stat[3]) * (1.0f / kC) + kBnEps);
    return t < 128 ? d * inv * w[t] + b[t] : 0.0f;
}

// Cell-centre position head, first layer (transfusion_decoder.c:236-250):
// (b + w_x x + w_y y - mean) * factor + beta, then ReLU.
__device__ __forceinline__ float position_hidden(const float *__restrict__ p, int c, float x,
                                                 float y) {
    const float v = p[2 * kC + c] + p[c] * x + p[kC + c] * y;
    const float r = (v - p[3 * kC + c]) * p[4 * kC + c] + p[5 * kC + c];
    return r > 0.0f ? r : 0.0f;
}

// Query gather (class encoding at the proposal's label), self position head,
// self-attention Q/K/V (transfusion_decoder.c:384-405).
__global__ __launch_bounds__(256) void query_kernel(
    Params prm, const uint64_t *__restrict__ top, const float *__restrict__ suppressed,
    const float *__restrict__ shared, unsigned keys, int width, int P, float *__restrict__ query,
    float *__restrict__ query_pos, float *__restrict__ qkv, int64_t *__restrict__ labels,
    int64_t *__restrict__ indices, float *__restrict__ query_scores) {
    __shared__ float hid[kC], tmp[kC], pos[kC], out[3 * kC], red[256];
    const int p = blockIdx.x, t = threadIdx.x;
    // Every one of the first P keys is a real candidate (P <= 10 H W at
    // create); the clamp only keeps a zero pad key from indexing outside.
    const uint32_t flat = min(0xffffffffu - (uint32_t)top[p], 10u * keys - 1u);
    const unsigned label = flat / keys, idx = flat - label * keys;
    if (t == 0) {
        labels[p] = (int64_t)label;
        indices[p] = (int64_t)idx;
    }
    if (t < kClasses) query_scores[t * P + p] = suppressed[(size_t)t * keys + idx];
    float q = 0.0f;
    if (t < kC) {
        q = shared[(size_t)t * keys + idx] + prm.class_b[t] + prm.class_w[t * kClasses + label];
        query[p * kC + t] = q;
        const float x = (float)(idx % (unsigned)width) + 0.5f,
                    y = (float)(idx / (unsigned)width) + 0.5f;
        hid[t] = position_hidden(prm.self_pos, t, x, y);
    }
    __syncthreads();
    row_linear<kC, kC>(hid, prm.self_pos_w2t, prm.self_pos_b2, pos, red);
    __syncthreads();
    if (t < kC) {
        query_pos[p * kC + t] = pos[t];
        tmp[t] = q + pos[t];
    }
    __syncthreads();
    row_linear<kC, 3 * kC>(tmp, prm.self_in_t, prm.self_in_b, out, red);
    __syncthreads();
    for (int n = t; n < 3 * kC; n += 256) qkv[(size_t)(n / kC) * P * kC + p * kC + (n % kC)] = out[n];
}

// Self attention of one proposal over all P (transfusion_decoder.c:259-313:
// scores / sqrt(16), max-shifted softmax), out projection, residual +
// norm1, then the cross-attention query (query + query_pos) projected,
// scaled by 0.25 log2(e) and stored fp16 for the matrix cores.
__global__ __launch_bounds__(256) void self_attention_kernel(
    Params prm, const float *__restrict__ qkv, int P, float *__restrict__ query,
    const float *__restrict__ query_pos, _Float16 *__restrict__ cross_q) {
    __shared__ float q[kC], att[kC], upd[kC], x[kC], red[256], stat[4];
    __shared__ float prob[kHeads][BF_MAX_PROPOSALS];
    const int p = blockIdx.x, t = threadIdx.x;
    const float *qs = qkv, *ks = qkv + (size_t)P * kC, *vs = qkv + (size_t)2 * P * kC;
    if (t < kC) q[t] = qs[p * kC + t];
    __syncthreads();
    const int h = t >> 5, l = t & 31;
    float m = -FLT_MAX;
    for (int k = l; k < P; k += 32) {
        const float *kr = ks + (size_t)k * kC + h * kHeadC;
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < kHeadC; ++d) dot = fmaf(q[h * kHeadC + d], kr[d], dot);
        dot *= 0.25f;
        prob[h][k] = dot;
        m = fmaxf(m, dot);
    }
    m = group_max<32>(m);
    float sum = 0.0f;
    for (int k = l; k < P; k += 32) {
        const float e = expf(prob[h][k] - m);
        prob[h][k] = e;
        sum += e;
    }
    sum = group_sum<32>(sum);
    __syncthreads();
    {
        const int d = t & 15, half = (t >> 4) & 1;
        float a = 0.0f;
        for (int k = half; k < P; k += 2) a = fmaf(prob[h][k], vs[(size_t)k * kC + h * kHeadC + d], a);
        a += __shfl_xor(a, 16, 32);
        if (!half) att[h * kHeadC + d] = a / sum;
    }
    __syncthreads();
    row_linear<kC, kC>(att, prm.self_out_t, prm.self_out_b, upd, red);
    __syncthreads();
    const float v = t < kC ? query[p * kC + t] + upd[t] : 0.0f;
    const float q1 = layer_norm128(v, prm.norm_w[0], prm.norm_b[0], stat);
    if (t < kC) {
        query[p * kC + t] = q1;
        x[t] = q1 + query_pos[p * kC + t];
    }
    __syncthreads();
    row_linear<kC, kC>(x, prm.cross_q_t, prm.cross_q_b, upd, red);
    __syncthreads();
    if (t < kC) cross_q[p * kC + t] = (_Float16)(upd[t] * (0.25f * kLog2e));
}

// ----------------------------------------------------------- key side (MFMA)
// One 64-key tile: position head + shared -> key_value (fp16, LDS), then
// K = key_value Wk^T + bk (head-major [8][keys64][16]) and
// V = key_value Wv^T + bv (channel-major [128][keys64]).
__global__ __launch_bounds__(256) void key_kernel(Params prm, const float *__restrict__ shared,
                                                  unsigned keys, int width, int keys64,
                                                  _Float16 *__restrict__ kh,
                                                  _Float16 *__restrict__ vt) {
    __shared__ __attribute__((aligned(16))) _Float16 hid[kKeyTile * kLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 kv[kKeyTile * kLdsRow];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
    const int key0 = blockIdx.x * kKeyTile;
    {
        const int r = t & 63, c0 = (t >> 6) * 32;
        const unsigned kk = (unsigned)(key0 + r);
        const float x = (float)(kk % (unsigned)width) + 0.5f, y = (float)(kk / (unsigned)width) + 0.5f;
#pragma unroll
        for (int c = 0; c < 32; c += 8) {
            h8 v;
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (_Float16)position_hidden(prm.cross_pos, c0 + c + j, x, y);
            *(h8 *)&hid[r * kLdsRow + c0 + c] = v;
        }
    }
    __syncthreads();
    // key_value^T tile: rows = channels 32w .. 32w+31 (A = W2), columns = keys.
    {
        f32x4 acc[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
            h8 a[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                a[rt] = *(const h8 *)&prm.cross_pos_w2[(32 * w + 16 * rt + col) * kC + 32 * ks + 8 * g];
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const h8 b = *(const h8 *)&hid[(16 * ct + col) * kLdsRow + 32 * ks + 8 * g];
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) acc[rt][ct] = mfma_16x16x32(a[rt], b, acc[rt][ct]);
            }
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const unsigned kk = (unsigned)(key0 + 16 * ct + col);
                const int c0 = 32 * w + 16 * rt + 4 * g;
                h4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c = c0 + j;
                    const float sv = kk < keys ? shared[(size_t)c * keys + kk] : 0.0f;
                    o[j] = (_Float16)(acc[rt][ct][j] + prm.cross_pos_b2[c] + sv);
                }
                *(h4 *)&kv[(16 * ct + col) * kLdsRow + c0] = o;
            }
    }
    __syncthreads();
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (w < 2) {
        // K^T: rows = K channels 64w .. 64w+63 (A = Wk), columns = keys.
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
            h8 a[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                a[rt] = *(const h8 *)&prm.cross_kv[(64 * w + 16 * rt + col) * kC + 32 * ks + 8 * g];
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const h8 b = *(const h8 *)&kv[(16 * ct + col) * kLdsRow + 32 * ks + 8 * g];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) acc[rt][ct] = mfma_16x16x32(a[rt], b, acc[rt][ct]);
            }
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int c0 = 64 * w + 16 * rt + 4 * g, head = c0 >> 4;
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const int kk = key0 + 16 * ct + col;
                h4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = (_Float16)(acc[rt][ct][j] + prm.cross_kv_b[c0 + j]);
                *(h4 *)&kh[((size_t)head * keys64 + kk) * kHeadC + (c0 & 15)] = o;
            }
        }
    } else {
        // V: rows = keys (A = key_value), columns = V channels 64(w-2) ...
        const int vw = w - 2;
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
            h8 b[4];
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
                b[ct] = *(const h8 *)&prm.cross_kv[(kC + 64 * vw + 16 * ct + col) * kC + 32 * ks + 8 * g];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const h8 a = *(const h8 *)&kv[(16 * rt + col) * kLdsRow + 32 * ks + 8 * g];
#pragma unroll
                for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = mfma_16x16x32(a, b[ct], acc[rt][ct]);
            }
        }
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int c = 64 * vw + 16 * ct + col;
            const float bias = prm.cross_kv_b[kC + c];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                h4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = (_Float16)(acc[rt][ct][j] + bias);
                *(h4 *)&vt[(size_t)c * keys64 + key0 + 16 * rt + 4 * g] = o;
            }
        }
    }
}

// --------------------------------------------------- cross attention (MFMA)
// Workgroup (split s, head h); wave w takes steps s*4*spw + 4i + w.  Partial
// results per (split, head, query): running max m (base 2), sum l and the
// unnormalised 16-wide output.
__global__ __launch_bounds__(256) void cross_attention_kernel(
    const _Float16 *__restrict__ cross_q, const _Float16 *__restrict__ kh,
    const _Float16 *__restrict__ vt, int keys, int keys64, int steps_per_wave,
    float *__restrict__ part_m, float *__restrict__ part_l, float *__restrict__ part_o) {
    __shared__ float wm[kWaves][kPPad], wl[kWaves][kPPad];
    __shared__ float wo[kWaves][kPPad * kHeadC];
    const int s = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int w = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
    const int total_steps = keys64 / kStepKeys;

    h4 qf[kQTiles];
#pragma unroll
    for (int qt = 0; qt < kQTiles; ++qt)
        qf[qt] = *(const h4 *)&cross_q[(qt * 16 + col) * kC + h * kHeadC + 4 * g];
    float m[kQTiles], l[kQTiles];
    f32x4 o[kQTiles];
#pragma unroll
    for (int qt = 0; qt < kQTiles; ++qt) {
        m[qt] = kNegBig;
        l[qt] = 0.0f;
        o[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const _Float16 *kbase = kh + (size_t)h * keys64 * kHeadC;
    const _Float16 *vbase = vt + (size_t)h * kHeadC * keys64;
    // Row r of score MFMA 2a+b is key 32a + 8(r>>2) + 4b + (r&3): lane group g
    // then holds keys 32a + 8g .. +7, the k-slice of PV MFMA a's B operand.
    const int krow = 8 * (col >> 2) + (col & 3);

    for (int i = 0; i < steps_per_wave; ++i) {
        const int step = (s * steps_per_wave + i) * kWaves + w;
        if (step >= total_steps) break;
        const int k0 = step * kStepKeys;
        h4 kf[4];
        h8 vf[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
                kf[2 * a + b] = *(const h4 *)&kbase[(size_t)(k0 + 32 * a + 4 * b + krow) * kHeadC + 4 * g];
            vf[a] = *(const h8 *)&vbase[(size_t)col * keys64 + k0 + 32 * a + 8 * g];
        }
        const bool partial = k0 + kStepKeys > keys;
#pragma unroll
        for (int qt = 0; qt < kQTiles; ++qt) {
            f32x4 sc[4];
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
                sc[i4] = mfma_16x16x16(kf[i4], qf[qt], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
            if (partial) {
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (k0 + 32 * a + 8 * g + 4 * b + j >= keys) sc[2 * a + b][j] = kNegBig;
            }
            float mx = sc[0][0];
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
#pragma unroll
                for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sc[i4][j]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mn = fmaxf(m[qt], mx);
            const float alpha = __builtin_amdgcn_exp2f(m[qt] - mn);
            m[qt] = mn;
            float ps = 0.0f;
            h8 pf[2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float e = __builtin_amdgcn_exp2f(sc[2 * a + b][j] - mn);
                        ps += e;
                        pf[a][4 * b + j] = (_Float16)e;
                    }
            l[qt] = l[qt] * alpha + ps;
            o[qt] *= alpha;
#pragma unroll
            for (int a = 0; a < 2; ++a) o[qt] = mfma_16x16x32(vf[a], pf[a], o[qt]);
        }
    }
#pragma unroll
    for (int qt = 0; qt < kQTiles; ++qt) {
        float lt = l[qt] + __shfl_xor(l[qt], 16);
        lt += __shfl_xor(lt, 32);
        const int q = qt * 16 + col;
        if (g == 0) {
            wm[w][q] = m[qt];
            wl[w][q] = lt;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) wo[w][q * kHeadC + 4 * g + j] = o[qt][j];
    }
    __syncthreads();
    const size_t base = ((size_t)s * kHeads + h) * kPPad;
    for (int e = t; e < kPPad * kHeadC; e += 256) {
        const int q = e >> 4;
        float mm = wm[0][q];
#pragma unroll
        for (int v = 1; v < kWaves; ++v) mm = fmaxf(mm, wm[v][q]);
        float lsum = 0.0f, osum = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
            const float f = __builtin_amdgcn_exp2f(wm[v][q] - mm);
            lsum += wl[v][q] * f;
            osum += wo[v][e] * f;
        }
        part_o[base * kHeadC + e] = osum;
        if ((e & 15) == 0) {
            part_m[base + q] = mm;
            part_l[base + q] = lsum;
        }
    }
}

__device__ __forceinline__ int head_of_output(int j) {
    return j < 2 ? 0 : j < 3 ? 1 : j < 6 ? 2 : j < 8 ? 3 : j < 10 ? 4 : 5;
}

// Split merge (fixed order), cross out projection + norm2, FFN + norm3, and
// the six heads (transfusion_decoder.c:406-450).
__global__ __launch_bounds__(256) void tail_kernel(
    Params prm, const float *__restrict__ part_m, const float *__restrict__ part_l,
    const float *__restrict__ part_o, int splits, int P, int width,
    const float *__restrict__ query, const int64_t *__restrict__ indices,
    bf_transfusion_raw_outputs out) {
    __shared__ float ws[kHeads][kMaxSplits], lh[kHeads];
    __shared__ float att[kC], upd[kC], x[kC], ffn[2 * kC], hid[3 * kC], red[256], stat[4];
    const int p = blockIdx.x, t = threadIdx.x, h = t >> 5, l32 = t & 31;
    {
        float mm = kNegBig;
        for (int s = l32; s < splits; s += 32) mm = fmaxf(mm, part_m[((size_t)s * kHeads + h) * kPPad + p]);
        mm = group_max<32>(mm);
        float lsum = 0.0f;
        for (int s = l32; s < splits; s += 32) {
            const size_t i = ((size_t)s * kHeads + h) * kPPad + p;
            const float f = __builtin_amdgcn_exp2f(part_m[i] - mm);
            ws[h][s] = f;
            lsum += part_l[i] * f;
        }
        lsum = group_sum<32>(lsum);
        if (l32 == 0) lh[h] = lsum;
    }
    __syncthreads();
    {
        const int d = t & 15, half = (t >> 4) & 1;
        float a = 0.0f;
        for (int s = half; s < splits; s += 2)
            a = fmaf(part_o[(((size_t)s * kHeads + h) * kPPad + p) * kHeadC + d], ws[h][s], a);
        a += __shfl_xor(a, 16, 32);
        if (!half) att[h * kHeadC + d] = a / lh[h];
    }
    __syncthreads();
    row_linear<kC, kC>(att, prm.cross_out_t, prm.cross_out_b, upd, red);
    __syncthreads();
    const float v2 = t < kC ? query[p * kC + t] + upd[t] : 0.0f;
    const float q2 = layer_norm128(v2, prm.norm_w[1], prm.norm_b[1], stat);
    if (t < kC) x[t] = q2;
    __syncthreads();
    row_linear<kC, 2 * kC>(x, prm.ffn1_t, prm.ffn1_b, ffn, red);
    __syncthreads();
    ffn[t] = fmaxf(ffn[t], 0.0f);
    __syncthreads();
    row_linear<2 * kC, kC>(ffn, prm.ffn2_t, prm.ffn2_b, upd, red);
    __syncthreads();
    const float v3 = t < kC ? q2 + upd[t] : 0.0f;
    const float q3 = layer_norm128(v3, prm.norm_w[2], prm.norm_b[2], stat);
    if (t < kC) x[t] = q3;
    __syncthreads();
    row_linear<kC, 3 * kC>(x, prm.head_t, nullptr, hid, red);
    __syncthreads();
    for (int n = t; n < 3 * kC; n += 256) {
        const float r = (hid[n] - prm.head_bn[n]) * prm.head_bn[3 * kC + n] + prm.head_bn[6 * kC + n];
        hid[n] = r > 0.0f ? r : 0.0f;
    }
    __syncthreads();
    if (t < kHeadOutputs) {
        const float *hv = hid + 64 * head_of_output(t), *wv = prm.head_out + t * 64;
        float a = prm.head_out_b[t];
        for (int k = 0; k < 64; ++k) a = fmaf(hv[k], wv[k], a);
        const unsigned idx = (unsigned)indices[p];
        if (t == 0) a += (float)(idx % (unsigned)width) + 0.5f;
        if (t == 1) a += (float)(idx / (unsigned)width) + 0.5f;
        float *dst = t < 2    ? out.center_b2p + t * P
                     : t < 3  ? out.height_b1p
                     : t < 6  ? out.dimension_log_b3p + (t - 3) * P
                     : t < 8  ? out.rotation_sincos_b2p + (t - 6) * P
                     : t < 10 ? out.velocity_b2p + (t - 8) * P
                              : out.heatmap_logits_b10p + (t - 10) * P;
        dst[p] = a;
    }
}

// Reference cuda_transfusion.cu:368-391 / transfusion.c:134-193: decode and
// range-filter, kept detections compacted in proposal order.  Products and
// sums are kept unfused so the box centres round as the host decode does.
__global__ __launch_bounds__(256) void decode_kernel(bf_transfusion_raw_outputs r, int P,
                                                     float threshold,
                                                     bf_detections *__restrict__ out) {
#pragma clang fp contract(off)
    __shared__ int wave_count[4];
    const int p = threadIdx.x;
    bf_detection d = {};
    bool keep = false;
    if (p < P) {
        const int64_t label = r.query_labels_bp[p];
        if (label >= 0 && label < kClasses) {
            const float score = logistic(r.heatmap_logits_b10p[label * P + p]) *
                                r.query_heatmap_scores_b10p[label * P + p];
            d.x = r.center_b2p[p] * 0.6f - 54.0f;
            d.y = r.center_b2p[P + p] * 0.6f - 54.0f;
            d.z = r.height_b1p[p];
            d.width = expf(r.dimension_log_b3p[p]);
            d.length = expf(r.dimension_log_b3p[P + p]);
            d.height = expf(r.dimension_log_b3p[2 * P + p]);
            d.yaw = atan2f(r.rotation_sincos_b2p[p], r.rotation_sincos_b2p[P + p]);
            d.velocity_x = r.velocity_b2p[p];
            d.velocity_y = r.velocity_b2p[P + p];
            d.score = score;
            d.class_id = (int)label;
            keep = isfinite(score) && score > threshold && isfinite(d.x) && isfinite(d.y) &&
                   isfinite(d.z) && d.x >= -61.2f && d.x <= 61.2f && d.y >= -61.2f &&
                   d.y <= 61.2f && d.z >= -10.0f && d.z <= 10.0f;
        }
    }
    const uint64_t ballot = __ballot(keep);
    const int lane = p & 63, w = p >> 6;
    if (lane == 0) wave_count[w] = __popcll(ballot);
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += wave_count[i];
    if (keep) out->items[base + __popcll(ballot & ((1ull << lane) - 1ull))] = d;
    if (p == 0) out->count = wave_count[0] + wave_count[1] + wave_count[2] + wave_count[3];
}

struct TopPass {
    int n, chunks, sort_n;
};

}  // namespace

struct bf_cuda_transfusion {
    size_t height, width, keys, proposals, resident_bytes;
    int keys64, steps_per_wave, splits;
    std::vector<TopPass> passes;
    unsigned char *params, *arena;
    Params prm;
    // Views into the arena.
    float *suppressed, *query, *query_pos, *qkv, *part_m, *part_l, *part_o;
    uint64_t *sort_keys, *tops[2];
    const uint64_t *final_top;
    _Float16 *cross_q, *kh, *vt;
    bf_detections *detections;
};

namespace {

std::vector<float> transpose(const float *w, int rows, int cols) {
    std::vector<float> t((size_t)rows * cols);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) t[(size_t)c * rows + r] = w[(size_t)r * cols + c];
    return t;
}

// Eval BatchNorm as (v - mean) * factor + beta, factor = scale / sqrt(var + eps)
// (transfusion_decoder.c:226-234).
int bind_bn(const bf_model *m, const char *prefix, uint32_t c, float *mean, float *factor,
            float *beta, char *error, size_t cap) {
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float *p[4];
    char name[192];
    for (int i = 0; i < 4; ++i) {
        std::snprintf(name, sizeof(name), "%s.%s", prefix, suffix[i]);
        if (!(p[i] = bind_f32(m, name, {c}, error, cap))) return 0;
    }
    for (uint32_t i = 0; i < c; ++i) {
        mean[i] = p[2][i];
        factor[i] = p[0][i] / std::sqrt(p[3][i] + kBnEps);
        beta[i] = p[1][i];
    }
    return 1;
}

// Position head (transfusion_decoder.c:121-139): first-layer terms and BN in
// [6][128], second layer returned for the caller's layout.
int bind_position(const bf_model *m, const char *base, std::vector<float> &first,
                  const float **w2, const float **b2, char *error, size_t cap) {
    char name[192];
    std::snprintf(name, sizeof(name), "%s.position_embedding_head.0.weight", base);
    const float *w1 = bind_f32(m, name, {(uint32_t)kC, 2u, 1u}, error, cap);
    std::snprintf(name, sizeof(name), "%s.position_embedding_head.0.bias", base);
    const float *b1 = bind_f32(m, name, {(uint32_t)kC}, error, cap);
    if (!w1 || !b1) return 0;
    first.assign(6 * kC, 0.0f);
    for (int c = 0; c < kC; ++c) {
        first[c] = w1[2 * c];
        first[kC + c] = w1[2 * c + 1];
        first[2 * kC + c] = b1[c];
    }
    std::snprintf(name, sizeof(name), "%s.position_embedding_head.1", base);
    if (!bind_bn(m, name, kC, &first[3 * kC], &first[4 * kC], &first[5 * kC], error, cap)) return 0;
    std::snprintf(name, sizeof(name), "%s.position_embedding_head.3.weight", base);
    *w2 = bind_f32(m, name, {(uint32_t)kC, (uint32_t)kC, 1u}, error, cap);
    std::snprintf(name, sizeof(name), "%s.position_embedding_head.3.bias", base);
    *b2 = bind_f32(m, name, {(uint32_t)kC}, error, cap);
    return *w2 && *b2;
}

int build_params(bf_cuda_transfusion *d, const bf_model *m, char *error, size_t cap) {
    ParamArena pa;
    const char *dec = "dense_head.decoder.";
    char name[192];
    auto f32 = [&](const char *suffix, std::initializer_list<uint32_t> dims) {
        std::snprintf(name, sizeof(name), "%s%s", dec, suffix);
        return bind_f32(m, name, dims, error, cap);
    };
    const float *class_w = bind_f32(m, "dense_head.class_encoding.weight", {128u, 10u, 1u}, error, cap);
    const float *class_b = class_w ? bind_f32(m, "dense_head.class_encoding.bias", {128u}, error, cap) : nullptr;
    if (!class_w || !class_b) return 0;
    const float *self_in_w = f32("self_attn.in_proj_weight", {384u, 128u});
    const float *self_in_b = self_in_w ? f32("self_attn.in_proj_bias", {384u}) : nullptr;
    const float *self_out_w = self_in_b ? f32("self_attn.out_proj.weight", {128u, 128u}) : nullptr;
    const float *self_out_b = self_out_w ? f32("self_attn.out_proj.bias", {128u}) : nullptr;
    const float *cross_in_w = self_out_b ? f32("multihead_attn.in_proj_weight", {384u, 128u}) : nullptr;
    const float *cross_in_b = cross_in_w ? f32("multihead_attn.in_proj_bias", {384u}) : nullptr;
    const float *cross_out_w = cross_in_b ? f32("multihead_attn.out_proj.weight", {128u, 128u}) : nullptr;
    const float *cross_out_b = cross_out_w ? f32("multihead_attn.out_proj.bias", {128u}) : nullptr;
    const float *lin1_w = cross_out_b ? f32("linear1.weight", {256u, 128u}) : nullptr;
    const float *lin1_b = lin1_w ? f32("linear1.bias", {256u}) : nullptr;
    const float *lin2_w = lin1_b ? f32("linear2.weight", {128u, 256u}) : nullptr;
    const float *lin2_b = lin2_w ? f32("linear2.bias", {128u}) : nullptr;
    if (!lin2_b) return 0;
    const float *norm_w[3], *norm_b[3];
    for (int i = 0; i < 3; ++i) {
        char s[32];
        std::snprintf(s, sizeof(s), "norm%d.weight", i + 1);
        if (!(norm_w[i] = f32(s, {128u}))) return 0;
        std::snprintf(s, sizeof(s), "norm%d.bias", i + 1);
        if (!(norm_b[i] = f32(s, {128u}))) return 0;
    }
    std::vector<float> self_first, cross_first;
    const float *self_w2, *self_b2, *cross_w2, *cross_b2;
    if (!bind_position(m, "dense_head.decoder.self_posembed", self_first, &self_w2, &self_b2, error, cap) ||
        !bind_position(m, "dense_head.decoder.cross_posembed", cross_first, &cross_w2, &cross_b2, error, cap))
        return 0;
    // Heads (transfusion_decoder.c:141-163): hidden conv1d 128 -> 64 without
    // bias + BN + ReLU, then conv1d 64 -> C with bias.
    static const char *heads[6] = {"center", "height", "dim", "rot", "vel", "heatmap"};
    static const uint32_t channels[6] = {2, 1, 3, 2, 2, 10};
    std::vector<float> head_w((size_t)3 * kC * kC), head_bn((size_t)9 * kC);
    std::vector<float> head_out((size_t)kHeadOutputs * 64), head_out_b(kHeadOutputs);
    for (int i = 0, j0 = 0; i < 6; ++i) {
        std::snprintf(name, sizeof(name), "dense_head.prediction_head.%s.0.0.weight", heads[i]);
        const float *hw = bind_f32(m, name, {64u, (uint32_t)kC, 1u}, error, cap);
        if (!hw) return 0;
        std::memcpy(&head_w[(size_t)64 * i * kC], hw, sizeof(float) * 64 * kC);
        std::snprintf(name, sizeof(name), "dense_head.prediction_head.%s.0.1", heads[i]);
        if (!bind_bn(m, name, 64, &head_bn[64 * i], &head_bn[3 * kC + 64 * i],
                     &head_bn[6 * kC + 64 * i], error, cap))
            return 0;
        std::snprintf(name, sizeof(name), "dense_head.prediction_head.%s.1.weight", heads[i]);
        const float *ow = bind_f32(m, name, {channels[i], 64u, 1u}, error, cap);
        std::snprintf(name, sizeof(name), "dense_head.prediction_head.%s.1.bias", heads[i]);
        const float *ob = ow ? bind_f32(m, name, {channels[i]}, error, cap) : nullptr;
        if (!ow || !ob) return 0;
        std::memcpy(&head_out[(size_t)64 * j0], ow, sizeof(float) * 64 * channels[i]);
        std::memcpy(&head_out_b[j0], ob, sizeof(float) * channels[i]);
        j0 += (int)channels[i];
    }

    struct Off {
        size_t class_w, class_b, self_pos, self_w2t, self_b2, self_in_t, self_in_b, self_out_t,
            self_out_b, cross_pos, cross_w2, cross_b2, cross_q_t, cross_q_b, cross_kv, cross_kv_b,
            cross_out_t, cross_out_b, norm_w[3], norm_b[3], ffn1_t, ffn1_b, ffn2_t, ffn2_b, head_t,
            head_bn, head_out, head_out_b;
    } o;
    o.class_w = pa.add_f32(class_w, (size_t)kC * kClasses);
    o.class_b = pa.add_f32(class_b, kC);
    o.self_pos = pa.add_f32(self_first);
    o.self_w2t = pa.add_f32(transpose(self_w2, kC, kC));
    o.self_b2 = pa.add_f32(self_b2, kC);
    o.self_in_t = pa.add_f32(transpose(self_in_w, 3 * kC, kC));
    o.self_in_b = pa.add_f32(self_in_b, 3 * kC);
    o.self_out_t = pa.add_f32(transpose(self_out_w, kC, kC));
    o.self_out_b = pa.add_f32(self_out_b, kC);
    o.cross_pos = pa.add_f32(cross_first);
    o.cross_w2 = pa.add_f16(cross_w2, (size_t)kC * kC);
    o.cross_b2 = pa.add_f32(cross_b2, kC);
    o.cross_q_t = pa.add_f32(transpose(cross_in_w, kC, kC));
    o.cross_q_b = pa.add_f32(cross_in_b, kC);
    o.cross_kv = pa.add_f16(cross_in_w + (size_t)kC * kC, (size_t)2 * kC * kC);
    o.cross_kv_b = pa.add_f32(cross_in_b + kC, 2 * kC);
    o.cross_out_t = pa.add_f32(transpose(cross_out_w, kC, kC));
    o.cross_out_b = pa.add_f32(cross_out_b, kC);
    for (int i = 0; i < 3; ++i) {
        o.norm_w[i] = pa.add_f32(norm_w[i], kC);
        o.norm_b[i] = pa.add_f32(norm_b[i], kC);
    }
    o.ffn1_t = pa.add_f32(transpose(lin1_w, 2 * kC, kC));
    o.ffn1_b = pa.add_f32(lin1_b, 2 * kC);
    o.ffn2_t = pa.add_f32(transpose(lin2_w, kC, 2 * kC));
    o.ffn2_b = pa.add_f32(lin2_b, kC);
    o.head_t = pa.add_f32(transpose(head_w.data(), 3 * kC, kC));
    o.head_bn = pa.add_f32(head_bn);
    o.head_out = pa.add_f32(head_out);
    o.head_out_b = pa.add_f32(head_out_b);

    if (!hip_ok(hipMalloc((void **)&d->params, pa.host.size()), error, cap, "allocate decoder weights") ||
        !hip_ok(hipMemcpy(d->params, pa.host.data(), pa.host.size(), hipMemcpyHostToDevice), error,
                cap, "upload decoder weights"))
        return 0;
    d->resident_bytes += pa.host.size();
    unsigned char *b = d->params;
    auto F = [&](size_t off) { return (const float *)(b + off); };
    auto H = [&](size_t off) { return (const _Float16 *)(b + off); };
    Params &p = d->prm;
    p.class_w = F(o.class_w);
    p.class_b = F(o.class_b);
    p.self_pos = F(o.self_pos);
    p.self_pos_w2t = F(o.self_w2t);
    p.self_pos_b2 = F(o.self_b2);
    p.self_in_t = F(o.self_in_t);
    p.self_in_b = F(o.self_in_b);
    p.self_out_t = F(o.self_out_t);
    p.self_out_b = F(o.self_out_b);
    p.cross_pos = F(o.cross_pos);
    p.cross_pos_w2 = H(o.cross_w2);
    p.cross_pos_b2 = F(o.cross_b2);
    p.cross_q_t = F(o.cross_q_t);
    p.cross_q_b = F(o.cross_q_b);
    p.cross_kv = H(o.cross_kv);
    p.cross_kv_b = F(o.cross_kv_b);
    p.cross_out_t = F(o.cross_out_t);
    p.cross_out_b = F(o.cross_out_b);
    for (int i = 0; i < 3; ++i) {
        p.norm_w[i] = F(o.norm_w[i]);
        p.norm_b[i] = F(o.norm_b[i]);
    }
    p.ffn1_t = F(o.ffn1_t);
    p.ffn1_b = F(o.ffn1_b);
    p.ffn2_t = F(o.ffn2_t);
    p.ffn2_b = F(o.ffn2_b);
    p.head_t = F(o.head_t);
    p.head_bn = F(o.head_bn);
    p.head_out = F(o.head_out);
    p.head_out_b = F(o.head_out_b);
    return 1;
}

int build_work(bf_cuda_transfusion *d, char *error, size_t cap) {
    const size_t keys = d->keys, P = d->proposals, cand = 10 * keys;
    d->keys64 = (int)((keys + kKeyTile - 1) / kKeyTile * kKeyTile);
    // Top-k passes: chunks of kChunk candidates keep kTopSlots each, until one
    // chunk remains.
    for (size_t n = cand;;) {
        const size_t chunks = (n + kChunk - 1) / kChunk;
        int sort_n = kTopSlots;
        while ((size_t)sort_n < std::min(n, (size_t)kChunk)) sort_n <<= 1;
        d->passes.push_back({(int)n, (int)chunks, sort_n});
        if (chunks == 1) break;
        n = chunks * kTopSlots;
    }
    // Key splits: about 512 workgroups (two per CU) over 8 heads, at most
    // kMaxSplits splits.
    const int steps = d->keys64 / kStepKeys;
    int spw = std::max(1, (steps + kWaves * 64 - 1) / (kWaves * 64));
    spw = std::max(spw, (steps + kWaves * kMaxSplits - 1) / (kWaves * kMaxSplits));
    d->steps_per_wave = spw;
    d->splits = (steps + kWaves * spw - 1) / (kWaves * spw);

    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~size_t(255);
        return at;
    };
    const size_t chunks0 = d->passes[0].chunks;
    const size_t o_supp = take(cand * 4), o_keys = take(cand * 8);
    const size_t o_top0 = take(chunks0 * kTopSlots * 8), o_top1 = take(chunks0 * kTopSlots * 8);
    const size_t o_query = take(P * kC * 4), o_pos = take(P * kC * 4), o_qkv = take(3 * P * kC * 4);
    const size_t o_cq = take((size_t)kPPad * kC * 2);
    const size_t o_kh = take((size_t)d->keys64 * kC * 2), o_vt = take((size_t)d->keys64 * kC * 2);
    const size_t parts = (size_t)d->splits * kHeads * kPPad;
    const size_t o_pm = take(parts * 4), o_pl = take(parts * 4), o_po = take(parts * kHeadC * 4);
    const size_t o_det = take(sizeof(bf_detections));
    if (!hip_ok(hipMalloc((void **)&d->arena, off), error, cap, "allocate decoder workspace") ||
        !hip_ok(hipMemset(d->arena, 0, off), error, cap, "clear decoder workspace"))
        return 0;
    d->resident_bytes += off;
    unsigned char *a = d->arena;
    d->suppressed = (float *)(a + o_supp);
    d->sort_keys = (uint64_t *)(a + o_keys);
    d->tops[0] = (uint64_t *)(a + o_top0);
    d->tops[1] = (uint64_t *)(a + o_top1);
    d->query = (float *)(a + o_query);
    d->query_pos = (float *)(a + o_pos);
    d->qkv = (float *)(a + o_qkv);
    d->cross_q = (_Float16 *)(a + o_cq);  // rows >= P stay zero
    d->kh = (_Float16 *)(a + o_kh);
    d->vt = (_Float16 *)(a + o_vt);
    d->part_m = (float *)(a + o_pm);
    d->part_l = (float *)(a + o_pl);
    d->part_o = (float *)(a + o_po);
    d->detections = (bf_detections *)(a + o_det);
    d->final_top = d->tops[(d->passes.size() - 1) & 1];
    return 1;
}

bool outputs_ok(const bf_transfusion_raw_outputs *o) {
    return o && o->center_b2p && o->height_b1p && o->dimension_log_b3p && o->rotation_sincos_b2p &&
           o->velocity_b2p && o->heatmap_logits_b10p && o->query_heatmap_scores_b10p &&
           o->query_labels_bp && o->query_indices_bp;
}

}  // namespace

extern "C" void bf_cuda_transfusion_destroy(bf_cuda_transfusion *d) {
    if (!d) return;
    if (d->params) (void)hipFree(d->params);
    if (d->arena) (void)hipFree(d->arena);
    delete d;
}

extern "C" size_t bf_cuda_transfusion_resident_bytes(const bf_cuda_transfusion *d) {
    return d ? d->resident_bytes : 0;
}

extern "C" int bf_cuda_transfusion_create(const bf_model *model, size_t height, size_t width,
                                          size_t proposals, bf_cuda_transfusion **out,
                                          char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!model || !out || !height || !width || !proposals || proposals > BF_MAX_PROPOSALS ||
        height > INT_MAX || width > INT_MAX || height > SIZE_MAX / width ||
        10 * height * width > UINT32_MAX)
        return fail(error, cap, "invalid HIP TransFusion contract");
    if (proposals > 10 * height * width || (unsigned long long)kC * height * width > INT_MAX)
        return fail(error, cap, "HIP TransFusion shape is out of range");
    bf_cuda_transfusion *d = new (std::nothrow) bf_cuda_transfusion{};
    if (!d) return fail(error, cap, "HIP TransFusion context allocation failed");
    d->height = height;
    d->width = width;
    d->keys = height * width;
    d->proposals = proposals;
    if (!build_params(d, model, error, cap) || !build_work(d, error, cap)) {
        bf_cuda_transfusion_destroy(d);
        return 0;
    }
    *out = d;
    return 1;
}

extern "C" int bf_cuda_transfusion_forward(bf_cuda_transfusion *d, const float *shared,
                                           const float *heatmap,
                                           bf_transfusion_raw_outputs *out, void *stream_value,
                                           char *error, size_t cap) {
    if (!d || !shared || !heatmap || !outputs_ok(out))
        return fail(error, cap, "invalid HIP TransFusion buffers");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    const unsigned keys = (unsigned)d->keys, cand = 10u * keys;
    const int P = (int)d->proposals, W = (int)d->width;
    suppress_kernel<<<(cand + 255) / 256, 256, 0, s>>>(heatmap, d->suppressed, d->sort_keys,
                                                      (int)d->height, W, keys);
    key_kernel<<<d->keys64 / kKeyTile, 256, 0, s>>>(d->prm, shared, keys, W, d->keys64, d->kh, d->vt);
    const uint64_t *in = d->sort_keys;
    for (size_t i = 0; i < d->passes.size(); ++i) {
        const TopPass &tp = d->passes[i];
        uint64_t *dst = d->tops[i & 1];
        topk_kernel<<<tp.chunks, 1024, 0, s>>>(in, tp.n, tp.sort_n, dst);
        in = dst;
    }
    query_kernel<<<P, 256, 0, s>>>(d->prm, d->final_top, d->suppressed, shared, keys, W, P,
                                   d->query, d->query_pos, d->qkv, out->query_labels_bp,
                                   out->query_indices_bp, out->query_heatmap_scores_b10p);
    self_attention_kernel<<<P, 256, 0, s>>>(d->prm, d->qkv, P, d->query, d->query_pos, d->cross_q);
    cross_attention_kernel<<<dim3(d->splits, kHeads), 256, 0, s>>>(
        d->cross_q, d->kh, d->vt, (int)keys, d->keys64, d->steps_per_wave, d->part_m, d->part_l,
        d->part_o);
    tail_kernel<<<P, 256, 0, s>>>(d->prm, d->part_m, d->part_l, d->part_o, d->splits, P, W,
                                  d->query, out->query_indices_bp, *out);
    return launch_ok(error, cap, "HIP TransFusion launch");
}

extern "C" int bf_cuda_transfusion_decode_detections(bf_cuda_transfusion *d,
                                                     const bf_transfusion_raw_outputs *out,
                                                     float threshold, bf_detections *host,
                                                     void *stream_value, char *error, size_t cap) {
    if (!d || !host || !std::isfinite(threshold) || !outputs_ok(out))
        return fail(error, cap, "invalid HIP detection decode contract");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    decode_kernel<<<1, 256, 0, s>>>(*out, (int)d->proposals, threshold, d->detections);
    if (!launch_ok(error, cap, "HIP detection decode launch") ||
        !hip_ok(hipMemcpyAsync(host, d->detections, sizeof(*host), hipMemcpyDeviceToHost, s), error,
                cap, "copy detections") ||
        !hip_ok(hipStreamSynchronize(s), error, cap, "synchronize detections"))
        return 0;
    if (host->count < 0 || host->count > BF_MAX_PROPOSALS)
        return fail(error, cap, "detection count out of range");
    return 1;
}
