// TransFusion decoder context (drop-in for reference src/cuda_transfusion.cu):
// proposal selection, query initialisation, self and cross multi-head
// attention with their position embeddings, FFN, three LayerNorms and the six
// prediction heads for one BEV map, plus the GPU detection decode.
//
// Work split by shape (P <= 200 proposals, K = H * W keys, C = 128 channels,
// 8 heads of 16):
//   suppress_kernel   sigmoid + 3x3 NMS over the 10 x K heatmap, one 32 x 32
//                     tile per workgroup with the logistic evaluated once per
//                     cell into LDS; writes the suppressed scores and one
//                     unique 64-bit sort key per candidate (score bits << 32 |
//                     ~flat), so descending key order is the reference's
//                     (score desc, flat asc) order, and counts the keys' top
//                     11 bits for the selection below.
//   top-P selection   exact radix select of the P-th largest key over
//                     11/10-bit digits, with no atomics between workgroups:
//                     suppress stores a per-tile histogram of the keys' top
//                     digit and hist_reduce_kernel sums them.  When more than
//                     8192 keys share or pass the P-th key's top digit (a
//                     flat heatmap: random weights put ~10^5 candidates in
//                     one bin), refine_kernel histograms the second digit
//                     within that bin and a second hist_reduce sums those;
//                     otherwise both return at once.  compact_kernel picks
//                     the threshold's top digit (two digits when refined) and
//                     gathers the keys at or above it into per-workgroup
//                     segments, and finish_kernel (one workgroup)
//                     pulls the segments into LDS, refines the remaining
//                     digits, keeps the P winners and sorts them (256-slot
//                     bitonic).  Every buffer is rewritten each forward
//                     (nothing to reset, no memsets: graph-capturable);
//                     integer histograms and a sort of unique keys make it
//                     deterministic.
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
#include "internal.h"

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
constexpr int kTopSlots = 256;
constexpr int kDigitBins = 2048, kLevels = 6;
constexpr int kMaxSegments = 4096, kLdsKeys = 8192;
constexpr int kNmsTile = 32, kNmsHalo = kNmsTile + 2;
constexpr int kKeyTile = 64, kLdsRow = kC + 8;      // fp16 LDS row: 272 B, conflict-free
constexpr int kStepKeys = 64;
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

// Digit of pass `level`: bits [shift, shift + width) of the key, most
// significant first (11 + 11 + 10 bits of score, then of ~flat).
__device__ __forceinline__ int digit_shift(int level) {
    return level == 0 ? 53 : level == 1 ? 42 : level == 2 ? 32 : level == 3 ? 21 : level == 4 ? 10 : 0;
}
__device__ __forceinline__ int digit_width(int level) { return level == 2 || level == 5 ? 10 : 11; }

// Finds the digit of a 2048-bin histogram that holds the k-th largest key
// (1 <= k <= total): res[0] = digit, res[1] = keys with a larger digit,
// res[2] = the digit's count.  T threads scan 2048 / T bins each; the suffix
// sums run in-wave by shuffles, `wsum` (T / 64 words of LDS) joins the waves.
// Every thread must call it; ends on a barrier.
template <int T>
__device__ void pick_digit(const unsigned *hist, unsigned k, unsigned *wsum, unsigned *res) {
    constexpr int B = kDigitBins / T;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    unsigned h[B], sum = 0;
#pragma unroll
    for (int j = 0; j < B; ++j) {
        h[j] = hist[B * t + j];
        sum += h[j];
    }
    unsigned v = sum;  // becomes the sum over lanes >= lane of this wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned u = __shfl_down(v, o);
        if (lane + o < 64) v += u;
    }
    if (lane == 0) wsum[wave] = v;
    __syncthreads();
    unsigned above = v - sum;
    for (int w2 = wave + 1; w2 < T / 64; ++w2) above += wsum[w2];
#pragma unroll
    for (int j = B - 1; j >= 0; --j) {
        if (above < k && k <= above + h[j]) {
            res[0] = B * t + j;
            res[1] = above;
            res[2] = h[j];
        }
        above += h[j];
    }
    __syncthreads();
}

// Reference transfusion.c:75-132 / cuda_transfusion.cu:164-170: classes 8 and
// 9 bypass NMS, border cells of the other classes are suppressed.  One
// workgroup per 32 x 32 tile of one class; the tile's histogram of key top
// digits is stored whole at part_hist[tile][2048].
__global__ __launch_bounds__(256) void suppress_kernel(const float *__restrict__ logits,
                                                       float *__restrict__ suppressed,
                                                       uint64_t *__restrict__ sort_keys, int h,
                                                       int w, unsigned keys, int tiles_x,
                                                       int tiles_y, unsigned *__restrict__ part_hist) {
    __shared__ float sig[kNmsHalo * kNmsHalo];
    __shared__ unsigned lh[kDigitBins];
    const int t = threadIdx.x, lane = t & 63;
    const int tile = blockIdx.x, cls = tile / (tiles_x * tiles_y);
    const int ty = (tile / tiles_x) % tiles_y, tx = tile % tiles_x;
    const int y0 = ty * kNmsTile, x0 = tx * kNmsTile;
    const float *plane = logits + (size_t)cls * keys;
    for (int i = t; i < kNmsHalo * kNmsHalo; i += 256) {
        const int yy = y0 - 1 + i / kNmsHalo, xx = x0 - 1 + i % kNmsHalo;
        sig[i] = yy >= 0 && yy < h && xx >= 0 && xx < w ? logistic(plane[yy * w + xx]) : 0.0f;
    }
    for (int d = t; d < kDigitBins; d += 256) lh[d] = 0u;
    __syncthreads();
    const bool exempt = cls == 8 || cls == 9;
#pragma unroll
    for (int j = 0; j < kNmsTile * kNmsTile / 256; ++j) {
        const int o = t + 256 * j, oy = o / kNmsTile, ox = o % kNmsTile;
        const int y = y0 + oy, x = x0 + ox;
        const bool inside = y < h && x < w;
        unsigned digit = 0;
        if (inside) {
            const float *c = &sig[(oy + 1) * kNmsHalo + ox + 1];
            const float v = c[0];
            bool keep = exempt;
            if (!keep && y > 0 && x > 0 && y + 1 < h && x + 1 < w) {
                float m = -FLT_MAX;
                for (int ky = -1; ky <= 1; ++ky)
                    for (int kx = -1; kx <= 1; ++kx) {
                        const float q = c[ky * kNmsHalo + kx];
                        if (q > m) m = q;
                    }
                keep = v == m;
            }
            const float out = keep ? v : 0.0f;
            const unsigned f = (unsigned)cls * keys + (unsigned)(y * w + x);
            suppressed[f] = out;
            const uint32_t bits = out != out ? 0x7fc00000u : __float_as_uint(out);
            const uint64_t key = ((uint64_t)bits << 32) | (uint32_t)(0xffffffffu - f);
            sort_keys[f] = key;
            digit = (unsigned)(key >> 53);
        }
        // Suppressed cells (digit 0) dominate: one LDS atomic per wave for them.
        const uint64_t zero = __ballot(inside && digit == 0);
        if (lane == 0 && zero) atomicAdd(&lh[0], (unsigned)__popcll(zero));
        if (inside && digit) atomicAdd(&lh[digit], 1u);
    }
    __syncthreads();
    unsigned *dst = part_hist + (size_t)tile * kDigitBins;
    for (int d = t; d < kDigitBins; d += 256) dst[d] = lh[d];
}

// hist[d] = sum over tiles of part_hist[tile][d]: workgroup b owns bins
// 8b .. 8b+7, its 32 thread slices stride over the tiles.  With `only_if`
// set, returns at once unless *only_if is nonzero.
__global__ __launch_bounds__(256) void hist_reduce_kernel(const unsigned *__restrict__ part_hist,
                                                          int tiles, unsigned *__restrict__ hist,
                                                          const unsigned *__restrict__ only_if) {
    if (only_if && !*only_if) return;  // whole workgroup: before the barrier
    __shared__ unsigned red[256];
    const int t = threadIdx.x, d = blockIdx.x * 8 + (t & 7);
    unsigned sum = 0;
#pragma unroll 4
    for (int p = t >> 3; p < tiles; p += 32) sum += part_hist[(size_t)p * kDigitBins + d];
    red[t] = sum;
    __syncthreads();
    if (t < 8) {
        unsigned total = 0;
        for (int i = 0; i < 32; ++i) total += red[8 * i + t];
        hist[blockIdx.x * 8 + t] = total;
    }
}

// Second radix level over the whole candidate set, for when the P-th key's
// top digit leaves more keys than the finish holds in LDS: workgroup g
// histograms the second digit of the keys in chunk g whose top digit is that
// digit, into part_hist1[g].  Workgroup 0 stores whether this level runs in
// *refined (every forward: nothing to reset).
__global__ __launch_bounds__(256) void refine_kernel(const uint64_t *__restrict__ keys, unsigned n,
                                                     unsigned chunk, const unsigned *__restrict__ hist,
                                                     int P, unsigned *__restrict__ part_hist1,
                                                     unsigned *__restrict__ refined) {
    __shared__ unsigned lh[kDigitBins], wsum[4], res[3];
    pick_digit<256>(hist, (unsigned)P, wsum, res);
    const int t = threadIdx.x;
    const bool run = res[1] + res[2] > (unsigned)kLdsKeys;  // keys the finish would gather
    if (blockIdx.x == 0 && t == 0) *refined = run ? 1u : 0u;
    if (!run) return;  // uniform over the workgroup
    const uint64_t top = res[0];
    const int shift = digit_shift(1);
    for (int d = t; d < kDigitBins; d += 256) lh[d] = 0u;
    __syncthreads();
    const unsigned begin = blockIdx.x * chunk, end = min(begin + chunk, n);
    for (unsigned i = begin + t; i < end; i += 256u) {
        const uint64_t key = keys[i];
        if (key >> digit_shift(0) == top)
            atomicAdd(&lh[(unsigned)(key >> shift) & (kDigitBins - 1u)], 1u);
    }
    __syncthreads();
    unsigned *dst = part_hist1 + (size_t)blockIdx.x * kDigitBins;
    for (int d = t; d < kDigitBins; d += 256) dst[d] = lh[d];
}

// Threshold of the gathered keys: the P-th largest key's top digit, and when
// refined its second digit too (hist1 then counts the second digits within
// the top digit's bin).  Returns the threshold key and leaves in *k the rank
// of the P-th key among the keys sharing that prefix, in *exact whether
// those are exactly the keys left.  Every thread must call it.
template <int T>
__device__ unsigned long long threshold_prefix(const unsigned *hist, const unsigned *hist1,
                                               bool refined, int P, unsigned *wsum,
                                               unsigned *res, unsigned *k, bool *exact) {
    pick_digit<T>(hist, (unsigned)P, wsum, res);
    unsigned long long prefix = (unsigned long long)res[0] << digit_shift(0);
    unsigned left = (unsigned)P - res[1];
    bool done = res[2] == left;
    if (refined) {
        pick_digit<T>(hist1, left, wsum, res);  // res is read above before its barrier
        prefix |= (unsigned long long)res[0] << digit_shift(1);
        left -= res[1];
        done = res[2] == left;
    }
    *k = left;
    *exact = done;
    return prefix;
}

// Gathers every key at or above the threshold prefix (threshold_prefix):
// workgroup g appends (LDS counter) into list[g * chunk ...] and stores its
// count in counts[g].
__global__ __launch_bounds__(256) void compact_kernel(const uint64_t *__restrict__ keys, unsigned n,
                                                      unsigned chunk, const unsigned *__restrict__ hist,
                                                      const unsigned *__restrict__ hist1,
                                                      const unsigned *__restrict__ refined, int P,
                                                      uint64_t *__restrict__ list,
                                                      unsigned *__restrict__ counts) {
    __shared__ unsigned wsum[4], res[3], taken;
    unsigned k;
    bool exact;
    const unsigned long long threshold =
        threshold_prefix<256>(hist, hist1, *refined != 0u, P, wsum, res, &k, &exact);
    const int t = threadIdx.x, lane = t & 63;
    if (t == 0) taken = 0u;
    __syncthreads();
    const unsigned begin = blockIdx.x * chunk, end = min(begin + chunk, n);
    for (unsigned base = begin + (t & ~63u); base < end; base += 256u) {
        const unsigned i = base + lane;
        const uint64_t key = i < end ? keys[i] : 0ull;
        const bool take = i < end && key >= threshold;
        const uint64_t b = __ballot(take);
        if (!b) continue;
        unsigned first = 0;
        if (lane == 0) first = atomicAdd(&taken, (unsigned)__popcll(b));
        first = __shfl(first, 0);
        if (take) list[begin + first + __popcll(b & ((1ull << lane) - 1ull))] = key;
    }
    __syncthreads();
    if (t == 0) counts[blockIdx.x] = taken;
}

// One workgroup: lines the gathered segments up (LDS when they fit, else read
// in place), refines the remaining digits of the threshold, keeps the P keys
// >= it and sorts them descending into `top`.
__global__ __launch_bounds__(1024) void finish_kernel(const uint64_t *__restrict__ list,
                                                      const unsigned *__restrict__ counts,
                                                      int segments, unsigned chunk,
                                                      const unsigned *__restrict__ hist,
                                                      const unsigned *__restrict__ hist1,
                                                      const unsigned *__restrict__ refined, int P,
                                                      uint64_t *__restrict__ top) {
    __shared__ unsigned lh[kDigitBins], wsum[16], res[3], off[kMaxSegments + 1], count;
    __shared__ uint64_t lk[kLdsKeys];
    __shared__ uint64_t s[kTopSlots];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const bool two = *refined != 0u;
    unsigned k;
    bool resolved;
    unsigned long long prefix =
        threshold_prefix<1024>(hist, hist1, two, P, wsum, res, &k, &resolved);
    // Exclusive scan of the segment counts, four segments per thread.
    unsigned c[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int g = 4 * t + j;
        c[j] = g < segments ? counts[g] : 0u;
        sum += c[j];
    }
    unsigned v = sum;  // inclusive prefix within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    unsigned before = v - sum;
    for (int w2 = 0; w2 < wave; ++w2) before += wsum[w2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (4 * t + j <= segments) off[4 * t + j] = before;
        before += c[j];
    }
    __syncthreads();
    const unsigned m = off[segments];
    const bool in_lds = m <= (unsigned)kLdsKeys;
    // Global position of the j-th gathered key.
    auto locate = [&](unsigned j) {
        int lo = 0, hi = segments - 1;  // last segment with off <= j
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (off[mid] <= j) lo = mid;
            else hi = mid - 1;
        }
        return (size_t)lo * chunk + (j - off[lo]);
    };
    if (in_lds) {
        // Eight loads in flight per thread.
        for (unsigned j0 = t; j0 < m; j0 += 8 * 1024) {
            uint64_t v8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const unsigned j = j0 + 1024u * u;
                v8[u] = j < m ? list[locate(j)] : 0ull;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const unsigned j = j0 + 1024u * u;
                if (j < m) lk[j] = v8[u];
            }
        }
        __syncthreads();
    }
    // Visits every gathered key once, in no set order: from LDS, or read in
    // place with eight loads in flight per thread (a flat heatmap leaves
    // ~10^5 keys past the first digit, and one load at a time per thread
    // took ~0.2 ms over the passes below).
    auto scan = [&](auto &&visit) {
        if (in_lds) {
            for (unsigned j = t; j < m; j += 1024) visit(lk[j]);
            return;
        }
        for (unsigned j0 = t; j0 < m; j0 += 8 * 1024) {
            uint64_t v8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const unsigned j = j0 + 1024u * u;
                v8[u] = j < m ? list[locate(j)] : 0ull;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (j0 + 1024u * u < m) visit(v8[u]);
        }
    };
    for (int level = two ? 2 : 1; level < kLevels && !resolved; ++level) {
        const int shift = digit_shift(level), hi = shift + digit_width(level);
        const unsigned mask = (1u << digit_width(level)) - 1u;
        const unsigned long long group = prefix >> hi;
        for (int d = t; d < kDigitBins; d += 1024) lh[d] = 0u;
        __syncthreads();
        scan([&](uint64_t key) {
            if ((key >> hi) == group) atomicAdd(&lh[(unsigned)(key >> shift) & mask], 1u);
        });
        __syncthreads();
        pick_digit<1024>(lh, k, wsum, res);
        prefix |= (unsigned long long)res[0] << shift;
        k -= res[1];
        resolved = res[2] == k || level == kLevels - 1;
    }
    if (t == 0) count = 0u;
    __syncthreads();
    scan([&](uint64_t key) {
        if (key >= prefix) {
            const unsigned slot = atomicAdd(&count, 1u);
            if (slot < kTopSlots) s[slot] = key;  // exactly P keys by construction
        }
    });
    __syncthreads();
    // Descending order by rank (keys are unique): four threads per key count
    // the larger keys among a quarter of the P each.
    const int i = t >> 2, part = t & 3, quarter = (P + 3) / 4;
    const uint64_t mine = i < P ? s[i] : 0ull;
    unsigned rank = 0;
    for (int j = part * quarter; j < min(P, (part + 1) * quarter); ++j) rank += s[j] > mine;
    rank += __shfl_xor(rank, 1);
    rank += __shfl_xor(rank, 2);
    if (i < P && part == 0) top[rank] = mine;
}

// ------------------------------------------------ per-proposal fp32 helpers
// y[n] = b[n] + sum_k x[k] wt[k][n] for one row; x in LDS, wt [K][N] fp32.
// Thread t owns four adjacent columns (one float4 of each wt row) over one of
// S k-slices, so a thread keeps its K / S loads in flight at once; the slices
// meet in `red` (S * N floats of LDS).  Results land in y (LDS) and are
// visible after the caller's barrier.
template <int K, int N>
__device__ __forceinline__ void row_linear(const float *x, const float *__restrict__ wt,
                                           const float *__restrict__ b, float *y, float *red) {
    constexpr int G = N / 4, S = 256 / G, KS = K / S;
    static_assert(N % 4 == 0 && G <= 256 && K % S == 0, "row_linear shape");
    const int t = threadIdx.x;
    if (t < G * S) {
        const int c4 = t % G, sl = t / G;
        const float4 *w4 = reinterpret_cast<const float4 *>(wt) + (size_t)sl * KS * G + c4;
        const float *xs = x + sl * KS;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 16
        for (int k = 0; k < KS; ++k) {
            const float4 w = w4[(size_t)k * G];
            const float xv = xs[k];
            acc.x = fmaf(xv, w.x, acc.x);
            acc.y = fmaf(xv, w.y, acc.y);
            acc.z = fmaf(xv, w.z, acc.z);
            acc.w = fmaf(xv, w.w, acc.w);
        }
        *reinterpret_cast<float4 *>(&red[sl * N + 4 * c4]) = acc;
    }
    __syncthreads();
    for (int n = t; n < N; n += 256) {
        float a = b ? b[n] : 0.0f;
#pragma unroll
        for (int j = 0; j < S; ++j) a += red[j * N + n];
        y[n] = a;
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
    __shared__ float hid[kC], tmp[kC], pos[kC], out[3 * kC];
    __shared__ __attribute__((aligned(16))) float red[1024];
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
// scaled by 0.25 log2(e) and stored fp16 for the matrix cores.  The 32 lanes
// of a head take keys l, l + 32, ...; each lane keeps its keys' 16-wide K
// and V rows in flight together.
__global__ __launch_bounds__(256) void self_attention_kernel(
    Params prm, const float *__restrict__ qkv, int P, float *__restrict__ query,
    const float *__restrict__ query_pos, _Float16 *__restrict__ cross_q) {
    constexpr int kPerLane = (BF_MAX_PROPOSALS + 31) / 32;
    __shared__ __attribute__((aligned(16))) float q[kC];
    __shared__ float att[kC], upd[kC], x[kC], stat[4];
    __shared__ __attribute__((aligned(16))) float red[1024];
    __shared__ float part[kHeads][32][kHeadC + 1];
    const int p = blockIdx.x, t = threadIdx.x;
    const float *qs = qkv, *ks = qkv + (size_t)P * kC, *vs = qkv + (size_t)2 * P * kC;
    if (t < kC) q[t] = qs[p * kC + t];
    __syncthreads();
    const int h = t >> 5, l = t & 31;
    float4 qh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qh[i] = reinterpret_cast<const float4 *>(q + h * kHeadC)[i];
    float sc[kPerLane];
    float m = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int k = l + 32 * j;
        float dot = 0.0f;
        if (k < P) {
            const float4 *kr = reinterpret_cast<const float4 *>(ks + (size_t)k * kC + h * kHeadC);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 kv = kr[i];
                dot = fmaf(qh[i].x, kv.x, dot);
                dot = fmaf(qh[i].y, kv.y, dot);
                dot = fmaf(qh[i].z, kv.z, dot);
                dot = fmaf(qh[i].w, kv.w, dot);
            }
            dot *= 0.25f;
            m = fmaxf(m, dot);
        }
        sc[j] = dot;
    }
    m = group_max<32>(m);
    float sum = 0.0f;
    float acc[kHeadC];
#pragma unroll
    for (int d = 0; d < kHeadC; ++d) acc[d] = 0.0f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int k = l + 32 * j;
        if (k < P) {
            const float e = expf(sc[j] - m);
            sum += e;
            const float4 *vr = reinterpret_cast<const float4 *>(vs + (size_t)k * kC + h * kHeadC);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 vv = vr[i];
                acc[4 * i] = fmaf(e, vv.x, acc[4 * i]);
                acc[4 * i + 1] = fmaf(e, vv.y, acc[4 * i + 1]);
                acc[4 * i + 2] = fmaf(e, vv.z, acc[4 * i + 2]);
                acc[4 * i + 3] = fmaf(e, vv.w, acc[4 * i + 3]);
            }
        }
    }
    sum = group_sum<32>(sum);
#pragma unroll
    for (int d = 0; d < kHeadC; ++d) part[h][l][d] = acc[d];
    __syncthreads();
    {
        // Thread (h, d, half) adds 16 lanes' partials; the halves meet by shuffle.
        const int d = t & 15, half = (t >> 4) & 1;
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) a += part[h][16 * half + i][d];
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
    // The wave index is uniform: channel-indexed parameters load as scalars.
    const int t = threadIdx.x, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63, col = lane & 15, g = lane >> 4;
    const int key0 = blockIdx.x * kKeyTile;
    {
        const int r = lane, c0 = w * 32;
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
    // key_value tile: rows = keys (A = hidden), columns = channels
    // 32w .. 32w+31 (B = W2); a lane then holds four consecutive keys of one
    // channel, so the channel-major `shared` rows load as 16-byte vectors.
    {
        f32x4 acc[4][2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
            h8 b[2];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                b[ct] = *(const h8 *)&prm.cross_pos_w2[(32 * w + 16 * ct + col) * kC + 32 * ks + 8 * g];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const h8 a = *(const h8 *)&hid[(16 * rt + col) * kLdsRow + 32 * ks + 8 * g];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = mfma_16x16x32(a, b[ct], acc[rt][ct]);
            }
        }
        const bool vec = (keys & 3u) == 0;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int c = 32 * w + 16 * ct + col;
            const float bias = prm.cross_pos_b2[c];
            const float *row = shared + (size_t)c * keys;
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const unsigned k0 = (unsigned)(key0 + 16 * rt + 4 * g);
                float sv[4];
                if (vec && k0 + 4 <= keys) {
                    const float4 v = *reinterpret_cast<const float4 *>(row + k0);
                    sv[0] = v.x;
                    sv[1] = v.y;
                    sv[2] = v.z;
                    sv[3] = v.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) sv[j] = k0 + j < keys ? row[k0 + j] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    kv[(16 * rt + 4 * g + j) * kLdsRow + c] = (_Float16)(acc[rt][ct][j] + bias + sv[j]);
            }
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
// Workgroup (split s, head h), four waves over the split's 64-key steps
// s spw .. s spw + spw - 1; wave w owns query tiles [tile0(w), tile0(w + 1))
// (4 + 3 + 3 + 3 of the 13).  Partial results per (split, head, query):
// running max m (base 2), sum l and the unnormalised 16-wide output.
constexpr int kTilesPerWave = 4;

__device__ __forceinline__ int first_tile(int w) { return w == 0 ? 0 : 3 * w + 1; }

__global__ __launch_bounds__(256) void cross_attention_kernel(
    const _Float16 *__restrict__ cross_q, const _Float16 *__restrict__ kh,
    const _Float16 *__restrict__ vt, int keys, int keys64, int steps_per_wave,
    float *__restrict__ part_m, float *__restrict__ part_l, float *__restrict__ part_o) {
    const int s = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int w = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
    const int tile0 = first_tile(w), ntiles = first_tile(w + 1) - tile0;
    const int total_steps = keys64 / kStepKeys;

    h4 qf[kTilesPerWave];
    float m[kTilesPerWave], l[kTilesPerWave];
    f32x4 o[kTilesPerWave];
#pragma unroll
    for (int i = 0; i < kTilesPerWave; ++i) {
        const int qt = min(tile0 + i, kQTiles - 1);
        qf[i] = *(const h4 *)&cross_q[(qt * 16 + col) * kC + h * kHeadC + 4 * g];
        m[i] = kNegBig;
        l[i] = 0.0f;
        o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const _Float16 *kbase = kh + (size_t)h * keys64 * kHeadC;
    const _Float16 *vbase = vt + (size_t)h * kHeadC * keys64;
    // Row r of score MFMA 2a+b is key 32a + 8(r>>2) + 4b + (r&3): lane group g
    // then holds keys 32a + 8g .. +7, the k-slice of PV MFMA a's B operand.
    const int krow = 8 * (col >> 2) + (col & 3);

    for (int i = 0; i < steps_per_wave; ++i) {
        const int step = s * steps_per_wave + i;
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
        for (int qi = 0; qi < kTilesPerWave; ++qi) {
            if (qi >= ntiles) break;
            f32x4 sc[4];
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
                sc[i4] = mfma_16x16x16(kf[i4], qf[qi], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
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
            const float mn = fmaxf(m[qi], mx);
            const float alpha = __builtin_amdgcn_exp2f(m[qi] - mn);
            m[qi] = mn;
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
            l[qi] = l[qi] * alpha + ps;
            o[qi] *= alpha;
#pragma unroll
            for (int a = 0; a < 2; ++a) o[qi] = mfma_16x16x32(vf[a], pf[a], o[qi]);
        }
    }
    const size_t base = ((size_t)s * kHeads + h) * kPPad;
#pragma unroll
    for (int qi = 0; qi < kTilesPerWave; ++qi) {
        if (qi >= ntiles) break;
        float lt = l[qi] + __shfl_xor(l[qi], 16);
        lt += __shfl_xor(lt, 32);
        const int q = (tile0 + qi) * 16 + col;
        if (g == 0) {
            part_m[base + q] = m[qi];
            part_l[base + q] = lt;
        }
        *(f32x4 *)&part_o[(base + q) * kHeadC + 4 * g] = o[qi];
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
    __shared__ float att[kC], upd[kC], x[kC], ffn[2 * kC], hid[3 * kC], stat[4];
    __shared__ __attribute__((aligned(16))) float red[1024];
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
#pragma unroll 8
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

}  // namespace

struct bf_cuda_transfusion {
    size_t height, width, keys, proposals, resident_bytes;
    int keys64, steps_per_wave, splits, nms_tiles_x, nms_tiles_y, segments;
    unsigned chunk;
    unsigned char *params, *arena;
    Params prm;
    // Views into the arena.
    float *suppressed, *query, *query_pos, *qkv, *part_m, *part_l, *part_o;
    uint64_t *sort_keys, *selected, *top;
    unsigned *part_hist, *hist, *counts, *part_hist1, *hist1, *refined;
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
    // NMS tiles, and compaction segments of >= 2048 keys, fewer than
    // kMaxSegments (the finish scan also stores the total at off[segments]).
    d->nms_tiles_x = (int)((d->width + kNmsTile - 1) / kNmsTile);
    d->nms_tiles_y = (int)((d->height + kNmsTile - 1) / kNmsTile);
    const size_t tiles = (size_t)kClasses * d->nms_tiles_x * d->nms_tiles_y;
    size_t chunk = std::max<size_t>(2048, (cand + kMaxSegments - 2) / (kMaxSegments - 1));
    chunk = (chunk + 255) / 256 * 256;
    d->chunk = (unsigned)chunk;
    d->segments = (int)((cand + chunk - 1) / chunk);
    // Key splits of steps_per_wave 64-key steps: about 512 workgroups (two
    // per CU) over 8 heads, at most kMaxSplits splits.
    const int steps = d->keys64 / kStepKeys;
    int spw = std::max(1, (steps + 63) / 64);
    spw = std::max(spw, (steps + kMaxSplits - 1) / kMaxSplits);
    d->steps_per_wave = spw;
    d->splits = (steps + spw - 1) / spw;

    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~size_t(255);
        return at;
    };
    const size_t o_supp = take(cand * 4), o_keys = take(cand * 8);
    const size_t o_part = take(tiles * kDigitBins * 4), o_hist = take(kDigitBins * 4);
    const size_t o_counts = take((size_t)d->segments * 4), o_list = take(cand * 8),
                 o_top = take(kTopSlots * 8);
    const size_t o_part1 = take((size_t)d->segments * kDigitBins * 4),
                 o_hist1 = take(kDigitBins * 4), o_refined = take(4);
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
    d->part_hist = (unsigned *)(a + o_part);
    d->hist = (unsigned *)(a + o_hist);
    d->counts = (unsigned *)(a + o_counts);
    d->part_hist1 = (unsigned *)(a + o_part1);
    d->hist1 = (unsigned *)(a + o_hist1);
    d->refined = (unsigned *)(a + o_refined);
    d->selected = (uint64_t *)(a + o_list);
    d->top = (uint64_t *)(a + o_top);
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
    const int tiles = kClasses * d->nms_tiles_x * d->nms_tiles_y;
    suppress_kernel<<<tiles, 256, 0, s>>>(heatmap, d->suppressed, d->sort_keys, (int)d->height, W,
                                          keys, d->nms_tiles_x, d->nms_tiles_y, d->part_hist);
    key_kernel<<<d->keys64 / kKeyTile, 256, 0, s>>>(d->prm, shared, keys, W, d->keys64, d->kh, d->vt);
    hist_reduce_kernel<<<kDigitBins / 8, 256, 0, s>>>(d->part_hist, tiles, d->hist, nullptr);
    refine_kernel<<<d->segments, 256, 0, s>>>(d->sort_keys, cand, d->chunk, d->hist, P,
                                              d->part_hist1, d->refined);
    hist_reduce_kernel<<<kDigitBins / 8, 256, 0, s>>>(d->part_hist1, d->segments, d->hist1,
                                                      d->refined);
    compact_kernel<<<d->segments, 256, 0, s>>>(d->sort_keys, cand, d->chunk, d->hist, d->hist1,
                                               d->refined, P, d->selected, d->counts);
    finish_kernel<<<1, 1024, 0, s>>>(d->selected, d->counts, d->segments, d->chunk, d->hist,
                                     d->hist1, d->refined, P, d->top);
    query_kernel<<<P, 256, 0, s>>>(d->prm, d->top, d->suppressed, shared, keys, W, P,
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

int bfhip::transfusion_decode_launch(bf_cuda_transfusion *d, const bf_transfusion_raw_outputs *out,
                                     float threshold, void *stream_value,
                                     const bf_detections **device_detections, char *error,
                                     size_t cap) {
    if (!d || !device_detections || !std::isfinite(threshold) || !outputs_ok(out))
        return fail(error, cap, "invalid HIP detection decode contract");
    decode_kernel<<<1, 256, 0, reinterpret_cast<hipStream_t>(stream_value)>>>(
        *out, (int)d->proposals, threshold, d->detections);
    *device_detections = d->detections;
    return launch_ok(error, cap, "HIP detection decode launch");
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
