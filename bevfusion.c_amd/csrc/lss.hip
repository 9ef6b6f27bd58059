// Lift-splat-shoot pooling on gfx950 (drop-in for reference src/cuda_lss.cu).
//
// Plan route (deterministic, no floating-point atomics):
//   prepare:  every sample (b, n, d, y, x) -> BEV cell key (rank + b * cells;
//             samples outside the grid get the key B * cells, which sorts
//             last); a stable LSD radix sort of (key, sample index) pairs
//             lists each cell's samples in ascending sample order; a lower
//             bound per cell gives each cell's run, padded to whole quads;
//             the list of {context row, sample} and the pool schedule are
//             stored.
//   forward:  one prologue launch computes the per-pixel softmax statistics
//             {max, 1 / sum} and turns the context NCHW into rows
//             [B*N*H*W][C]; per BEV cell a group of lanes sums
//             expf(l - max) * inv * row over the cell's run in list order,
//             and each workgroup stores 64 consecutive cells of every channel
//             plane as coalesced rows; cells cut by a slice bound are added
//             up by a last pass.
// Stateless routes: the reference's atomic accumulation (one wave per pixel,
// softmax on the wave, atomicAdd per (channel, depth) sample).
//
// The metric-point -> cell map reproduces the CPU oracle bit for bit: the
// calibration transform is evaluated with floating-point contraction off and
// in the oracle's operation order (inverse by cofactors, row sums left to
// right), and the cell is trunc((p - min) / step) with IEEE division.
#include "bf_cuda.h"
#include "hip_common.h"


#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdlib>

using namespace bfhip;

namespace {

constexpr int kMaxDepth = 128;

struct Grid {
    float min[3], step[3];
    int cells[3];
};

Grid grid_of(const bf_lss_desc *d) {
    Grid g;
    for (int a = 0; a < 3; ++a) {
        g.min[a] = d->grid_minimum[a];
        g.step[a] = d->grid_step[a];
        g.cells[a] = (int)d->grid_cells[a];
    }
    return g;
}

bool checked_mul(size_t a, size_t b, size_t *r) {
    if (a && b > SIZE_MAX / a) return false;
    *r = a * b;
    return true;
}

// Contract of the reference (cuda_lss.cu:50-61) plus finite grid minima.
bool desc_ok(const bf_lss_desc *d) {
    if (!d || !d->batches || !d->cameras || !d->depth_bins || !d->feature_height ||
        !d->feature_width || !d->channels || d->depth_bins > (size_t)kMaxDepth ||
        d->batches > INT32_MAX || d->cameras > INT32_MAX || d->feature_height > INT32_MAX ||
        d->feature_width > INT32_MAX || d->channels > INT32_MAX)
        return false;
    for (int a = 0; a < 3; ++a)
        if (!d->grid_cells[a] || d->grid_cells[a] > INT32_MAX || !std::isfinite(d->grid_step[a]) ||
            !(d->grid_step[a] > 0.0f) || !std::isfinite(d->grid_minimum[a]))
            return false;
    return true;
}

struct Sizes {
    size_t samples, pixels, cams, cells, cell_count, bev_count, context_count;
};

// Element counts; every index the kernels form must fit in int.
bool sizes_of(const bf_lss_desc *d, Sizes *s) {
    size_t hw;
    if (!checked_mul(d->batches, d->cameras, &s->cams) ||
        !checked_mul(d->feature_height, d->feature_width, &hw) ||
        !checked_mul(s->cams, hw, &s->pixels) ||
        !checked_mul(s->pixels, d->depth_bins, &s->samples) ||
        !checked_mul(s->pixels, d->channels, &s->context_count) ||
        !checked_mul(d->grid_cells[0], d->grid_cells[1], &s->cells) ||
        !checked_mul(s->cells, d->grid_cells[2], &s->cells) ||
        !checked_mul(s->cells, d->batches, &s->cell_count) ||
        !checked_mul(s->cell_count, d->channels, &s->bev_count))
        return false;
    return s->samples <= INT_MAX && s->context_count <= INT_MAX && s->cell_count < INT_MAX &&
           s->bev_count <= INT_MAX;
}

// ------------------------------------------------------------------ kernels
// Cell rank of a metric point within its batch, -1 outside the grid
// (reference lss.c:182-191 / cuda_lss.cu:244-253).
__device__ __forceinline__ int point_rank(const float p[3], const Grid &g) {
    int c[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const float t = (p[a] - g.min[a]) / g.step[a];
        if (!isfinite(t) || t < -2147483648.0f || t >= 2147483648.0f) return -1;
        c[a] = (int)t;  // truncation toward zero, as torch .long()
        if (c[a] < 0 || c[a] >= g.cells[a]) return -1;
    }
    return (c[2] * g.cells[0] + c[0]) * g.cells[1] + c[1];
}

// Stateless ranks: the cell within the sample's batch, -1 outside.
__global__ __launch_bounds__(256) void geometry_rank_kernel(const float *__restrict__ geometry,
                                                            int *__restrict__ out, int samples,
                                                            Grid g) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= samples) return;
    const float p[3] = {geometry[3 * (size_t)s], geometry[3 * (size_t)s + 1],
                        geometry[3 * (size_t)s + 2]};
    out[s] = point_rank(p, g);
}

// Per-camera transform coefficients, 40 floats: [0,9) post-rotation^-1,
// [9,18) rotation * intrinsics^-1, [18,21) camera translation,
// [21,24) post translation, [24,33) extra rotation, [33,36) extra
// translation, [36] valid, [37] has extra rotation, [38] has extra
// translation (reference lss.c:72-130 operation order).
constexpr int kCalib = 40;

__device__ bool inverse3(const float *m, float *r) {
#pragma clang fp contract(off)
    const float a = m[4] * m[8] - m[5] * m[7], b = m[2] * m[7] - m[1] * m[8];
    const float c = m[1] * m[5] - m[2] * m[4], d = m[5] * m[6] - m[3] * m[8];
    const float e = m[0] * m[8] - m[2] * m[6], f = m[2] * m[3] - m[0] * m[5];
    const float g = m[3] * m[7] - m[4] * m[6], h = m[1] * m[6] - m[0] * m[7];
    const float k = m[0] * m[4] - m[1] * m[3];
    const float det = m[0] * a + m[1] * d + m[2] * g;
    if (!isfinite(det) || fabsf(det) <= FLT_MIN) return false;
    const float s = 1.0f / det;
    r[0] = a * s; r[1] = b * s; r[2] = c * s;
    r[3] = d * s; r[4] = e * s; r[5] = f * s;
    r[6] = g * s; r[7] = h * s; r[8] = k * s;
    return true;
}

__device__ void apply3(const float *m, const float *v, float *r) {
#pragma clang fp contract(off)
    for (int i = 0; i < 3; ++i) r[i] = m[3 * i] * v[0] + m[3 * i + 1] * v[1] + m[3 * i + 2] * v[2];
}

__global__ void calibration_kernel(const float *__restrict__ cam_rot,
                                   const float *__restrict__ cam_trans,
                                   const float *__restrict__ intrinsics,
                                   const float *__restrict__ post_rot,
                                   const float *__restrict__ post_trans,
                                   const float *__restrict__ extra_rot,
                                   const float *__restrict__ extra_trans, float *__restrict__ out,
                                   int cameras, int cams) {
#pragma clang fp contract(off)
    const int cam = blockIdx.x * blockDim.x + threadIdx.x;
    if (cam >= cams) return;
    const int b = cam / cameras;
    float *o = out + (size_t)cam * kCalib;
    float k_inv[9];
    const bool ok = inverse3(post_rot + 9 * cam, o) & inverse3(intrinsics + 9 * cam, k_inv);
    const float *r = cam_rot + 9 * cam;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < 3; ++k) acc += r[3 * i + k] * k_inv[3 * k + j];
            o[9 + 3 * i + j] = acc;
        }
    for (int i = 0; i < 3; ++i) {
        o[18 + i] = cam_trans[3 * cam + i];
        o[21 + i] = post_trans[3 * cam + i];
        o[33 + i] = extra_trans ? extra_trans[3 * b + i] : 0.0f;
    }
    for (int i = 0; i < 9; ++i) o[24 + i] = extra_rot ? extra_rot[9 * b + i] : 0.0f;
    o[36] = ok ? 1.0f : 0.0f;
    o[37] = extra_rot ? 1.0f : 0.0f;
    o[38] = extra_trans ? 1.0f : 0.0f;
}

// Key of frustum point `local` seen by camera `cam` with coefficient row o.
__device__ __forceinline__ int calibration_key(const float *__restrict__ frustum, const float *o,
                                               int local, int cam, int cams_per_batch, int cells,
                                               const Grid &g, int invalid) {
#pragma clang fp contract(off)
    if (o[36] == 0.0f) return invalid;
    const float *f = frustum + 3 * (size_t)local;
    const float p[3] = {f[0] - o[21], f[1] - o[22], f[2] - o[23]};
    float u[3], q[3], l[3], r[3];
    apply3(o, p, u);
    q[0] = u[0] * u[2];
    q[1] = u[1] * u[2];
    q[2] = u[2];
    apply3(o + 9, q, l);
    for (int i = 0; i < 3; ++i) l[i] += o[18 + i];
    if (o[37] != 0.0f) apply3(o + 24, l, r);
    else { r[0] = l[0]; r[1] = l[1]; r[2] = l[2]; }
    if (o[38] != 0.0f)
        for (int i = 0; i < 3; ++i) r[i] += o[33 + i];
    const int rank = point_rank(r, g);
    return rank >= 0 ? rank + (cam / cams_per_batch) * cells : invalid;
}

__global__ __launch_bounds__(256) void fill_float_kernel(float *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// starts[c] = first sorted position whose key is >= c (c in [0, cell_count]):
// a lower bound over the sorted keys, so empty cells get empty runs.
// Padded cell lists.  Every cell's run is padded to a multiple of 4 entries
// (kQuad) so that cell boundaries fall on quad boundaries; padding entries
// carry sample -1 (weight 0 on an all-zero context row).
constexpr int kQuad = 4;
constexpr int kStartThreads = 256;

__device__ __forceinline__ int lower_bound_key(const int *__restrict__ sorted_keys, int samples,
                                               int c) {
    int lo = 0, hi = samples;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sorted_keys[mid] < c) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Run start of every cell c <= cell_count (the last is the end of the valid
// samples) by lower bound in the sorted keys, and per workgroup of
// kStartThreads cells the sum of their padded run lengths.
__global__ __launch_bounds__(kStartThreads) void cell_starts_kernel(const int *__restrict__ sorted_keys,
                                                                   int samples,
                                                                   int *__restrict__ starts,
                                                                   int *__restrict__ block_sums,
                                                                   int cell_count) {
    __shared__ int s_start[kStartThreads + 1];
    __shared__ int wave_sums[kStartThreads / kWave];
    const int c0 = blockIdx.x * kStartThreads, t = threadIdx.x, c = c0 + t;
    const int st = lower_bound_key(sorted_keys, samples, min(c, cell_count));
    if (c <= cell_count) starts[c] = st;
    s_start[t] = st;
    if (t == kStartThreads - 1)
        s_start[kStartThreads] = lower_bound_key(sorted_keys, samples, min(c + 1, cell_count));
    __syncthreads();
    const int len = c < cell_count ? s_start[t + 1] - s_start[t] : 0;
    int v = (len + kQuad - 1) & ~(kQuad - 1);
    const int lane = t & (kWave - 1), wave = t / kWave;
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) wave_sums[wave] = v;
    __syncthreads();
    if (t == 0) {
        int sum = 0;
#pragma unroll
        for (int w = 0; w < kStartThreads / kWave; ++w) sum += wave_sums[w];
        block_sums[blockIdx.x] = sum;
    }
}

// Exclusive scan of the block sums in place (one workgroup).
__global__ __launch_bounds__(1024) void block_sums_scan_kernel(int *__restrict__ block_sums,
                                                               int blocks) {
    __shared__ int part[1024];
    int carry = 0;
    for (int b0 = 0; b0 < blocks; b0 += 1024) {
        const int b = b0 + (int)threadIdx.x;
        const int v = b < blocks ? block_sums[b] : 0;
        part[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int u = threadIdx.x >= (unsigned)off ? part[threadIdx.x - off] : 0;
            __syncthreads();
            part[threadIdx.x] += u;
            __syncthreads();
        }
        if (b < blocks) block_sums[b] = carry + part[threadIdx.x] - v;
        carry += part[1023];
        __syncthreads();
    }
}

// padded_starts[c] = sum of the padded run lengths of the cells before c.
__global__ __launch_bounds__(kStartThreads) void padded_starts_kernel(
    const int *__restrict__ starts, const int *__restrict__ block_prefix,
    int *__restrict__ padded_starts, int cell_count) {
    __shared__ int wave_sums[kStartThreads / kWave];
    const int c = blockIdx.x * kStartThreads + threadIdx.x;
    const int len = c < cell_count ? starts[c + 1] - starts[c] : 0;
    const int v = (len + kQuad - 1) & ~(kQuad - 1);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int u = __shfl_up(incl, o);
        if (lane >= o) incl += u;
    }
    if (lane == kWave - 1) wave_sums[wave] = incl;
    __syncthreads();
    int before = block_prefix[blockIdx.x];
#pragma unroll
    for (int w = 0; w < kStartThreads / kWave; ++w) before += w < wave ? wave_sums[w] : 0;
    if (c <= cell_count) padded_starts[c] = before + incl - v;
}

// Sorted position i of a valid sample -> its padded slot: {pixel, sample};
// the last sample of a cell also writes the cell's padding entries.
__global__ __launch_bounds__(256) void list_entries_kernel(const int *__restrict__ order,
                                                          const int *__restrict__ sorted_keys,
                                                          const int *__restrict__ starts,
                                                          const int *__restrict__ padded_starts,
                                                          int2 *__restrict__ list, int samples,
                                                          int cell_count, int depth_hw, int hw) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= samples) return;
    const int key = sorted_keys[i];
    if (key >= cell_count) return;
    const int s = order[i];
    const int cam = s / depth_hw, first = starts[key], slot = padded_starts[key] + (i - first);
    list[slot] = make_int2(cam * hw + (s - cam * depth_hw) % hw, s);
    if (i + 1 == starts[key + 1])
        for (int k = slot + 1; k < padded_starts[key + 1]; ++k) list[k] = make_int2(0, -1);
}

// Stable LSD radix sort of the (key, sample) pairs, keys < 2^end_bit, in
// passes of up to kDigitBits bits; pass 0 reads the samples as 0..n-1.  One
// pass, over tiles of kSortTile consecutive pairs:
//   digit_count_kernel    each tile's count of every digit -> counts[digit][tile];
//   digit_offsets_kernel  per digit, the exclusive scan of its counts over the
//                         tiles, and the digit's total;
//   digit_scatter_kernel  per tile, a stable sort by digit in LDS (splits on
//                         three digit bits at a time), then each pair goes to
//                         (pairs of smaller digits) + (its digit's pairs in
//                         earlier tiles) + (its rank among them in the tile).
// Every pass keeps equal digits in input order, so equal keys end in
// ascending sample order.  Integer counts only: the result is the unique
// stable order, the same on every run.
constexpr int kDigitBits = 9, kDigits = 1 << kDigitBits, kSplitBits = 3;
constexpr int kSortThreads = 256, kSortItems = 16, kSortTile = kSortThreads * kSortItems;
static_assert(kSplitBits == 3 && kSortTile < 65536, "eight 16-bit bucket counts in four words");
// LDS index of tile position i: one pad word per kSortItems, so the blocked
// reads (thread t, items t*kSortItems + j) fall in distinct banks.
__device__ __forceinline__ int sort_slot(int i) { return i + i / kSortItems; }
constexpr int kSortSlots = kSortTile + kSortTile / kSortItems;

__device__ __forceinline__ int digit_of(int key, int shift) {
    return (int)(((unsigned)key >> shift) & (kDigits - 1));
}

__global__ __launch_bounds__(kSortThreads) void digit_count_kernel(const int *__restrict__ keys,
                                                                  int n, int shift, int tiles,
                                                                  int *__restrict__ counts) {
    __shared__ int hist[kDigits];
    for (int d = threadIdx.x; d < kDigits; d += kSortThreads) hist[d] = 0;
    __syncthreads();
    const int base = blockIdx.x * kSortTile;
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = base + j * kSortThreads + (int)threadIdx.x;
        if (i < n) atomicAdd(&hist[digit_of(keys[i], shift)], 1);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kDigits; d += kSortThreads)
        counts[(size_t)d * tiles + blockIdx.x] = hist[d];
}

// Inclusive scan of one int per thread over the workgroup (kSortThreads);
// `total` receives the sum.  Ends with the workgroup synchronised.
__device__ __forceinline__ int block_inclusive_scan(int v, int *wave_sums, int *total) {
    constexpr int kWaves = kSortThreads / kWave;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    if (lane == kWave - 1) wave_sums[wave] = v;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int x = wave_sums[w];
        before += w < wave ? x : 0;
        all += x;
    }
    *total = all;
    __syncthreads();  // wave_sums may be reused
    return v + before;
}

// Inclusive scan of four words per thread over the workgroup (out[w]) and
// the four totals.  Ends with the workgroup synchronised.
__device__ __forceinline__ void block_scan4(const unsigned (&in)[4], unsigned (*wave_sums)[4],
                                            unsigned (&out)[4], unsigned (&total)[4]) {
    constexpr int kWaves = kSortThreads / kWave;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
    for (int w = 0; w < 4; ++w) out[w] = in[w];
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const unsigned u = __shfl_up(out[w], o);
            if (lane >= o) out[w] += u;
        }
    }
    if (lane == kWave - 1)
#pragma unroll
        for (int w = 0; w < 4; ++w) wave_sums[wave][w] = out[w];
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        unsigned before = 0, all = 0;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
            const unsigned x = wave_sums[q][w];
            before += q < wave ? x : 0u;
            all += x;
        }
        out[w] += before;
        total[w] = all;
    }
    __syncthreads();  // wave_sums may be reused
}

__global__ __launch_bounds__(kSortThreads) void digit_offsets_kernel(const int *__restrict__ counts,
                                                                    int tiles,
                                                                    int *__restrict__ offs,
                                                                    int *__restrict__ totals) {
    __shared__ int wave_sums[kSortThreads / kWave];
    const int d = blockIdx.x;
    const int *c = counts + (size_t)d * tiles;
    int *o = offs + (size_t)d * tiles;
    const int per = (tiles + kSortThreads - 1) / kSortThreads;
    const int lo = min(tiles, (int)threadIdx.x * per), hi = min(tiles, lo + per);
    int sum = 0;
    for (int i = lo; i < hi; ++i) sum += c[i];
    int total;
    int run = block_inclusive_scan(sum, wave_sums, &total) - sum;
    for (int i = lo; i < hi; ++i) {
        o[i] = run;
        run += c[i];
    }
    if (threadIdx.x == 0) totals[d] = total;
}

// vals_in == nullptr: the sample of pair i is i.
__global__ __launch_bounds__(kSortThreads) void digit_scatter_kernel(
    const int *__restrict__ keys_in, const int *__restrict__ vals_in, int n, int shift, int bits,
    int tiles, const int *__restrict__ offs, const int *__restrict__ totals,
    int *__restrict__ keys_out, int *__restrict__ vals_out) {
    __shared__ int K[kSortSlots], V[kSortSlots];
    __shared__ int first[kDigits];  // output position of the tile's first pair of each digit
    __shared__ int start[kDigits];  // tile position of that pair
    __shared__ int wave_sums[kSortThreads / kWave];
    __shared__ unsigned wave_sums4[kSortThreads / kWave][4];
    const int t = threadIdx.x, base = blockIdx.x * kSortTile, valid = min(kSortTile, n - base);

    // The tile in position order (coalesced loads, issued first so that they
    // overlap the offsets below); past n, key -1 (digit kDigits - 1, after
    // every real pair of the tile in a stable sort).
    int k[kSortItems], v[kSortItems];
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = j * kSortThreads + t;
        const bool live = i < valid;
        k[j] = live ? keys_in[base + i] : -1;
        v[j] = live ? (vals_in ? vals_in[base + i] : base + i) : 0;
    }
    // Pairs of smaller digits (exclusive scan of the totals, two digits per
    // thread) plus this digit's pairs in earlier tiles.
    {
        static_assert(kDigits == 2 * kSortThreads, "two digits per thread");
        const int a = totals[2 * t], b = totals[2 * t + 1];
        const int oa = offs[(size_t)(2 * t) * tiles + blockIdx.x];
        const int ob = offs[(size_t)(2 * t + 1) * tiles + blockIdx.x];
        int total;
        const int incl = block_inclusive_scan(a + b, wave_sums, &total);
        first[2 * t] = incl - a - b + oa;
        first[2 * t + 1] = incl - b + ob;
    }
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = j * kSortThreads + t;
        K[sort_slot(i)] = k[j];
        V[sort_slot(i)] = v[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        k[j] = K[sort_slot(t * kSortItems + j)];
        v[j] = V[sort_slot(t * kSortItems + j)];
    }
    // Stable splits on kSplitBits digit bits at a time: a pair's new tile
    // position is (pairs of smaller buckets) + (its bucket's pairs in earlier
    // threads) + (in this thread, before it).  The eight per-bucket counts
    // travel as 16-bit fields, two per 32-bit word (a tile has < 2^16 pairs,
    // so no field carries into the next).
    for (int b0 = 0; b0 < bits; b0 += kSplitBits) {
        const int mask = (1 << min(kSplitBits, bits - b0)) - 1;
        unsigned c[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < kSortItems; ++j) {
            const int bk = (digit_of(k[j], shift) >> b0) & mask;
            const unsigned one = 1u << (16 * (bk & 1));
#pragma unroll
            for (int w = 0; w < 4; ++w) c[w] += (bk >> 1) == w ? one : 0u;
        }
        // (the scan's barriers also order the previous split's LDS reads
        // before the stores below)
        unsigned tot[4], r[4];
        block_scan4(c, wave_sums4, r, tot);  // r: inclusive prefix per word
        // bucket bases: exclusive scan of the eight totals
        unsigned base = 0, packed[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const unsigned lo = tot[w] & 0xffffu, hi = tot[w] >> 16;
            packed[w] = base | ((base + lo) << 16);
            base += lo + hi;
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) r[w] = packed[w] + (r[w] - c[w]);
#pragma unroll
        for (int j = 0; j < kSortItems; ++j) {
            const int bk = (digit_of(k[j], shift) >> b0) & mask, sh = 16 * (bk & 1), wd = bk >> 1;
            unsigned word = r[0];
#pragma unroll
            for (int w = 1; w < 4; ++w) word = wd == w ? r[w] : word;
            const int pos = (int)((word >> sh) & 0xffffu);
#pragma unroll
            for (int w = 0; w < 4; ++w) r[w] += wd == w ? 1u << sh : 0u;
            K[sort_slot(pos)] = k[j];
            V[sort_slot(pos)] = v[j];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kSortItems; ++j) {
            k[j] = K[sort_slot(t * kSortItems + j)];
            v[j] = V[sort_slot(t * kSortItems + j)];
        }
    }
    // K / V hold the tile sorted by digit.  Each digit's first tile position,
    // then every real pair to its output slot (consecutive threads take
    // consecutive positions, so a digit's run is stored contiguously).
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int p = j * kSortThreads + t;
        const int d = digit_of(K[sort_slot(p)], shift);
        if (p < valid && (p == 0 || digit_of(K[sort_slot(p - 1)], shift) != d)) start[d] = p;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int p = j * kSortThreads + t;
        if (p >= valid) continue;
        const int key = K[sort_slot(p)], d = digit_of(key, shift);
        const int dst = first[d] + (p - start[d]);
        if ((unsigned)dst >= (unsigned)n) continue;  // unreachable for a sorted tile
        keys_out[dst] = key;
        vals_out[dst] = V[sort_slot(p)];
    }
}

// Plan keys, one workgroup of kKeyThreads per sort tile, with the tile's
// count of each first-pass digit (the sort's first count pass, fused).
constexpr int kKeyThreads = 1024, kKeyItems = kSortTile / kKeyThreads;
template <class KeyOf>
__device__ __forceinline__ void keys_tile(const KeyOf &key_of, int *__restrict__ keys, int samples,
                                          int tiles, int *__restrict__ counts, int *hist) {
    for (int d = threadIdx.x; d < kDigits; d += kKeyThreads) hist[d] = 0;
    __syncthreads();
    const int base = blockIdx.x * kSortTile;
    int key[kKeyItems];
#pragma unroll
    for (int j = 0; j < kKeyItems; ++j) {
        const int i = base + j * kKeyThreads + (int)threadIdx.x;
        key[j] = i < samples ? key_of(i) : 0;
    }
#pragma unroll
    for (int j = 0; j < kKeyItems; ++j) {
        const int i = base + j * kKeyThreads + (int)threadIdx.x;
        if (i < samples) {
            keys[i] = key[j];
            atomicAdd(&hist[digit_of(key[j], 0)], 1);
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kDigits; d += kKeyThreads)
        counts[(size_t)d * tiles + blockIdx.x] = hist[d];
}

__global__ __launch_bounds__(kKeyThreads) void geometry_keys_kernel(
    const float *__restrict__ geometry, int *__restrict__ keys, int samples, int per_batch,
    int cells, Grid g, int invalid, int tiles, int *__restrict__ counts) {
    __shared__ int hist[kDigits];
    keys_tile([&](int s) {
        const float p[3] = {geometry[3 * (size_t)s], geometry[3 * (size_t)s + 1],
                            geometry[3 * (size_t)s + 2]};
        const int r = point_rank(p, g);
        return r < 0 ? invalid : r + (s / per_batch) * cells;
    }, keys, samples, tiles, counts, hist);
}

// The calibration of the first kStageCams cameras the tile touches is read
// from LDS (a tile spans two cameras at production sizes); any further ones
// from global memory.
constexpr int kStageCams = 8;
__global__ __launch_bounds__(kKeyThreads) void calibration_keys_kernel(
    const float *__restrict__ frustum, const float *__restrict__ calib, int *__restrict__ keys,
    int samples, int cams, int depth_hw, int cams_per_batch, int cells, Grid g, int invalid,
    int tiles, int *__restrict__ counts) {
    __shared__ int hist[kDigits];
    __shared__ float stage[kStageCams * kCalib];
    const int cam0 = blockIdx.x * kSortTile / depth_hw, staged = min(kStageCams, cams - cam0);
    for (int i = threadIdx.x; i < staged * kCalib; i += kKeyThreads)
        stage[i] = calib[(size_t)cam0 * kCalib + i];
    // (keys_tile's first barrier publishes the stage)
    keys_tile([&](int s) {
        const int cam = s / depth_hw;
        const float *o = cam - cam0 < staged ? stage + (cam - cam0) * kCalib
                                             : calib + (size_t)cam * kCalib;
        return calibration_key(frustum, o, s - cam * depth_hw, cam, cams_per_batch, cells, g,
                               invalid);
    }, keys, samples, tiles, counts, hist);
}

// Pool schedule.  The BEV output is cut into tiles of kTileCells consecutive
// cells of one batch; a tile whose lists hold more than kSliceEntries entries
// is cut into equal slices, each pooled by its own workgroup.  A slice stores
// the cells whose lists begin inside it; a cell that runs on into the next
// slice leaves partial rows (the owner's and each later slice's share) that a
// second pass adds up in slice order.
constexpr int kTileCells = 64;
constexpr int kSliceEntries = 2048;
constexpr int kScheduleThreads = 1024;

// One workgroup: per tile, slice count; exclusive scans give each tile's
// first work item and its index among multi-slice tiles.  sched layout:
// slices[tiles], slice_base[tiles + 1], multi_base[tiles + 1].  Work list:
// item slice_base[t] + k = (tile t, slice k); multi-slice tiles listed in
// tile order.
__global__ __launch_bounds__(kScheduleThreads) void schedule_kernel(const int *__restrict__ starts,
                                                                   int *__restrict__ sched,
                                                                   int2 *__restrict__ work,
                                                                   int *__restrict__ multi,
                                                                   int tiles, int tiles_per_batch,
                                                                   int cells) {
    __shared__ int part[2][kScheduleThreads];
    int *slices = sched, *slice_base = sched + tiles, *multi_base = slice_base + tiles + 1;
    const int t = threadIdx.x, per = (tiles + kScheduleThreads - 1) / kScheduleThreads;
    const int lo = min(tiles, t * per), hi = min(tiles, lo + per);
    int sum[2] = {0, 0};
    for (int i = lo; i < hi; ++i) {
        const int b = i / tiles_per_batch, j0 = (i - b * tiles_per_batch) * kTileCells;
        const int first = b * cells + j0, last = b * cells + min(cells, j0 + kTileCells);
        const int entries = starts[last] - starts[first];
        const int ns = max(1, (entries + kSliceEntries - 1) / kSliceEntries);
        slices[i] = ns;
        sum[0] += ns;
        sum[1] += ns > 1;
    }
    for (int q = 0; q < 2; ++q) part[q][t] = sum[q];
    __syncthreads();
    for (int off = 1; off < kScheduleThreads; off <<= 1) {  // inclusive scans
        int v[2];
        for (int q = 0; q < 2; ++q) v[q] = t >= off ? part[q][t - off] : 0;
        __syncthreads();
        for (int q = 0; q < 2; ++q) part[q][t] += v[q];
        __syncthreads();
    }
    int run[2];
    for (int q = 0; q < 2; ++q) run[q] = part[q][t] - sum[q];
    for (int i = lo; i < hi; ++i) {
        const int ns = slices[i];
        slice_base[i] = run[0];
        multi_base[i] = run[1];
        for (int k = 0; k < ns; ++k) work[run[0] + k] = make_int2(i, k);
        if (ns > 1) multi[run[1]] = i;
        run[0] += ns;
        run[1] += ns > 1;
    }
    if (t == kScheduleThreads - 1) {
        slice_base[tiles] = part[0][t];
        multi_base[tiles] = part[1][t];
    }
}

// Entry bound k of a tile's ns slices: whole quads of [start, end).
__device__ __forceinline__ int slice_bound(int start, int end, int k, int ns) {
    const int Q0 = start / kQuad, Qn = end / kQuad - Q0;
    return kQuad * (Q0 + (int)((long long)Qn * k / ns));
}

// Forward prologue, one launch: workgroups [0, softmax_blocks) compute the
// per-pixel depth softmax statistics, the rest turn the context NCHW into
// rows.
//
// Statistics {max, 1 / sum exp(l - max)} (reference lss.c:144-158 operation
// order: float max, double sum of expf(l - max), the inverse rounded to
// float); a sample's probability is then expf(l - max) * inv.  Workgroup =
// 32 pixels x 8 depth slices of kSlice bins.
constexpr int kSoftmaxPixels = 32, kSlices = 8, kSlice = kMaxDepth / kSlices;
// Context rows: workgroup = 64 pixels of one camera; channels in chunks of
// up to kRowChunk through an LDS tile [channel][pixel] (65-float pitch), so
// both the plane reads and the row writes are contiguous runs.
constexpr int kRowPixels = 64, kRowChunk = 128, kRowPitch = kRowPixels + 1;

__device__ __forceinline__ void softmax_stats_block(const float *__restrict__ logits,
                                                    float2 *__restrict__ stats, int pixels,
                                                    int depths, int hw, int block, float *smem) {
    float(*part_max)[kSoftmaxPixels] = reinterpret_cast<float(*)[kSoftmaxPixels]>(smem);
    double(*part_sum)[kSoftmaxPixels] =
        reinterpret_cast<double(*)[kSoftmaxPixels]>(smem + kSlices * kSoftmaxPixels);
    const int lane = threadIdx.x & (kSoftmaxPixels - 1), slice = threadIdx.x / kSoftmaxPixels;
    const int px = block * kSoftmaxPixels + lane;
    const bool live = px < pixels;
    const int cam = live ? px / hw : 0, p = live ? px - cam * hw : 0;
    const size_t base = (size_t)cam * depths * hw + p;
    const int d0 = slice * kSlice;
    float v[kSlice];
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < kSlice; ++k) {
        const int d = d0 + k;
        v[k] = (live && d < depths) ? logits[base + (size_t)d * hw] : -FLT_MAX;
        m = fmaxf(m, v[k]);
    }
    part_max[slice][lane] = m;
    __syncthreads();
    m = part_max[0][lane];
#pragma unroll
    for (int j = 1; j < kSlices; ++j) m = fmaxf(m, part_max[j][lane]);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < kSlice; ++k)
        if (d0 + k < depths) sum += expf(v[k] - m);
    part_sum[slice][lane] = sum;
    __syncthreads();
    if (slice != 0 || !live) return;
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < kSlices; ++j) total += part_sum[j][lane];
    stats[px] = make_float2(m, (float)(1.0 / total));
}

__device__ __forceinline__ void context_rows_block(const float *__restrict__ ctx,
                                                   float *__restrict__ rows, int C, int hw,
                                                   int groups, int block, float *tile) {
    const int cam = block / groups, p0 = (block - cam * groups) * kRowPixels;
    const int np = min(kRowPixels, hw - p0), t = threadIdx.x;
    const float *src = ctx + (size_t)cam * C * hw + p0;
    float *dst = rows + ((size_t)cam * hw + p0) * C;
    for (int c0 = 0; c0 < C; c0 += kRowChunk) {
        const int cc = min(kRowChunk, C - c0);
        constexpr int kLoads = kRowChunk * kRowPixels / 256;
        float v[kLoads];
        const int pl = t & (kRowPixels - 1), cl = t / kRowPixels;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int c = cl + 4 * i;
            v[i] = (c < cc && pl < np) ? src[(size_t)(c0 + c) * hw + pl] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            if (cl + 4 * i < cc) tile[(cl + 4 * i) * kRowPitch + pl] = v[i];
        __syncthreads();
        // row-major [np][cc] run of the output (contiguous when cc == C)
        for (int o = t; o < np * cc; o += 256) {
            const int p = o / cc, c = o - p * cc;
            dst[(size_t)p * C + c0 + c] = tile[c * kRowPitch + p];
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void forward_prologue_kernel(
    const float *__restrict__ logits, float2 *__restrict__ stats, const float *__restrict__ ctx,
    float *__restrict__ rows, int pixels, int depths, int hw, int C, int softmax_blocks,
    int row_groups) {
    __shared__ __align__(16) float smem[kRowChunk * kRowPitch];
    static_assert(kSlices * kSoftmaxPixels * (sizeof(float) + sizeof(double)) <= sizeof(smem),
                  "softmax partials fit the tile");
    if ((int)blockIdx.x < softmax_blocks)
        softmax_stats_block(logits, stats, pixels, depths, hw, blockIdx.x, smem);
    else
        context_rows_block(ctx, rows, C, hw, row_groups, blockIdx.x - softmax_blocks, smem);
}

// ------------------------------------------------------------------ pooling
// Work item = (tile, slice): quads [e0, e1) of the tile's padded list.  The
// workgroup's lane groups (L lanes x VW channels each) split [e0, e1) evenly
// in quads and walk their share in list order, ROUND entries at a time (all
// their context rows in flight together; ROUND = 16 when every group has at
// least 16 lanes, else 4).  Lane u of a group prepares entry
// u of the round (its probability and row offset) and the group reads them by
// lane permutes.  A cell's sum is closed at each list boundary (a quad
// boundary) into an LDS tile [channel][cell]; a cell that began in an earlier
// group is continued as a carry, added to the owner's sum in group order.
// Single-slice tiles store the tile; slices of larger tiles store partial
// tiles for the combine pass.  Every sum runs in a fixed order, so results
// are bit-identical from run to run.
constexpr int kRoundWide = 16;

struct PoolArgs {
    const int2 *list;          // padded sorted {pixel, sample}
    const float *logits;       // [B,N,D,H,W]
    const float2 *stats;       // per pixel {max, inv}
    const float *rows;         // [B*N*H*W + 1][C]; the last row is zero
    const int *starts;         // padded list start per cell [cell_count + 1]
    const int *sched;          // schedule_kernel layout
    const int2 *work;          // (tile, slice)
    float *scratch;            // partial rows of multi-slice tiles: [work item][2][C]
    float *bev;
    int cells, tiles, tiles_per_batch, C, passes, chunk_max, zero_row;
    unsigned row_bytes, rows_bytes;  // C * 4; (B*N*H*W + 1) * C * 4 < 2^32
};

template <int VW>
__device__ __forceinline__ void close_cell(float *tile, float *carry, int *carry_cell, bool is_carry,
                                           int t, const float *acc, int g, int L, int lig,
                                           bool live) {
    if (is_carry) {
#pragma unroll
        for (int j = 0; j < VW; ++j) carry[(g * L + lig) * VW + j] = acc[j];
        if (lig == 0) carry_cell[g] = t;
    } else if (live) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
            const int c = VW * lig + j;
            tile[c * kTileCells + (t ^ (c & 63))] = acc[j];
        }
    }
}

template <int VW, int ROUND>
__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
    static_assert(ROUND % kQuad == 0, "rounds are whole quads");
    extern __shared__ float tile[];  // [chunk_max][64], cell XOR-swizzled by channel
    __shared__ int s_start[kTileCells + 1];
    __shared__ int carry_cell[256];
    __shared__ float carry[256 * VW];
    const int *slices = a.sched, *slice_base = a.sched + a.tiles;
    if ((int)blockIdx.x >= slice_base[a.tiles]) return;
    const int2 wk = a.work[blockIdx.x];
    const int tile_id = wk.x, k = wk.y;
    const int b = tile_id / a.tiles_per_batch, j0 = (tile_id - b * a.tiles_per_batch) * kTileCells;
    const int tile_cells = min(kTileCells, a.cells - j0);
    const int oc0 = b * a.cells + j0;
    if ((int)threadIdx.x <= tile_cells) s_start[threadIdx.x] = a.starts[oc0 + threadIdx.x];
    __syncthreads();
    const int ns = slices[tile_id];
    const int e0 = slice_bound(s_start[0], s_start[tile_cells], k, ns);
    const int e1 = slice_bound(s_start[0], s_start[tile_cells], k + 1, ns);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int pass = 0; pass < a.passes; ++pass) {
        const int c0 = pass * a.chunk_max, chunk = min(a.chunk_max, a.C - c0);
        // L >= ROUND lanes per group: lane u < ROUND prepares entry u
        const int L = max(ROUND, (chunk + VW - 1) / VW), G = 64 / L, NG = 4 * G;
        constexpr int E = ROUND;
        const int gi = lane / L, lig = lane - gi * L, gbase = gi * L, g = wave * G + gi;
        const bool live = VW * lig < chunk;  // this lane owns channels
        for (int i = threadIdx.x; i < chunk * kTileCells; i += 256) tile[i] = 0.0f;
        carry_cell[threadIdx.x] = -1;
        __syncthreads();
        const int nq = (e1 - e0) / kQuad;
        const int g_lo = e0 + kQuad * (int)((long long)nq * g / NG);
        const int g_hi = e0 + kQuad * (int)((long long)nq * (g + 1) / NG);
        if (gi < G && g_lo < g_hi) {
            // context rows through a buffer resource: 32-bit byte offsets
            const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(a.rows), 0, (int)a.rows_bytes, 0x00020000);
            const unsigned ch_bytes = live ? 4u * (unsigned)(c0 + VW * lig) : 0u;
            // the cell holding entry g_lo: last t with s_start[t] <= g_lo
            int lo_t = 0, hi_t = tile_cells;
            while (hi_t - lo_t > 1) {
                const int mid = (lo_t + hi_t) >> 1;
                if (s_start[mid] <= g_lo) lo_t = mid;
                else hi_t = mid;
            }
            int t = lo_t, boundary = s_start[t + 1];
            bool is_carry = g_lo > max(s_start[t], e0);
            float acc[VW];
#pragma unroll
            for (int j = 0; j < VW; ++j) acc[j] = 0.0f;
            // Rounds in flight: entries of round r + 2, softmax inputs of
            // round r + 1, context rows of round r.
            int2 e_next = make_int2(0, -1), e_cur = make_int2(0, -1);
            float2 st = make_float2(0.0f, 0.0f);
            float lg = 0.0f;
            if (lig < E && g_lo + lig < g_hi) e_cur = a.list[g_lo + lig];
            if (lig < E && g_lo + E + lig < g_hi) e_next = a.list[g_lo + E + lig];
            if (e_cur.y >= 0) {
                st = a.stats[e_cur.x];
                lg = a.logits[e_cur.y];
            }
            for (int base = g_lo; base < g_hi; base += E) {
                const int n = min(E, g_hi - base);  // whole quads
                const int2 cur = e_cur;
                const float2 cst = st;
                const float clg = lg;
                e_cur = e_next;
                e_next = make_int2(0, -1);
                if (lig < E && base + 2 * E + lig < g_hi) e_next = a.list[base + 2 * E + lig];
                if (e_cur.y >= 0) {
                    st = a.stats[e_cur.x];
                    lg = a.logits[e_cur.y];
                }
                // entry of lane u: probability and row offset (zero row for padding)
                const bool real = cur.y >= 0;
                const float pr = real ? expf(clg - cst.x) * cst.y : 0.0f;
                const unsigned off = (unsigned)(real ? cur.x : a.zero_row) * a.row_bytes;
                float v[ROUND][VW], w[ROUND];
#pragma unroll
                for (int u = 0; u < ROUND; ++u) {
                    const unsigned pk = (unsigned)__shfl((int)off, gbase + u) + ch_bytes;
                    w[u] = __shfl(pr, gbase + u);
                    if constexpr (VW == 4) {
                        const auto q = __builtin_amdgcn_raw_buffer_load_b128(rows, pk, 0, 0);
#pragma unroll
                        for (int j = 0; j < VW; ++j) v[u][j] = __uint_as_float(q[j]);
                    } else {
                        v[u][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rows, pk, 0, 0));
                    }
                }
#pragma unroll
                for (int q = 0; q < ROUND / kQuad; ++q) {
                    if (kQuad * q < n) {
                        if (base + kQuad * q == boundary) {
                            close_cell<VW>(tile, carry, carry_cell, is_carry, t, acc, g, L, lig, live);
                            is_carry = false;
#pragma unroll
                            for (int j = 0; j < VW; ++j) acc[j] = 0.0f;
                            do {
                                ++t;
                                boundary = s_start[t + 1];
                            } while (boundary <= base + kQuad * q);
                        }
#pragma unroll
                        for (int u = kQuad * q; u < kQuad * (q + 1); ++u)
#pragma unroll
                            for (int j = 0; j < VW; ++j) acc[j] += w[u] * v[u][j];
                    }
                }
            }
            close_cell<VW>(tile, carry, carry_cell, is_carry, t, acc, g, L, lig, live);
        }
        __syncthreads();
        if ((int)threadIdx.x < chunk) {  // carries, in group order
            const int c = threadIdx.x, lg = c / VW, jj = c - lg * VW;
            for (int q = 0; q < NG; ++q) {
                const int t = carry_cell[q];
                if (t >= 0) tile[c * kTileCells + (t ^ (c & 63))] += carry[(q * L + lg) * VW + jj];
            }
        }
        __syncthreads();
        // Cells whose lists begin in [e0, e1) (the last slice: every cell from
        // e0 on) are this slice's; one that runs past e1 is stored as its
        // partial row 1, and a cell begun before e0 that runs into the slice
        // as its partial row 0, for the combine pass.
        const int j = threadIdx.x & 63;
        const int st = j < tile_cells ? s_start[j] : 0, en = j < tile_cells ? s_start[j + 1] : 0;
        const bool owned = j < tile_cells && st >= e0 && (k == ns - 1 || st < e1);
        const bool tail = owned && en > e1, head = !owned && st < e0 && en > e0;
        float *out = a.bev + ((size_t)b * a.C + c0) * a.cells + j0;
        const size_t row = (size_t)(slice_base[tile_id] + k) * 2 + (tail ? 1 : 0);
        float *part = a.scratch + row * a.C + c0;
        for (int c = threadIdx.x >> 6; c < chunk; c += 4) {
            const float v = tile[c * kTileCells + (j ^ (c & 63))];
            if (tail || head) part[c] = v;
            else if (owned) out[(size_t)c * a.cells + j] = v;
        }
        __syncthreads();
    }
}

// The cells of multi-slice tiles that run across a slice bound: the owner's
// partial row plus each later slice's, in slice order.
__global__ __launch_bounds__(256) void combine_kernel(PoolArgs a, const int *__restrict__ multi) {
    const int *slices = a.sched, *slice_base = a.sched + a.tiles;
    const int *multi_base = slice_base + a.tiles + 1;
    if ((int)blockIdx.x >= multi_base[a.tiles]) return;
    const int tile_id = multi[blockIdx.x], ns = slices[tile_id], w0 = slice_base[tile_id];
    const int b = tile_id / a.tiles_per_batch, j0 = (tile_id - b * a.tiles_per_batch) * kTileCells;
    const int tile_cells = min(kTileCells, a.cells - j0);
    const int *start = a.starts + (size_t)b * a.cells + j0;
    const int first = start[0], last = start[tile_cells];
    for (int k = 0; k + 1 < ns; ++k) {
        const int e0 = slice_bound(first, last, k, ns), e1 = slice_bound(first, last, k + 1, ns);
        // the cell holding entry e1 - 1: last t with start[t] <= e1 - 1
        int lo = 0, hi = tile_cells;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (start[mid] <= e1 - 1) lo = mid;
            else hi = mid;
        }
        const int t = lo, end = start[t + 1];
        if (start[t] < e0 || end <= e1) continue;  // not slice k's, or ends at the bound
        float *out = a.bev + (size_t)b * a.C * a.cells + j0 + t;
        for (int c = threadIdx.x; c < a.C; c += 256) {
            float sum = a.scratch[((size_t)(w0 + k) * 2 + 1) * a.C + c];
            for (int m = k + 1; m < ns; ++m) {
                sum += a.scratch[(size_t)(w0 + m) * 2 * a.C + c];
                if (end <= slice_bound(first, last, m + 1, ns)) break;
            }
            out[(size_t)c * a.cells] = sum;
        }
    }
}

// Stateless route: one wave per pixel; lanes own depth bins for the softmax
// and channels for the scatter (float atomics, as the reference).
__global__ __launch_bounds__(64) void lift_pool_atomic_kernel(
    const float *__restrict__ logits, const float *__restrict__ ctx,
    const float *__restrict__ geometry, const int *__restrict__ ranks, float *__restrict__ bev,
    int cameras, int depths, int hw, int C, int cells, Grid g) {
    __shared__ float prob[kMaxDepth];
    __shared__ int rank[kMaxDepth];
    const int px = blockIdx.x, lane = threadIdx.x;
    const int cam = px / hw, p = px - cam * hw, b = cam / cameras;
    const float *col = logits + (size_t)cam * depths * hw + p;
    float v[2], m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = lane + 64 * k;
        v[k] = d < depths ? col[(size_t)d * hw] : -FLT_MAX;
        m = fmaxf(m, v[k]);
    }
    m = group_max<64>(m);
    float e[2], sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = lane + 64 * k;
        e[k] = d < depths ? expf(v[k] - m) : 0.0f;
        sum += e[k];
    }
    const float inv = 1.0f / group_sum<64>(sum);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = lane + 64 * k;
        if (d >= depths) continue;
        const size_t s = ((size_t)cam * depths + d) * hw + p;
        prob[d] = e[k] * inv;
        if (ranks) {
            const int r = ranks[s];  // caller-supplied: anything outside [0, cells) is skipped
            rank[d] = (unsigned)r < (unsigned)cells ? r : -1;
        } else {
            const float q[3] = {geometry[3 * s], geometry[3 * s + 1], geometry[3 * s + 2]};
            rank[d] = point_rank(q, g);
        }
    }
    __syncthreads();
    for (int c = lane; c < C; c += 64) {
        const float f = ctx[((size_t)cam * C + c) * hw + p];
        float *plane = bev + ((size_t)b * C + c) * cells;
        for (int d = 0; d < depths; ++d)
            if (rank[d] >= 0) atomicAdd(plane + rank[d], prob[d] * f);
    }
}

inline unsigned blocks_for(size_t n, int per = 256) { return (unsigned)((n + per - 1) / per); }

// Scratch of the pair sort: the ping-pong keys and samples, the per-tile
// digit counts and offsets, the digit totals.
size_t sort_tmp_bytes(size_t n) {
    const size_t tiles = (n + kSortTile - 1) / kSortTile;
    return (2 * n + 2 * (size_t)kDigits * tiles + kDigits) * sizeof(int);
}

int fail_contract(char *error, size_t cap, const char *what) { return fail(error, cap, "%s", what); }

int stateless_pool(const float *logits, const float *ctx, const float *geometry, const int *ranks,
                   float *bev, const bf_lss_desc *d, void *stream_value, char *error, size_t cap) {
    Sizes z;
    if (!sizes_of(d, &z)) return fail(error, cap, "HIP LSS size overflow");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    hipLaunchKernelGGL(fill_float_kernel, dim3(blocks_for(z.bev_count)), dim3(256), 0, s, bev,
                       (int)z.bev_count);
    hipLaunchKernelGGL(lift_pool_atomic_kernel, dim3((unsigned)z.pixels), dim3(64), 0, s, logits,
                       ctx, geometry, ranks, bev, (int)d->cameras, (int)d->depth_bins,
                       (int)(d->feature_height * d->feature_width), (int)d->channels,
                       (int)z.cells, grid_of(d));
    return launch_ok(error, cap, "HIP LSS launch");
}

}  // namespace

// Plan memory (one arena).  keys / sorted keys / order are used only while
// preparing; the forward reads the padded list, its starts and the schedule.
struct bf_cuda_lss_plan {
    bf_lss_desc desc;
    Sizes z;
    int prepared;
    unsigned end_bit;  // sort key width: cell_count (the invalid key) is below 2^end_bit
    int tiles, tiles_per_batch, max_work, max_multi, vw, chunk_max, passes, round;
    size_t list_capacity;  // samples + (kQuad - 1) * cells: every cell padded to whole quads
    int *keys, *sorted_keys, *order, *starts, *padded_starts, *sched, *multi;
    int2 *list, *work;
    float2 *stats;
    float *rows, *calib, *scratch;
    void *tmp;  // pair-sort scratch, then the padded-start block sums
    size_t tmp_bytes;
    void *arena;
    size_t resident_bytes;
};

extern "C" int bf_cuda_available(char *error, size_t cap) {
    int count = 0;
    const hipError_t st = hipGetDeviceCount(&count);
    if (st != hipSuccess) return hip_ok(st, error, cap, "HIP device query");
    if (!count) return fail(error, cap, "no HIP device available");
    return 1;
}

extern "C" int bf_cuda_lss_lift_pool_f32(const float *logits, const float *context,
                                         const float *geometry, float *bev,
                                         const bf_lss_desc *d, void *stream, char *error,
                                         size_t cap) {
    if (!logits || !context || !geometry || !bev || !desc_ok(d))
        return fail_contract(error, cap, "invalid HIP LSS contract");
    return stateless_pool(logits, context, geometry, nullptr, bev, d, stream, error, cap);
}

extern "C" int bf_cuda_lss_geometry_to_ranks_f32(const float *geometry, int *ranks,
                                                 const bf_lss_desc *d, void *stream,
                                                 char *error, size_t cap) {
    if (!geometry || !ranks || !desc_ok(d))
        return fail_contract(error, cap, "invalid HIP LSS rank contract");
    Sizes z;
    if (!sizes_of(d, &z)) return fail(error, cap, "HIP LSS rank size overflow");
    hipLaunchKernelGGL(geometry_rank_kernel, dim3(blocks_for(z.samples)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), geometry, ranks, (int)z.samples,
                       grid_of(d));
    return launch_ok(error, cap, "HIP LSS rank launch");
}

extern "C" int bf_cuda_lss_lift_pool_ranks_f32(const float *logits, const float *context,
                                               const int *ranks, float *bev,
                                               const bf_lss_desc *d, void *stream, char *error,
                                               size_t cap) {
    if (!logits || !context || !ranks || !bev || !desc_ok(d))
        return fail_contract(error, cap, "invalid HIP LSS ranked contract");
    return stateless_pool(logits, context, nullptr, ranks, bev, d, stream, error, cap);
}

extern "C" void bf_cuda_lss_plan_destroy(bf_cuda_lss_plan *plan) {
    if (!plan) return;
    if (plan->arena) (void)hipFree(plan->arena);
    std::free(plan);
}

extern "C" int bf_cuda_lss_plan_create(const bf_lss_desc *d, bf_cuda_lss_plan **out,
                                       char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!out || !desc_ok(d)) return fail_contract(error, cap, "invalid HIP LSS plan contract");
    Sizes z;
    if (!sizes_of(d, &z)) return fail(error, cap, "HIP LSS plan size overflow");
    bf_cuda_lss_plan *p = (bf_cuda_lss_plan *)std::calloc(1, sizeof(*p));
    if (!p) return fail(error, cap, "HIP LSS plan host allocation failed");
    p->desc = *d;
    p->z = z;
    p->end_bit = 1;
    while (p->end_bit < 31 && (size_t(1) << p->end_bit) <= z.cell_count) ++p->end_bit;
    p->list_capacity = z.samples + (size_t)(kQuad - 1) * z.cell_count;
    // the pool addresses the context rows (plus a zero row) with 32-bit
    // buffer offsets
    if (p->list_capacity > (size_t)INT_MAX || (z.context_count + d->channels) * 4 > (size_t)INT_MAX) {
        bf_cuda_lss_plan_destroy(p);
        return fail(error, cap, "HIP LSS plan size overflow");
    }
    // the sort's scratch, then (reused) the block sums of the padded starts
    const size_t start_blocks = (z.cell_count + kStartThreads) / kStartThreads;
    p->tmp_bytes = std::max(sort_tmp_bytes(z.samples), start_blocks * sizeof(int));
    p->tiles_per_batch = (int)((z.cells + kTileCells - 1) / kTileCells);
    p->tiles = p->tiles_per_batch * (int)d->batches;
    p->max_multi = (int)std::max<size_t>(1, (p->list_capacity + kSliceEntries - 1) / kSliceEntries);
    p->max_work = p->tiles + p->max_multi;
    p->vw = d->channels % 4 == 0 ? 4 : 1;
    p->chunk_max = (int)std::min<size_t>(d->channels, p->vw == 4 ? 128 : 64);
    p->passes = (int)((d->channels + p->chunk_max - 1) / p->chunk_max);
    // wide rounds need >= 16 lanes per group in every channel pass
    const int last_chunk = (int)d->channels - (p->passes - 1) * p->chunk_max;
    p->round = (last_chunk + p->vw - 1) / p->vw >= kRoundWide ? kRoundWide : kQuad;
    // keys + sorted keys, order [samples]; starts, padded starts [cells + 1];
    // padded list; softmax stats [pixels]; context rows + one zero row;
    // calibration; schedule; work list; multi-slice tiles; partial rows;
    // sort / scan scratch.
    const size_t scratch_floats = (size_t)2 * p->max_work * d->channels;
    const size_t parts[13] = {z.samples * 8, z.samples * 4, (z.cell_count + 1) * 4,
                              (z.cell_count + 1) * 4, p->list_capacity * 8, z.pixels * 8,
                              (z.context_count + d->channels) * 4, z.cams * kCalib * 4,
                              ((size_t)3 * p->tiles + 2) * 4, (size_t)p->max_work * 8,
                              (size_t)p->max_multi * 4, scratch_floats * 4, p->tmp_bytes};
    size_t offs[13], total = 0;
    for (int i = 0; i < 13; ++i) {
        offs[i] = total;
        total += (parts[i] + 255) & ~size_t(255);
    }
    if (!hip_ok(hipMalloc(&p->arena, total), error, cap, "allocate HIP LSS plan")) {
        bf_cuda_lss_plan_destroy(p);
        return 0;
    }
    unsigned char *a = (unsigned char *)p->arena;
    p->keys = (int *)(a + offs[0]);
    p->sorted_keys = p->keys + z.samples;
    p->order = (int *)(a + offs[1]);
    p->starts = (int *)(a + offs[2]);
    p->padded_starts = (int *)(a + offs[3]);
    p->list = (int2 *)(a + offs[4]);
    p->stats = (float2 *)(a + offs[5]);
    p->rows = (float *)(a + offs[6]);
    p->calib = (float *)(a + offs[7]);
    p->sched = (int *)(a + offs[8]);
    p->work = (int2 *)(a + offs[9]);
    p->multi = (int *)(a + offs[10]);
    p->scratch = (float *)(a + offs[11]);
    p->tmp = a + offs[12];
    // the zero context row that padding entries read
    hipLaunchKernelGGL(fill_float_kernel, dim3(blocks_for(d->channels)), dim3(256), 0, nullptr,
                       p->rows + z.context_count, (int)d->channels);
    if (!hip_ok(hipDeviceSynchronize(), error, cap, "initialise HIP LSS plan")) {
        bf_cuda_lss_plan_destroy(p);
        return 0;
    }
    p->resident_bytes = total;
    *out = p;
    return 1;
}

extern "C" size_t bf_cuda_lss_plan_resident_bytes(const bf_cuda_lss_plan *plan) {
    return plan ? plan->resident_bytes : 0;
}

namespace {

// The pair sort's scratch in the plan's tmp region.
struct SortScratch {
    int tiles;
    int *alt_k, *alt_v;   // ping-pong pairs
    int *counts, *offs;   // [digit][tile]
    int *totals;          // [digit]
};
SortScratch sort_scratch(const bf_cuda_lss_plan *p) {
    SortScratch w;
    const int n = (int)p->z.samples;
    w.tiles = (n + kSortTile - 1) / kSortTile;
    w.alt_k = reinterpret_cast<int *>(p->tmp);
    w.alt_v = w.alt_k + n;
    w.counts = w.alt_v + n;
    w.offs = w.counts + (size_t)kDigits * w.tiles;
    w.totals = w.offs + (size_t)kDigits * w.tiles;
    return w;
}

// The stable sort of (plan->keys, sample index) into sorted_keys / order:
// ceil(end_bit / kDigitBits) digit passes, ping-ponging through the plan's
// scratch so that the last pass writes the outputs.  The key kernels leave
// the first pass's digit counts.
void sort_pairs(bf_cuda_lss_plan *p, hipStream_t s) {
    const int n = (int)p->z.samples;
    const SortScratch w = sort_scratch(p);
    const int passes = ((int)p->end_bit + kDigitBits - 1) / kDigitBits;
    const int *in_k = p->keys, *in_v = nullptr;
    for (int q = 0; q < passes; ++q) {
        const bool last = (passes - 1 - q) % 2 == 0;
        int *out_k = last ? p->sorted_keys : w.alt_k, *out_v = last ? p->order : w.alt_v;
        const int shift = q * kDigitBits, bits = std::min(kDigitBits, (int)p->end_bit - shift);
        if (q > 0)
            hipLaunchKernelGGL(digit_count_kernel, dim3(w.tiles), dim3(kSortThreads), 0, s, in_k,
                               n, shift, w.tiles, w.counts);
        hipLaunchKernelGGL(digit_offsets_kernel, dim3(kDigits), dim3(kSortThreads), 0, s,
                           w.counts, w.tiles, w.offs, w.totals);
        hipLaunchKernelGGL(digit_scatter_kernel, dim3(w.tiles), dim3(kSortThreads), 0, s, in_k,
                           in_v, n, shift, bits, w.tiles, w.offs, w.totals, out_k, out_v);
        in_k = out_k;
        in_v = out_v;
    }
}

// Cell lists from the keys in plan->keys: the stable sort of (key, sample)
// pairs orders every cell's samples by sample index (out-of-grid samples sort
// after the last cell); a lower bound per cell locates each cell's run; runs
// padded to whole quads give the padded list of {pixel, sample}; then the
// pool schedule.
int build_lists(bf_cuda_lss_plan *p, hipStream_t s, char *error, size_t cap) {
    const bf_lss_desc *d = &p->desc;
    const int n = (int)p->z.samples, cell_count = (int)p->z.cell_count;
    const int hw = (int)(d->feature_height * d->feature_width);
    sort_pairs(p, s);
    // run starts, then the padded starts: per-block sums, their scan, and
    // each block's scan on top
    const int start_blocks = cell_count / kStartThreads + 1;  // cells 0..cell_count
    int *block_sums = reinterpret_cast<int *>(p->tmp);
    hipLaunchKernelGGL(cell_starts_kernel, dim3(start_blocks), dim3(kStartThreads), 0, s,
                       p->sorted_keys, n, p->starts, block_sums, cell_count);
    hipLaunchKernelGGL(block_sums_scan_kernel, dim3(1), dim3(1024), 0, s, block_sums,
                       start_blocks);
    hipLaunchKernelGGL(padded_starts_kernel, dim3(start_blocks), dim3(kStartThreads), 0, s,
                       p->starts, block_sums, p->padded_starts, cell_count);
    hipLaunchKernelGGL(list_entries_kernel, dim3(blocks_for(n)), dim3(256), 0, s, p->order,
                       p->sorted_keys, p->starts, p->padded_starts, p->list, n, cell_count,
                       (int)d->depth_bins * hw, hw);
    hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(kScheduleThreads), 0, s, p->padded_starts,
                       p->sched, p->work, p->multi, p->tiles, p->tiles_per_batch, (int)p->z.cells);
    if (!launch_ok(error, cap, "HIP LSS plan list build")) return 0;
    p->prepared = 1;
    return 1;
}

}  // namespace

extern "C" int bf_cuda_lss_plan_prepare_geometry_f32(bf_cuda_lss_plan *plan,
                                                     const float *geometry, void *stream,
                                                     char *error, size_t cap) {
    if (!plan || !geometry) return fail_contract(error, cap, "invalid HIP LSS plan geometry");
    const bf_lss_desc *d = &plan->desc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    plan->prepared = 0;
    const SortScratch w = sort_scratch(plan);
    hipLaunchKernelGGL(geometry_keys_kernel, dim3(w.tiles), dim3(kKeyThreads), 0, s, geometry,
                       plan->keys, (int)plan->z.samples, (int)(plan->z.samples / d->batches),
                       (int)plan->z.cells, grid_of(d), (int)plan->z.cell_count, w.tiles, w.counts);
    if (!launch_ok(error, cap, "HIP LSS plan rank launch")) return 0;
    return build_lists(plan, s, error, cap);
}

extern "C" int bf_cuda_lss_plan_prepare_calibration_f32(
    bf_cuda_lss_plan *plan, const float *frustum, const float *camera_rotation,
    const float *camera_translation, const float *intrinsics, const float *post_rotation,
    const float *post_translation, const float *extra_rotation, const float *extra_translation,
    void *stream, char *error, size_t cap) {
    if (!plan || !frustum || !camera_rotation || !camera_translation || !intrinsics ||
        !post_rotation || !post_translation)
        return fail_contract(error, cap, "invalid HIP LSS calibration contract");
    const bf_lss_desc *d = &plan->desc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    plan->prepared = 0;
    const int cams = (int)plan->z.cams;
    hipLaunchKernelGGL(calibration_kernel, dim3(blocks_for(cams, 64)), dim3(64), 0, s,
                       camera_rotation, camera_translation, intrinsics, post_rotation,
                       post_translation, extra_rotation, extra_translation, plan->calib,
                       (int)d->cameras, cams);
    const int depth_hw = (int)(d->depth_bins * d->feature_height * d->feature_width);
    const SortScratch w = sort_scratch(plan);
    hipLaunchKernelGGL(calibration_keys_kernel, dim3(w.tiles), dim3(kKeyThreads), 0, s, frustum,
                       plan->calib, plan->keys, (int)plan->z.samples, cams, depth_hw,
                       (int)d->cameras, (int)plan->z.cells, grid_of(d), (int)plan->z.cell_count,
                       w.tiles, w.counts);
    if (!launch_ok(error, cap, "HIP LSS calibration rank launch")) return 0;
    return build_lists(plan, s, error, cap);
}

extern "C" int bf_cuda_lss_plan_forward_f32(bf_cuda_lss_plan *plan, const float *logits,
                                            const float *context, float *bev, void *stream,
                                            char *error, size_t cap) {
    if (!plan || !plan->prepared || !logits || !context || !bev)
        return fail_contract(error, cap, "invalid or unprepared HIP LSS plan");
    const bf_lss_desc *d = &plan->desc;
    const Sizes &z = plan->z;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int hw = (int)(d->feature_height * d->feature_width), C = (int)d->channels;
    const int softmax_blocks = (int)blocks_for(z.pixels, kSoftmaxPixels);
    const int row_groups = (hw + kRowPixels - 1) / kRowPixels;
    hipLaunchKernelGGL(forward_prologue_kernel,
                       dim3((unsigned)(softmax_blocks + row_groups * (int)z.cams)), dim3(256), 0, s,
                       logits, plan->stats, context, plan->rows, (int)z.pixels,
                       (int)d->depth_bins, hw, C, softmax_blocks, row_groups);
    PoolArgs args;
    args.list = plan->list;
    args.logits = logits;
    args.stats = plan->stats;
    args.rows = plan->rows;
    args.starts = plan->padded_starts;
    args.sched = plan->sched;
    args.work = plan->work;
    args.scratch = plan->scratch;
    args.bev = bev;
    args.cells = (int)z.cells;
    args.tiles = plan->tiles;
    args.tiles_per_batch = plan->tiles_per_batch;
    args.C = C;
    args.passes = plan->passes;
    args.chunk_max = plan->chunk_max;
    args.zero_row = (int)z.pixels;
    args.row_bytes = (unsigned)C * 4u;
    args.rows_bytes = (unsigned)((z.context_count + C) * 4);
    const size_t lds = (size_t)plan->chunk_max * kTileCells * sizeof(float);
    const dim3 grid(plan->max_work);
    if (plan->vw == 4 && plan->round == kRoundWide)
        hipLaunchKernelGGL((pool_kernel<4, kRoundWide>), grid, dim3(256), lds, s, args);
    else if (plan->vw == 4)
        hipLaunchKernelGGL((pool_kernel<4, kQuad>), grid, dim3(256), lds, s, args);
    else if (plan->round == kRoundWide)
        hipLaunchKernelGGL((pool_kernel<1, kRoundWide>), grid, dim3(256), lds, s, args);
    else
        hipLaunchKernelGGL((pool_kernel<1, kQuad>), grid, dim3(256), lds, s, args);
    hipLaunchKernelGGL(combine_kernel, dim3(plan->max_multi), dim3(256), 0, s, args,
                       (const int *)plan->multi);
    return launch_ok(error, cap, "HIP LSS plan forward");
}
