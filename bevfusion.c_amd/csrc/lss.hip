// Lift-splat-shoot pooling on gfx950 (drop-in for reference src/cuda_lss.cu).
//
// Plan route (deterministic, no floating-point atomics):
//   prepare:  every sample (b, n, d, y, x) -> BEV cell key (rank + b * cells;
//             samples outside the grid get the key B * cells, which sorts
//             last); a stable radix sort of (key, sample index) pairs
//             (rocPRIM, AMD's device primitives) lists each cell's samples in
//             ascending sample order; a lower bound per cell gives each
//             cell's run; each sample's list slot and each slot's context row
//             are stored.
//   forward:  depth softmax per pixel, each probability stored at its
//             sample's list slot; context NCHW -> rows [B*N*H*W][C]; per BEV
//             cell a group of lanes sums prob * row over the cell's run in
//             list order, and each workgroup stores 64 consecutive cells of
//             every channel plane as coalesced rows.
// Stateless routes: the reference's atomic accumulation (one wave per pixel,
// softmax on the wave, atomicAdd per (channel, depth) sample).
//
// The metric-point -> cell map reproduces the CPU oracle bit for bit: the
// calibration transform is evaluated with floating-point contraction off and
// in the oracle's operation order (inverse by cofactors, row sums left to
// right), and the cell is trunc((p - min) / step) with IEEE division.
#include "bf_cuda.h"
#include "hip_common.h"

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

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

// Stateless ranks (within a batch, -1 outside) or plan keys (rank + batch *
// cells, `invalid` outside).
__global__ __launch_bounds__(256) void geometry_rank_kernel(const float *__restrict__ geometry,
                                                            int *__restrict__ out, int samples,
                                                            int per_batch, int cells, Grid g,
                                                            int with_batch, int invalid) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= samples) return;
    const float p[3] = {geometry[3 * (size_t)s], geometry[3 * (size_t)s + 1], geometry[3 * (size_t)s + 2]};
    const int r = point_rank(p, g);
    out[s] = r < 0 ? invalid : (with_batch ? r + (s / per_batch) * cells : r);
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

__global__ __launch_bounds__(256) void calibration_rank_kernel(const float *__restrict__ frustum,
                                                               const float *__restrict__ calib,
                                                               int *__restrict__ keys, int samples,
                                                               int depth_hw, int cams_per_batch,
                                                               int cells, Grid g, int invalid) {
#pragma clang fp contract(off)
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= samples) return;
    const int cam = s / depth_hw, local = s - cam * depth_hw;
    const float *o = calib + (size_t)cam * kCalib;
    if (o[36] == 0.0f) { keys[s] = invalid; return; }
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
    keys[s] = rank >= 0 ? rank + (cam / cams_per_batch) * cells : invalid;
}

__global__ __launch_bounds__(256) void fill_float_kernel(float *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// starts[c] = first sorted position whose key is >= c (c in [0, cell_count]):
// a lower bound over the sorted keys, so empty cells get empty runs.
__global__ __launch_bounds__(256) void cell_starts_kernel(const int *__restrict__ sorted_keys,
                                                         int samples, int *__restrict__ starts,
                                                         int cell_count) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c > cell_count) return;
    int lo = 0, hi = samples;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sorted_keys[mid] < c) lo = mid + 1;
        else hi = mid;
    }
    starts[c] = lo;
}

// From the sorted sample order: every sample's position in the list (where the
// forward's softmax stores its probability) and the context row each list
// entry reads.
__global__ __launch_bounds__(256) void list_maps_kernel(const int *__restrict__ order,
                                                       int *__restrict__ position,
                                                       int *__restrict__ list_pixel, int samples,
                                                       int depth_hw, int hw) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= samples) return;
    const int s = order[i];
    const int cam = s / depth_hw;
    position[s] = i;
    list_pixel[i] = cam * hw + (s - cam * depth_hw) % hw;
}

// Max-shifted depth softmax (reference lss.c:144-158 operation order: float
// max, double sum of expf(l - max), inverse rounded to float, p = e * inv).
// Workgroup = 32 pixels x 8 depth slices of kSlice bins; each probability is
// stored at its sample's list position.
constexpr int kSoftmaxPixels = 32, kSlices = 8, kSlice = kMaxDepth / kSlices;
__global__ __launch_bounds__(256) void softmax_list_kernel(const float *__restrict__ logits,
                                                          const int *__restrict__ position,
                                                          float *__restrict__ list_prob,
                                                          int pixels, int depths, int hw) {
    __shared__ float part_max[kSlices][kSoftmaxPixels];
    __shared__ double part_sum[kSlices][kSoftmaxPixels];
    const int lane = threadIdx.x & (kSoftmaxPixels - 1), slice = threadIdx.x / kSoftmaxPixels;
    const int px = blockIdx.x * kSoftmaxPixels + lane;
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
    for (int k = 0; k < kSlice; ++k) {
        v[k] = (d0 + k < depths) ? expf(v[k] - m) : 0.0f;
        sum += v[k];
    }
    part_sum[slice][lane] = sum;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < kSlices; ++j) total += part_sum[j][lane];
    const float inv = (float)(1.0 / total);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < kSlice; ++k) {
        const int d = d0 + k;
        if (d < depths) {
            const size_t s = base + (size_t)d * hw;
            list_prob[position[s]] = v[k] * inv;
        }
    }
}

// Context [cams][C][hw] -> [cams * hw][C] through a 64 x 64 LDS tile.
__global__ __launch_bounds__(256) void context_rows_kernel(const float *__restrict__ ctx,
                                                           float *__restrict__ rows, int C,
                                                           int hw) {
    __shared__ float tile[64][65];
    const int cam = blockIdx.z, c0 = blockIdx.y * 64, p0 = blockIdx.x * 64, t = threadIdx.x;
    const float *src = ctx + (size_t)cam * C * hw;
    for (int i = 0; i < 16; ++i) {
        const int cl = (t >> 6) + 4 * i, pl = t & 63, c = c0 + cl, p = p0 + pl;
        tile[cl][pl] = (c < C && p < hw) ? src[(size_t)c * hw + p] : 0.0f;
    }
    __syncthreads();
    float *dst = rows + (size_t)cam * hw * C;
    for (int i = 0; i < 16; ++i) {
        const int pl = (t >> 6) + 4 * i, cl = t & 63, c = c0 + cl, p = p0 + pl;
        if (c < C && p < hw) dst[(size_t)p * C + c] = tile[cl][pl];
    }
}

// Cell pooling over the sorted lists: a group of L lanes (VW channels each)
// owns one cell at a time and sums prob * context row over the cell's list in
// list order; the workgroup's 64 consecutive cells land in an LDS tile
// [channel][cell] that is stored as coalesced 64-cell rows of every channel
// plane.  The next chunk of (row, prob) list entries is loaded while the
// current one is consumed.
constexpr int kTileCells = 64;
template <int VW>
__global__ __launch_bounds__(256) void pool_tile_kernel(const float *__restrict__ list_prob,
                                                       const int *__restrict__ list_pixel,
                                                       const float *__restrict__ rows,
                                                       const int *__restrict__ starts,
                                                       float *__restrict__ bev, int cells, int C) {
    // [64 * VW channels][64 cells], cell index XOR-swizzled by the channel so
    // that both the per-cell column writes and the per-channel row reads are
    // free of bank conflicts.
    extern __shared__ float tile[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.y, cell0 = blockIdx.x * kTileCells;
    const int tile_cells = min(kTileCells, cells - cell0);
    for (int c0 = 0; c0 < C; c0 += 64 * VW) {
        const int chunk = min(64 * VW, C - c0);
        const int L = (chunk + VW - 1) / VW, G = 64 / L;
        const int gi = lane / L, lig = lane - gi * L, gbase = gi * L;
        const int ch = c0 + VW * lig;
        if (gi < G) {
            for (int t = wave * G + gi; t < tile_cells; t += 4 * G) {
                const int oc = b * cells + cell0 + t;
                const int lo = starts[oc], hi = starts[oc + 1];
                float acc[VW];
#pragma unroll
                for (int j = 0; j < VW; ++j) acc[j] = 0.0f;
                int next_pix = 0;
                float next_pr = 0.0f;
                if (lo + lig < hi) {
                    next_pix = list_pixel[lo + lig];
                    next_pr = list_prob[lo + lig];
                }
                for (int base = lo; base < hi; base += L) {
                    const int n = min(L, hi - base);
                    const int my_pix = next_pix;
                    const float my_pr = next_pr;
                    if (base + L + lig < hi) {
                        next_pix = list_pixel[base + L + lig];
                        next_pr = list_prob[base + L + lig];
                    }
                    for (int k = 0; k < n; k += 4) {
                        int pk[4];
                        float wk[4], vk[4][VW];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int src = gbase + (k + u < n ? k + u : 0);
                            pk[u] = __shfl(my_pix, src);
                            wk[u] = __shfl(my_pr, src);
                            const float *row = rows + (size_t)pk[u] * C + ch;
                            if (VW == 4) {
                                const float4 q = *reinterpret_cast<const float4 *>(row);
                                vk[u][0] = q.x; vk[u][1 % VW] = q.y;
                                vk[u][2 % VW] = q.z; vk[u][3 % VW] = q.w;
                            } else {
                                vk[u][0] = ch < C ? row[0] : 0.0f;
                            }
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            if (k + u < n)
#pragma unroll
                                for (int j = 0; j < VW; ++j) acc[j] += wk[u] * vk[u][j];
                    }
                }
#pragma unroll
                for (int j = 0; j < VW; ++j) {
                    const int c = VW * lig + j;
                    tile[c * kTileCells + (t ^ (c & 63))] = acc[j];
                }
            }
        }
        __syncthreads();
        float *out = bev + ((size_t)b * C + c0) * cells + cell0;
        const int j = threadIdx.x & 63;
        for (int c = threadIdx.x >> 6; c < chunk; c += 4)
            if (j < tile_cells) out[(size_t)c * cells + j] = tile[c * kTileCells + (j ^ (c & 63))];
        __syncthreads();
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

// Plan memory (one arena).  Three sample-sized arrays change role once the
// sort is done:  keys -> position (sample -> list slot),  sorted keys ->
// list_pixel (list slot -> context row),  order -> list_prob (written by
// every forward).
struct bf_cuda_lss_plan {
    bf_lss_desc desc;
    Sizes z;
    int prepared;
    unsigned end_bit;  // sort key width: cell_count (the invalid key) is below 2^end_bit
    int *keys, *sorted_keys, *order, *starts;
    float *rows, *calib;
    void *sort_tmp;
    size_t sort_tmp_bytes;
    void *arena;
    size_t resident_bytes;
    int *position() const { return keys; }
    int *list_pixel() const { return sorted_keys; }
    float *list_prob() const { return reinterpret_cast<float *>(order); }
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
                       (int)(z.samples / d->batches), (int)z.cells, grid_of(d), 0, -1);
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
    if (!hip_ok(rocprim::radix_sort_pairs(nullptr, p->sort_tmp_bytes, (const unsigned *)nullptr,
                                          (unsigned *)nullptr, rocprim::counting_iterator<int>(0),
                                          (int *)nullptr, (unsigned)z.samples, 0u, p->end_bit),
                error, cap, "size HIP LSS plan sort")) {
        bf_cuda_lss_plan_destroy(p);
        return 0;
    }
    // keys, sorted keys, order [samples]; starts [cells + 1]; context rows;
    // calibration; sort scratch.
    const size_t parts[7] = {z.samples * 4, z.samples * 4, z.samples * 4, (z.cell_count + 1) * 4,
                             z.context_count * 4, z.cams * kCalib * 4, p->sort_tmp_bytes};
    size_t offs[7], total = 0;
    for (int i = 0; i < 7; ++i) {
        offs[i] = total;
        total += (parts[i] + 255) & ~size_t(255);
    }
    if (!hip_ok(hipMalloc(&p->arena, total), error, cap, "allocate HIP LSS plan")) {
        bf_cuda_lss_plan_destroy(p);
        return 0;
    }
    unsigned char *a = (unsigned char *)p->arena;
    p->keys = (int *)(a + offs[0]);
    p->sorted_keys = (int *)(a + offs[1]);
    p->order = (int *)(a + offs[2]);
    p->starts = (int *)(a + offs[3]);
    p->rows = (float *)(a + offs[4]);
    p->calib = (float *)(a + offs[5]);
    p->sort_tmp = a + offs[6];
    p->resident_bytes = total;
    *out = p;
    return 1;
}

extern "C" size_t bf_cuda_lss_plan_resident_bytes(const bf_cuda_lss_plan *plan) {
    return plan ? plan->resident_bytes : 0;
}

namespace {

// Cell lists from the keys in plan->keys: the stable sort of (key, sample)
// pairs orders every cell's samples by sample index (out-of-grid samples sort
// after the last cell); a lower bound per cell locates each cell's run; then
// the sorted order becomes the position / list_pixel maps the forward reads.
int build_lists(bf_cuda_lss_plan *p, hipStream_t s, char *error, size_t cap) {
    const bf_lss_desc *d = &p->desc;
    const int n = (int)p->z.samples, cell_count = (int)p->z.cell_count;
    const int hw = (int)(d->feature_height * d->feature_width);
    if (!hip_ok(rocprim::radix_sort_pairs(p->sort_tmp, p->sort_tmp_bytes,
                                          reinterpret_cast<const unsigned *>(p->keys),
                                          reinterpret_cast<unsigned *>(p->sorted_keys),
                                          rocprim::counting_iterator<int>(0), p->order,
                                          (unsigned)n, 0u, p->end_bit, s),
                error, cap, "HIP LSS plan sort"))
        return 0;
    hipLaunchKernelGGL(cell_starts_kernel, dim3(blocks_for((size_t)cell_count + 1)), dim3(256), 0, s,
                       p->sorted_keys, n, p->starts, cell_count);
    hipLaunchKernelGGL(list_maps_kernel, dim3(blocks_for(n)), dim3(256), 0, s, p->order,
                       p->position(), p->list_pixel(), n, (int)d->depth_bins * hw, hw);
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
    hipLaunchKernelGGL(geometry_rank_kernel, dim3(blocks_for(plan->z.samples)), dim3(256), 0, s,
                       geometry, plan->keys, (int)plan->z.samples,
                       (int)(plan->z.samples / d->batches), (int)plan->z.cells, grid_of(d), 1,
                       (int)plan->z.cell_count);
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
    hipLaunchKernelGGL(calibration_rank_kernel, dim3(blocks_for(plan->z.samples)), dim3(256), 0, s,
                       frustum, plan->calib, plan->keys, (int)plan->z.samples, depth_hw,
                       (int)d->cameras, (int)plan->z.cells, grid_of(d), (int)plan->z.cell_count);
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
    hipLaunchKernelGGL(softmax_list_kernel, dim3(blocks_for(z.pixels, kSoftmaxPixels)), dim3(256),
                       0, s, logits, plan->position(), plan->list_prob(), (int)z.pixels,
                       (int)d->depth_bins, hw);
    hipLaunchKernelGGL(context_rows_kernel, dim3((hw + 63) / 64, (C + 63) / 64, (unsigned)z.cams),
                       dim3(256), 0, s, context, plan->rows, C, hw);
    const dim3 grid((unsigned)((z.cells + kTileCells - 1) / kTileCells), (unsigned)d->batches);
    if (C % 4 == 0)
        hipLaunchKernelGGL(pool_tile_kernel<4>, grid, dim3(256),
                           min(C, 256) * kTileCells * sizeof(float), s, plan->list_prob(),
                           plan->list_pixel(), plan->rows, plan->starts, bev, (int)z.cells, C);
    else
        hipLaunchKernelGGL(pool_tile_kernel<1>, grid, dim3(256),
                           min(C, 64) * kTileCells * sizeof(float), s, plan->list_prob(),
                           plan->list_pixel(), plan->rows, plan->starts, bev, (int)z.cells, C);
    return launch_ok(error, cap, "HIP LSS plan forward");
}
