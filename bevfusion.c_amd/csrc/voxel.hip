// Voxeliser with MeanVFE (drop-in for reference src/cuda_voxel.cu).
//
// The reference CPU voxeliser walks the points in order and creates a voxel
// at its first point (voxel.c:57-138).  The same result in parallel, with no
// sort, no memset and no host round trip (so a caller can capture it in a
// HIP graph):
//   1. key_kernel: each point's cell key ((z GY + y) GX + x), or an invalid
//      key for non-finite / out-of-range points (the CPU's cell arithmetic);
//      an atomic min of the point index into a dense per-cell word gives each
//      cell its first point, whatever the order the atomics land in;
//   2. flag/sums/rank kernels: a point is a voxel head when it is its cell's
//      first point; an exclusive scan of the head flags in point order gives
//      every voxel its first-encounter rank, the CPU's voxel index;
//   3. insert_kernel: each point of a kept voxel is inserted into the voxel's
//      max_points_per_voxel slots by an atomic-min cascade (the slot keeps
//      the smaller index and the larger one moves on to the next slot), which
//      leaves exactly the voxel's smallest point indices, ascending, for any
//      interleaving of the atomics: slot k receives every index but the k
//      smallest and keeps the least of them;
//   4. mean_kernel: the mean of the slotted points, summed in input order and
//      divided once (kernels_ref.c:477-490), bit-identical to the CPU; the
//      cell words are reset for the next call.
#include "bf_cuda_voxel.h"
#include "hip_common.h"
#include "internal.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>

using namespace bfhip;

namespace {

constexpr unsigned kInvalid = 0xffffffffu, kEmpty = 0xffffffffu;
constexpr int kTile = 1024;  // points per scan workgroup (256 threads x 4)

struct VoxelGeom {
    float min[3], max[3], size[3];
    unsigned grid[3];
    int max_points;
    unsigned max_voxels;
};

__global__ void count_init_kernel(const unsigned *__restrict__ src, unsigned host, unsigned bound,
                                  unsigned *__restrict__ dst) {
    if (threadIdx.x || blockIdx.x) return;
    const unsigned n = src ? *src : host;
    *dst = n < bound ? n : bound;
}

__global__ __launch_bounds__(256) void key_kernel(const float *__restrict__ points,
                                                  const unsigned *__restrict__ count_word,
                                                  VoxelGeom g,
                                                  unsigned *__restrict__ keys,
                                                  unsigned *__restrict__ first) {
    const unsigned i = blockIdx.x * 256 + threadIdx.x;
    if (i >= *count_word) return;
    const float *p = points + (size_t)i * 5;
    bool ok = isfinite(p[0]) && isfinite(p[1]) && isfinite(p[2]) && isfinite(p[3]) &&
              isfinite(p[4]);
    unsigned cell[3] = {0, 0, 0};
    for (int a = 0; a < 3 && ok; ++a) {
        if (p[a] < g.min[a] || p[a] >= g.max[a]) {
            ok = false;
            break;
        }
        const int c = (int)floorf((p[a] - g.min[a]) / g.size[a]);
        if (c < 0 || (unsigned)c >= g.grid[a]) ok = false;
        cell[a] = (unsigned)c;
    }
    const unsigned key = ok ? (cell[2] * g.grid[1] + cell[1]) * g.grid[0] + cell[0] : kInvalid;
    keys[i] = key;
    if (ok) atomicMin(first + key, i);
}

__device__ __forceinline__ unsigned wave_inclusive(unsigned v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

// Exclusive scan of 256 per-thread values inside the workgroup; *total gets
// the workgroup sum.
__device__ __forceinline__ unsigned block_exclusive(unsigned v, unsigned *total) {
    __shared__ unsigned waves[4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const unsigned inc = wave_inclusive(v, lane);
    if (lane == 63) waves[w] = inc;
    __syncthreads();
    unsigned before = 0;
    for (int k = 0; k < w; ++k) before += waves[k];
    *total = waves[0] + waves[1] + waves[2] + waves[3];
    __syncthreads();
    return before + inc - v;
}

__device__ __forceinline__ bool is_head(const unsigned *keys, const unsigned *first, unsigned i) {
    const unsigned k = keys[i];
    return k != kInvalid && first[k] == i;
}

// Head flags per tile of kTile points -> tile sums.
__global__ __launch_bounds__(256) void flag_kernel(const unsigned *__restrict__ keys,
                                                   const unsigned *__restrict__ first,
                                                   const unsigned *__restrict__ count_word,
                                                   unsigned *__restrict__ sums) {
    const unsigned count = *count_word, base = blockIdx.x * kTile + threadIdx.x * 4;
    unsigned c = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (base + k < count) c += is_head(keys, first, base + k);
    unsigned total;
    (void)block_exclusive(c, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One workgroup: exclusive scan of the tile sums in place; the voxel count.
__global__ __launch_bounds__(256) void sums_kernel(unsigned *__restrict__ sums, unsigned tiles,
                                                   unsigned max_voxels,
                                                   unsigned *__restrict__ voxel_count) {
    unsigned carry = 0;
    for (unsigned b = 0; b < tiles; b += 256) {
        const unsigned i = b + threadIdx.x;
        const unsigned v = i < tiles ? sums[i] : 0u;
        unsigned total;
        const unsigned ex = block_exclusive(v, &total);
        if (i < tiles) sums[i] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0) *voxel_count = carry < max_voxels ? carry : max_voxels;
}

// Ranks of the head points; a kept voxel gets its coordinate and empty slots.
__global__ __launch_bounds__(256) void rank_kernel(const unsigned *__restrict__ keys,
                                                   const unsigned *__restrict__ first,
                                                   const unsigned *__restrict__ count_word,
                                                   const unsigned *__restrict__ offsets,
                                                   VoxelGeom g, unsigned *__restrict__ rank,
                                                   bf_coord4 *__restrict__ coords,
                                                   unsigned *__restrict__ slots) {
    const unsigned count = *count_word, base = blockIdx.x * kTile + threadIdx.x * 4;
    bool head[4];
    unsigned c = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        head[k] = base + k < count && is_head(keys, first, base + k);
        c += head[k];
    }
    unsigned total;
    unsigned r = offsets[blockIdx.x] + block_exclusive(c, &total);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (!head[k]) continue;
        const unsigned i = base + k;
        rank[i] = r;
        if (r < g.max_voxels) {
            const unsigned key = keys[i], x = key % g.grid[0], q = key / g.grid[0];
            coords[r] = bf_coord4{0, (int)(q / g.grid[1]), (int)(q % g.grid[1]), (int)x};
            for (int s = 0; s < g.max_points; ++s) slots[(size_t)r * g.max_points + s] = kEmpty;
        }
        ++r;
    }
}

__global__ __launch_bounds__(256) void insert_kernel(const unsigned *__restrict__ keys,
                                                     const unsigned *__restrict__ first,
                                                     const unsigned *__restrict__ rank,
                                                     const unsigned *__restrict__ count_word,
                                                     VoxelGeom g, unsigned *__restrict__ slots) {
    const unsigned i = blockIdx.x * 256 + threadIdx.x;
    if (i >= *count_word) return;
    const unsigned key = keys[i];
    if (key == kInvalid) return;
    const unsigned v = rank[first[key]];
    if (v >= g.max_voxels) return;
    unsigned *slot = slots + (size_t)v * g.max_points;
    unsigned x = i;
    for (int s = 0; s < g.max_points; ++s) {
        const unsigned old = atomicMin(slot + s, x);
        if (old == kEmpty) break;  // x took a free slot
        x = old > x ? old : x;     // the larger index moves on
    }
}

__global__ __launch_bounds__(256) void mean_kernel(const float *__restrict__ points,
                                                   const unsigned *__restrict__ slots,
                                                   const unsigned *__restrict__ voxel_count,
                                                   int max_points, float *__restrict__ means) {
    const unsigned v = blockIdx.x * 256 + threadIdx.x;
    if (v >= *voxel_count) return;
    float sum[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int live = 0;
    for (; live < max_points; ++live) {
        const unsigned i = slots[(size_t)v * max_points + live];
        if (i == kEmpty) break;
        const float *p = points + (size_t)i * 5;
#pragma unroll
        for (int c = 0; c < 5; ++c) sum[c] += p[c];
    }
#pragma unroll
    for (int c = 0; c < 5; ++c) means[(size_t)v * 5 + c] = sum[c] / (float)live;
}

__global__ __launch_bounds__(256) void clear_kernel(const unsigned *__restrict__ keys,
                                                    const unsigned *__restrict__ count_word,
                                                    unsigned *__restrict__ first) {
    const unsigned i = blockIdx.x * 256 + threadIdx.x;
    if (i >= *count_word) return;
    const unsigned key = keys[i];
    if (key != kInvalid) first[key] = kEmpty;
}

__global__ void zero_count_kernel(unsigned *__restrict__ out) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *out = 0u;
}

}  // namespace

struct bf_cuda_voxelizer {
    VoxelGeom geom;
    size_t max_points, resident_bytes;
    unsigned *keys, *first, *rank, *sums, *slots, *count_word;
};

extern "C" void bf_cuda_voxelizer_destroy(bf_cuda_voxelizer *v) {
    if (!v) return;
    for (void *p : {(void *)v->keys, (void *)v->first, (void *)v->rank, (void *)v->sums,
                    (void *)v->slots, (void *)v->count_word})
        if (p) (void)hipFree(p);
    std::free(v);
}

extern "C" size_t bf_cuda_voxelizer_resident_bytes(const bf_cuda_voxelizer *v) {
    return v ? v->resident_bytes : 0;
}

extern "C" int bf_cuda_voxelizer_create(const bf_voxel_config *cfg, size_t max_points,
                                        bf_cuda_voxelizer **out, char *error, size_t cap) {
    if (out) *out = nullptr;
    if (!cfg || !out || !max_points || max_points >= INT_MAX || cfg->point_features != 5 ||
        !cfg->max_points_per_voxel || cfg->max_points_per_voxel > 4096 || !cfg->max_voxels ||
        cfg->max_voxels >= UINT_MAX)
        return fail(error, cap, "invalid HIP voxelizer contract");
    VoxelGeom g{};
    unsigned long long cells = 1;
    for (int a = 0; a < 3; ++a) {
        // Grid shape as voxel.c:31-49: round(extent / size), within 1e-4.
        const float extent = cfg->maximum[a] - cfg->minimum[a], size = cfg->voxel_size[a];
        if (!std::isfinite(extent) || !std::isfinite(size) || extent <= 0.0f || size <= 0.0f)
            return fail(error, cap, "invalid HIP voxelizer contract");
        const double c = (double)extent / size;
        const long long r = std::llround(c);
        if (r <= 0 || std::fabs(c - (double)r) > 1e-4 * std::fmax(1.0, c))
            return fail(error, cap, "invalid HIP voxelizer contract");
        g.min[a] = cfg->minimum[a];
        g.max[a] = cfg->maximum[a];
        g.size[a] = size;
        g.grid[a] = (unsigned)r;
        cells *= (unsigned long long)r;
        if (cells >= kInvalid) return fail(error, cap, "HIP voxel grid is too large");
    }
    g.max_points = (int)cfg->max_points_per_voxel;
    g.max_voxels = (unsigned)cfg->max_voxels;
    bf_cuda_voxelizer *v = (bf_cuda_voxelizer *)std::calloc(1, sizeof(*v));
    if (!v) return fail(error, cap, "HIP voxelizer allocation failed");
    v->geom = g;
    v->max_points = max_points;
    const size_t n = max_points, tiles = (n + kTile - 1) / kTile;
    const size_t slot_words = (size_t)g.max_voxels * g.max_points;
    const size_t bytes[6] = {n * 4, (size_t)cells * 4, n * 4, tiles * 4, slot_words * 4, 4};
    unsigned **bufs[6] = {&v->keys, &v->first, &v->rank, &v->sums, &v->slots, &v->count_word};
    for (int b = 0; b < 6; ++b) {
        if (!hip_ok(hipMalloc((void **)bufs[b], bytes[b]), error, cap, "allocate voxel buffers")) {
            bf_cuda_voxelizer_destroy(v);
            return 0;
        }
        v->resident_bytes += bytes[b];
    }
    // Every cell word is "no point" between calls; forwards reset what they set.
    if (!hip_ok(hipMemset(v->first, 0xff, bytes[1]), error, cap, "clear voxel cells") ||
        !hip_ok(hipDeviceSynchronize(), error, cap, "clear voxel cells")) {
        bf_cuda_voxelizer_destroy(v);
        return 0;
    }
    *out = v;
    return 1;
}

namespace {

// count is the exact point count, or with count_device the bound of *count_device.
int voxelize(bf_cuda_voxelizer *v, const float *points, const unsigned *count_device,
             size_t count, bf_coord4 *coords, float *means, unsigned *voxel_count,
             void *stream_value, char *error, size_t cap) {
    if (!v || (!points && count) || count > v->max_points || !coords || !means || !voxel_count)
        return fail(error, cap, "invalid HIP voxelize buffers");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream_value);
    const unsigned n = (unsigned)count, blocks = (n + 255) / 256, tiles = (n + kTile - 1) / kTile;
    if (!n) {
        zero_count_kernel<<<1, 64, 0, s>>>(voxel_count);
        return launch_ok(error, cap, "HIP voxelize launch");
    }
    const VoxelGeom &g = v->geom;
    count_init_kernel<<<1, 64, 0, s>>>(count_device, n, n, v->count_word);
    key_kernel<<<blocks, 256, 0, s>>>(points, v->count_word, g, v->keys, v->first);
    flag_kernel<<<tiles, 256, 0, s>>>(v->keys, v->first, v->count_word, v->sums);
    sums_kernel<<<1, 256, 0, s>>>(v->sums, tiles, g.max_voxels, voxel_count);
    rank_kernel<<<tiles, 256, 0, s>>>(v->keys, v->first, v->count_word, v->sums, g, v->rank,
                                      coords, v->slots);
    insert_kernel<<<blocks, 256, 0, s>>>(v->keys, v->first, v->rank, v->count_word, g, v->slots);
    const unsigned vblocks = (unsigned)std::min<size_t>((g.max_voxels + 255) / 256, blocks);
    mean_kernel<<<vblocks, 256, 0, s>>>(points, v->slots, voxel_count, g.max_points, means);
    clear_kernel<<<blocks, 256, 0, s>>>(v->keys, v->count_word, v->first);
    return launch_ok(error, cap, "HIP voxelize launch");
}

}  // namespace

extern "C" int bf_cuda_voxelize_mean_f32(bf_cuda_voxelizer *v, const float *points,
                                         size_t count, bf_coord4 *coords, float *means,
                                         unsigned *voxel_count, void *stream, char *error,
                                         size_t cap) {
    return voxelize(v, points, nullptr, count, coords, means, voxel_count, stream, error, cap);
}

int bfhip::voxelize_count_device(bf_cuda_voxelizer *v, const float *points,
                                 const unsigned *count_device, size_t bound, bf_coord4 *coords,
                                 float *means, unsigned *voxel_count, void *stream, char *error,
                                 size_t cap) {
    if (!count_device || !points || !bound) return fail(error, cap, "invalid HIP voxelize buffers");
    return voxelize(v, points, count_device, bound, coords, means, voxel_count, stream, error, cap);
}
