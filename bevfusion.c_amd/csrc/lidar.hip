// SECOND sparse LiDAR encoder (drop-in for reference src/cuda_lidar.cu).
//
// Active sites of each level live in a dense int32 index grid over that
// level's batches x depth x height x width cells (340 MB at the production
// 41 x 1440 x 1440 input; the coarser levels add 50 MB): a cell holds the
// site's row or -1.  The grids are -1 between forwards — a forward writes
// exactly its sites' cells and clears them at the end — so finding a
// neighbour is one load, with no hashing and no atomics.
//
//   level 0      the caller's voxel rows, in the caller's order;
//   submanifold  27-tap neighbour table per row (same level, pad 1);
//   strided      each input site marks every output cell one of its taps
//                reaches, one byte per cell in a mark map, then the marked
//                cells are compacted in cell order — ascending
//                (batch, z, y, x), the reference's site order — by per-chunk
//                counts and an in-order write pass that also clears the map
//                (no atomics across workgroups); then a neighbour table from
//                output to input;
//   convolution  gather GEMM on the matrix cores: 32 output rows per wave,
//                K = taps x input channels, each lane gathering its row's
//                neighbour features as the A operand and the BN-folded
//                weights [tap][co][ci] as B; taps no row of the wave uses
//                are skipped; bias, residual add and ReLU fused in the
//                epilogue.  The 5-channel input conv runs in fp32 on the
//                vector units (its inputs are metric coordinates).
// Precision: features and weights are kept as split fp16 pairs, x = hi + lo
// with hi = fp16(x) and lo = fp16(x - hi), and every product is formed as
// hi*Whi + lo*Whi + hi*Wlo on fp16 MFMAs with fp32 accumulation (the
// dropped lo*Wlo term is 2^-22 relative) -- the split-operand scheme of
// Ootomo and Yokota, "Recovering single precision accuracy from Tensor Cores
// while surpassing the FP32 theoretical peak performance" (IJHPCA 2022).
// Sixteen chained layers of plain fp16 operands drift to ~1e-1 of the BEV's
// RMS at its largest entries; the split keeps the encoder near fp32.
// The output conv writes fp32 rows, gathered into the dense BEV.
#include "bf_cuda_lidar.h"
#include "host_util.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <vector>

using namespace bfhip;

namespace {

constexpr int kTaps = 27, kChunk = 8192, kRowsPerWave = 32, kRowsPerGroup = 4 * kRowsPerWave;
constexpr int kEmpty = -1;
constexpr float kBnEps = 1e-3f;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

struct Grid {
    int b, d, h, w;
};
struct Geom {
    int kd, kh, kw, sd, sh, sw, pd, ph, pw;
};

__device__ __forceinline__ long long cell_of(const Grid &g, int b, int z, int y, int x) {
    return (((long long)b * g.d + z) * g.h + y) * g.w + x;
}
__device__ __forceinline__ bool inside(const Grid &g, int b, int z, int y, int x) {
    return (unsigned)b < (unsigned)g.b && (unsigned)z < (unsigned)g.d &&
           (unsigned)y < (unsigned)g.h && (unsigned)x < (unsigned)g.w;
}

__global__ void count_init_kernel(const unsigned *__restrict__ src, unsigned host, unsigned cap,
                                  unsigned *__restrict__ dst) {
    if (threadIdx.x || blockIdx.x) return;
    const unsigned n = src ? *src : host;
    *dst = n < cap ? n : cap;
}

__global__ __launch_bounds__(256) void index_kernel(const bf_coord4 *__restrict__ coords,
                                                    const unsigned *__restrict__ count, Grid g,
                                                    int *__restrict__ grid) {
    const unsigned n = *count;
    for (unsigned j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        const bf_coord4 c = coords[j];
        if (inside(g, c.batch, c.z, c.y, c.x)) grid[cell_of(g, c.batch, c.z, c.y, c.x)] = (int)j;
    }
}

// The five levels' site lists and index grids, for one clearing launch.
struct LevelGrids {
    const bf_coord4 *coords[5];
    const unsigned *count[5];
    int *grid[5];
    Grid g[5];
};

// Returns every level's index grid to empty at its own sites (blockIdx.y is
// the level), so the grids are clean for the next forward.
__global__ __launch_bounds__(256) void clear_kernel(LevelGrids lg) {
    const int l = (int)blockIdx.y;
    const bf_coord4 *coords = lg.coords[l];
    int *grid = lg.grid[l];
    const Grid g = lg.g[l];
    const unsigned n = *lg.count[l];
    for (unsigned j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        const bf_coord4 c = coords[j];
        if (inside(g, c.batch, c.z, c.y, c.x)) grid[cell_of(g, c.batch, c.z, c.y, c.x)] = kEmpty;
    }
}

// Neighbour tables, one thread per (row, tap) entry so the table stores are
// contiguous.  Submanifold 3x3x3 (pad 1): tap (kz, ky, kx) of site s reads
// s + (k - 1).
__global__ __launch_bounds__(256) void subm_neighbors_kernel(const bf_coord4 *__restrict__ coords,
                                                             const unsigned *__restrict__ count,
                                                             Grid g, const int *__restrict__ grid,
                                                             int *__restrict__ nbr) {
    const size_t total = (size_t)*count * kTaps;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (size_t)gridDim.x * 256) {
        const unsigned j = (unsigned)(e / kTaps);
        const int t = (int)(e - (size_t)j * kTaps);
        const bf_coord4 c = coords[j];
        const int z = c.z + t / 9 - 1, y = c.y + (t / 3) % 3 - 1, x = c.x + t % 3 - 1;
        nbr[e] = inside(g, c.batch, z, y, x) ? grid[cell_of(g, c.batch, z, y, x)] : kEmpty;
    }
}

// Strided conv: tap k of output site o reads input o * s - p + k.
__global__ __launch_bounds__(256) void down_neighbors_kernel(const bf_coord4 *__restrict__ coords,
                                                             const unsigned *__restrict__ count,
                                                             Grid gin, Geom q,
                                                             const int *__restrict__ grid,
                                                             int *__restrict__ nbr) {
    const int taps = q.kd * q.kh * q.kw;
    const size_t total = (size_t)*count * kTaps;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (size_t)gridDim.x * 256) {
        const unsigned j = (unsigned)(e / kTaps);
        const int t = (int)(e - (size_t)j * kTaps);
        if (t >= taps) continue;
        const bf_coord4 c = coords[j];
        const int kz = t / (q.kh * q.kw), ky = (t / q.kw) % q.kh, kx = t % q.kw;
        const int z = c.z * q.sd - q.pd + kz, y = c.y * q.sh - q.ph + ky, x = c.x * q.sw - q.pw + kx;
        nbr[e] = inside(gin, c.batch, z, y, x) ? grid[cell_of(gin, c.batch, z, y, x)] : kEmpty;
    }
}

// Marks every output cell some tap of an input site reaches (the exact
// strided images of kernels_ref.c:632-644 / 686-707): byte `cell` of the
// mark map, by plain stores of one value (no atomics).
__global__ __launch_bounds__(256) void mark_kernel(const bf_coord4 *__restrict__ coords,
                                                   const unsigned *__restrict__ count, Grid gout,
                                                   Geom q, unsigned char *__restrict__ marks) {
    const unsigned n = *count;
    for (unsigned j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        const bf_coord4 c = coords[j];
        if ((unsigned)c.batch >= (unsigned)gout.b) continue;
        for (int kz = 0; kz < q.kd; ++kz) {
            const int nz = c.z + q.pd - kz;
            if (nz < 0 || nz % q.sd || nz / q.sd >= gout.d) continue;
            for (int ky = 0; ky < q.kh; ++ky) {
                const int ny = c.y + q.ph - ky;
                if (ny < 0 || ny % q.sh || ny / q.sh >= gout.h) continue;
                for (int kx = 0; kx < q.kw; ++kx) {
                    const int nx = c.x + q.pw - kx;
                    if (nx < 0 || nx % q.sw || nx / q.sw >= gout.w) continue;
                    marks[cell_of(gout, c.batch, nz / q.sd, ny / q.sh, nx / q.sw)] = 1;
                }
            }
        }
    }
}

// Bit b of the result: byte b of the 32-cell group w of the mark map is set.
// The map is padded to whole chunks, so every group is in bounds.
__device__ __forceinline__ unsigned group_bits(const unsigned char *marks, long long w) {
    const uint4 *p = reinterpret_cast<const uint4 *>(marks + w * 32);
    const uint4 lo = p[0], hi = p[1];
    const unsigned v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    unsigned bits = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) bits |= (unsigned)((v[i] >> (8 * k)) & 0xffu ? 1u : 0u) << (4 * i + k);
    return bits;
}

// Marked cells per chunk of kChunk cells (256 groups of 32 cells).
__global__ __launch_bounds__(256) void compact_count_kernel(const unsigned char *__restrict__ marks,
                                                            long long words,
                                                            unsigned *__restrict__ chunk_counts) {
    __shared__ unsigned part[4];
    const long long w = (long long)blockIdx.x * 256 + threadIdx.x;
    unsigned c = w < words ? (unsigned)__popc(group_bits(marks, w)) : 0u;
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) chunk_counts[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// In-order compaction of the marked cells: chunk c starts at the sum of the
// earlier chunks' counts; inside a chunk, each thread's word starts at the
// exclusive scan of the words' popcounts, and its set bits follow in
// ascending order.  Rows past the capacity are dropped (their cells stay
// empty).  The groups are cleared for the next strided conv.
__global__ __launch_bounds__(256) void compact_write_kernel(
    unsigned char *__restrict__ marks, long long words, const unsigned *__restrict__ chunk_counts,
    int chunks, unsigned capacity, Grid g, int *__restrict__ grid, bf_coord4 *__restrict__ coords,
    unsigned *__restrict__ count_out) {
    __shared__ unsigned part[4], wave_total[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    unsigned before = 0, total = 0;
    for (int c = t; c < chunks; c += 256) {
        const unsigned v = chunk_counts[c];
        before += c < (int)blockIdx.x ? v : 0u;
        total += v;
    }
    for (int o = 32; o > 0; o >>= 1) {
        before += __shfl_xor(before, o);
        total += __shfl_xor(total, o);
    }
    if (lane == 0) {
        part[wave] = before;
        wave_total[wave] = total;
    }
    __syncthreads();
    const unsigned base = part[0] + part[1] + part[2] + part[3];
    if (blockIdx.x == 0 && t == 0) {
        const unsigned all = wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
        *count_out = all < capacity ? all : capacity;
    }
    __syncthreads();
    const long long w = (long long)blockIdx.x * 256 + t;
    unsigned bits = 0;
    if (w < words) {
        bits = group_bits(marks, w);
        if (bits) {
            uint4 *p = reinterpret_cast<uint4 *>(marks + w * 32);
            p[0] = make_uint4(0u, 0u, 0u, 0u);
            p[1] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    const unsigned c = (unsigned)__popc(bits);
    unsigned inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
    }
    if (lane == 63) part[wave] = inc;
    __syncthreads();
    unsigned idx = base + inc - c;
    for (int w2 = 0; w2 < wave; ++w2) idx += part[w2];
    while (bits) {
        const int b = __ffs(bits) - 1;
        bits &= bits - 1;
        if (idx < capacity) {
            long long q = w * 32 + b;
            grid[q] = (int)idx;
            const int x = (int)(q % g.w);
            q /= g.w;
            const int y = (int)(q % g.h);
            q /= g.h;
            const int z = (int)(q % g.d);
            coords[idx] = bf_coord4{(int)(q / g.d), z, y, x};
        }
        ++idx;
    }
}

// Input SubM conv, 5 -> 16 channels, fp32 on the vector units; output fp16.
__device__ __forceinline__ void split_store(float v, _Float16 *hi, _Float16 *lo) {
    const _Float16 h = (_Float16)v;
    *hi = h;
    *lo = (_Float16)(v - (float)h);
}

__global__ __launch_bounds__(256) void conv_input_kernel(const int *__restrict__ nbr,
                                                         const unsigned *__restrict__ count,
                                                         const float *__restrict__ feat,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ bias,
                                                         _Float16 *__restrict__ out_hi,
                                                         _Float16 *__restrict__ out_lo) {
    const unsigned n = *count;
    for (unsigned j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        float acc[16];
#pragma unroll
        for (int co = 0; co < 16; ++co) acc[co] = bias[co];
        for (int t = 0; t < kTaps; ++t) {
            const int src = nbr[(size_t)j * kTaps + t];
            if (src < 0) continue;
            const float *x = feat + (size_t)src * 5;
#pragma unroll
            for (int ci = 0; ci < 5; ++ci) {
                const float xv = x[ci];
#pragma unroll
                for (int co = 0; co < 16; ++co) acc[co] = fmaf(xv, w[(t * 5 + ci) * 16 + co], acc[co]);
            }
        }
        h8 hi[2], lo[2];
#pragma unroll
        for (int co = 0; co < 16; ++co) {
            const float v = fmaxf(acc[co], 0.0f);
            const _Float16 h = (_Float16)v;
            hi[co >> 3][co & 7] = h;
            lo[co >> 3][co & 7] = (_Float16)(v - (float)h);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            *(h8 *)&out_hi[(size_t)j * 16 + 8 * q] = hi[q];
            *(h8 *)&out_lo[(size_t)j * 16 + 8 * q] = lo[q];
        }
    }
}

template <int CI>
struct KOp {
    static constexpr int kb = CI >= 32 ? 32 : 16;  // k per MFMA
    typedef typename std::conditional<(CI >= 32), h8, h4>::type frag;
    static constexpr int per_lane = CI >= 32 ? 8 : 4;
    __device__ static f32x4 mfma(frag a, frag b, f32x4 c) {
        if constexpr (CI >= 32) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
        else return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

// Split fp16 feature planes of one level (rows x channels each).
struct Feat {
    _Float16 *hi, *lo;
};

// LDS plan of one conv instantiation: the split weights of TPB taps, double
// buffered, rows padded by 8 halves so the 16 lanes of a fragment read spread
// over the banks; then the workgroup's neighbour table and active-tap list.
// CO here is the workgroup's output columns; BUFS is 2 (double buffered) or 1.
template <int CI, int CO, int BUFS = 2, int TPB = 1>
struct ConvLds {
    static constexpr int LD = CI + 8;        // halves per weight row in LDS
    static constexpr int PLANE = CO * LD;    // halves per hi or lo plane
    static constexpr int CHUNKS = 2 * CO * CI / 8;  // 16-byte pieces of one tap (hi + lo)
    static constexpr int PER = (CHUNKS + 255) / 256;
    static constexpr size_t W_BYTES = (size_t)BUFS * TPB * 2 * PLANE * sizeof(_Float16);
    static constexpr size_t NBR_BYTES = (size_t)kRowsPerGroup * kTaps * sizeof(int);
    static constexpr size_t BYTES = W_BYTES + NBR_BYTES + 32 * sizeof(int);
};

// Workgroup shape per layer width: output columns per workgroup and weight
// buffers.  The 128-channel convs split their columns in two and stage one
// tap at a time: 49 KB of LDS instead of 153 KB, so two workgroups share a
// CU (the level-3 convs otherwise run one wave per SIMD), at the price of
// gathering each feature row twice.  The 32-channel convs, with little math
// per tap, stage two taps per barrier (TPB): 3% off the encoder on MI355X,
// where three taps cost a wave per SIMD and lost, and two taps for the
// 64-channel convs would do the same.
template <int CI, int CO>
struct ConvShape {
    static constexpr int COW = CI == 128 ? 64 : CO;
    static constexpr int BUFS = CI == 128 ? 1 : 2;
    static constexpr int TPB = CI == 32 ? 2 : 1;
};

// Tap groups: a level with few rows has few 128-row workgroups, each walking
// every tap in turn while most CUs idle, so up to kTapGroups workgroups share
// a row block, each taking a contiguous part of its active-tap list and
// writing fp32 partial sums; split_reduce_kernel adds them in group order.
// Whether to split is decided on the device from the row count (the launch
// carries the groups and the extra ones exit), so one graph fits any frame.
constexpr int kTapGroups = 4;
constexpr unsigned kSplitRows = 16384;  // split at most this many rows

__device__ __forceinline__ int tap_groups(unsigned n, int launched) {
    return n <= kSplitRows ? launched : 1;
}

// Gather GEMM: out[r][co] = bias[co] + sum_t sum_ci in[nbr[r][t]][ci] w[t][co][ci]
// (+ identity[r][co]) (ReLU), operands split as hi + lo.  A workgroup owns
// 128 rows x COW of the CO columns (blockIdx.z picks the slice); each wave
// 32 rows (two 16-row MFMA tiles).  Taps go in chunks of TPB per barrier.
// BUFS = 1 stages one chunk's weights at a time (two barriers per chunk) to
// leave room for more workgroups per CU.
// blockIdx.y is the tap group; with several groups in effect the workgroup
// writes its fp32 partial sums to `part` [group][row][co] instead.
// Per workgroup: the rows' neighbour lists go to LDS and the taps some row
// uses are listed; per chunk of listed taps the split weights [co][ci] are
// staged in LDS (double buffered: the next chunk's weights are fetched into
// registers while this chunk's MFMAs run) and every wave reads its B
// fragments there, so a weight leaves L2 once per 128 rows instead of once
// per 32.  A fragments are gathered straight from the feature rows, one chunk
// ahead.  Taps are summed in list order whatever TPB is.  A wave skips
// the MFMAs of a tap none of its rows reaches.  out32, when set, receives
// fp32 rows instead of a split pair.
template <int CI, int CO, int COW, int BUFS, int TPB>
__global__ __launch_bounds__(256) void sparse_conv_kernel(
    const int *__restrict__ nbr, const unsigned *__restrict__ count, int taps, Feat in,
    const _Float16 *__restrict__ w_hi, const _Float16 *__restrict__ w_lo,
    const float *__restrict__ bias, Feat identity, int relu, Feat out,
    float *__restrict__ out32, float *__restrict__ part) {
    using K = KOp<CI>;
    using L = ConvLds<CI, COW, BUFS, TPB>;
    typedef typename K::frag frag;
    constexpr int CT = COW / 16, KC = CI / K::kb;
    const int co0 = (int)blockIdx.z * COW;
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16 *sw = reinterpret_cast<_Float16 *>(smem);  // [buffer][hi, lo][CO][LD]
    int *snbr = reinterpret_cast<int *>(smem + L::W_BYTES);  // [row][kTaps]
    int *stap = snbr + kRowsPerGroup * kTaps;                // [0] mask, [1] count, [2..] list
    const unsigned n = *count;
    const int groups = tap_groups(n, (int)gridDim.y), group = (int)blockIdx.y;
    if (group >= groups) return;  // whole workgroup: before any barrier
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 15, g = lane >> 4;
    const int wrow = wave * kRowsPerWave;

    // 16-byte pieces of tap t's weights: piece c < CHUNKS/2 of the hi plane,
    // the rest of the lo plane; row cc / (CI/8), halves k..k+7.
    auto fetch = [&](int t, h8 (&reg)[L::PER]) {
#pragma unroll
        for (int q = 0; q < L::PER; ++q) {
            const int c = tid + 256 * q;
            if (c < L::CHUNKS) {
                const int half = c >= L::CHUNKS / 2, cc = c - half * (L::CHUNKS / 2);
                const _Float16 *src = (half ? w_lo : w_hi) + ((size_t)t * CO + co0) * CI +
                                      (size_t)cc * 8;
                reg[q] = *reinterpret_cast<const h8 *>(src);
            }
        }
    };
    auto stage = [&](int buf, const h8 (&reg)[L::PER]) {
#pragma unroll
        for (int q = 0; q < L::PER; ++q) {
            const int c = tid + 256 * q;
            if (c < L::CHUNKS) {
                const int half = c >= L::CHUNKS / 2, cc = c - half * (L::CHUNKS / 2);
                const int co = cc / (CI / 8), k = (cc % (CI / 8)) * 8;
                *reinterpret_cast<h8 *>(sw + (size_t)(2 * buf + half) * L::PLANE + co * L::LD + k) =
                    reg[q];
            }
        }
    };
    auto gather = [&](int t, frag (&ah)[2][KC], frag (&al)[2][KC], bool (&live)[2]) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int src = snbr[(wrow + 16 * rt + col) * kTaps + t];
            live[rt] = src >= 0;
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) {
                const int k0 = kc * K::kb + g * K::per_lane;
                if (src >= 0) {
                    ah[rt][kc] = *(const frag *)&in.hi[(size_t)src * CI + k0];
                    al[rt][kc] = *(const frag *)&in.lo[(size_t)src * CI + k0];
                } else {
                    ah[rt][kc] = frag{};
                    al[rt][kc] = frag{};
                }
            }
        }
    };

    for (unsigned base = blockIdx.x * kRowsPerGroup; base < n; base += gridDim.x * kRowsPerGroup) {
        if (tid == 0) stap[0] = 0;
        __syncthreads();
        unsigned used = 0;
        for (int i = tid; i < kRowsPerGroup * taps; i += 256) {
            const int r = i / taps, t = i - r * taps;
            const int v = base + r < n ? nbr[(size_t)(base + r) * kTaps + t] : kEmpty;
            snbr[r * kTaps + t] = v;
            if (v >= 0) used |= 1u << t;
        }
        for (int o = 32; o > 0; o >>= 1) used |= __shfl_xor(used, o);
        if (lane == 0) atomicOr(reinterpret_cast<unsigned *>(stap), used);
        __syncthreads();
        if (tid == 0) {
            const unsigned m = (unsigned)stap[0];
            int c = 0;
            for (int t = 0; t < taps; ++t)
                if (m >> t & 1u) stap[2 + c++] = t;
            stap[1] = c;
        }
        __syncthreads();
        // This group's part of the active-tap list: entries [first, last).
        const int listed = stap[1], per = (listed + groups - 1) / groups;
        const int first = min(listed, group * per), last = min(listed, first + per);
        const int *list = stap + 2 + first;
        const int active = last - first;

        f32x4 acc[2][CT];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // Chunk c holds list entries [c * TPB, min(active, c * TPB + TPB)).
        const int chunks = (active + TPB - 1) / TPB;
        h8 wreg[TPB][L::PER];
        frag ah[TPB][2][KC], al[TPB][2][KC];
        bool live[TPB][2] = {};
        // Callers pass chunks that exist, so with TPB = 1 every entry does.
        auto fetch_chunk = [&](int c) {
#pragma unroll
            for (int u = 0; u < TPB; ++u)
                if (TPB == 1 || c * TPB + u < active) fetch(list[c * TPB + u], wreg[u]);
        };
        auto stage_chunk = [&](int buf, int c) {
#pragma unroll
            for (int u = 0; u < TPB; ++u)
                if (TPB == 1 || c * TPB + u < active) stage(buf * TPB + u, wreg[u]);
        };
        auto gather_chunk = [&](int c, frag (&h)[TPB][2][KC], frag (&lo)[TPB][2][KC],
                                bool (&lv)[TPB][2]) {
#pragma unroll
            for (int u = 0; u < TPB; ++u)  // entries past the end keep lv false
                if (TPB == 1 || c * TPB + u < active) gather(list[c * TPB + u], h[u], lo[u], lv[u]);
        };
        if (chunks) {
            fetch_chunk(0);
            stage_chunk(0, 0);
            gather_chunk(0, ah, al, live);
        }
        __syncthreads();
        for (int c = 0; c < chunks; ++c) {
            const int buf = BUFS == 2 ? c & 1 : 0;
            const bool more = c + 1 < chunks;
            if (more) fetch_chunk(c + 1);
            frag nh[TPB][2][KC], nl[TPB][2][KC];
            bool nlive[TPB][2] = {};
            if (more) gather_chunk(c + 1, nh, nl, nlive);
#pragma unroll
            for (int u = 0; u < TPB; ++u) {
                // Wave-uniform: a tap none of the wave's rows reaches (or an
                // entry past the list's end) adds nothing.
                if (__ballot(live[u][0] || live[u][1])) {
                    const _Float16 *bh_base = sw + (size_t)(2 * (buf * TPB + u)) * L::PLANE;
                    const _Float16 *bl_base = bh_base + L::PLANE;
#pragma unroll
                    for (int kc = 0; kc < KC; ++kc) {
                        const int k0 = kc * K::kb + g * K::per_lane;
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct) {
                            const int wo = (16 * ct + col) * L::LD + k0;
                            const frag bh = *(const frag *)&bh_base[wo];
                            const frag bl = *(const frag *)&bl_base[wo];
#pragma unroll
                            for (int rt = 0; rt < 2; ++rt) {
                                acc[rt][ct] = K::mfma(al[u][rt][kc], bh, acc[rt][ct]);
                                acc[rt][ct] = K::mfma(ah[u][rt][kc], bl, acc[rt][ct]);
                                acc[rt][ct] = K::mfma(ah[u][rt][kc], bh, acc[rt][ct]);
                            }
                        }
                    }
                }
            }
            if (more) {
                if (BUFS == 1) __syncthreads();  // every wave is done with this chunk's weights
                stage_chunk(BUFS == 2 ? buf ^ 1 : 0, c + 1);
#pragma unroll
                for (int u = 0; u < TPB; ++u)
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) {
                        live[u][rt] = nlive[u][rt];
#pragma unroll
                        for (int kc = 0; kc < KC; ++kc) {
                            ah[u][rt][kc] = nh[u][rt][kc];
                            al[u][rt][kc] = nl[u][rt][kc];
                        }
                    }
            }
            __syncthreads();
        }
        const unsigned row0 = base + wrow;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int co = co0 + 16 * ct + col;
            const float b = bias[co];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const unsigned r = row0 + 16 * rt + 4 * g + j;
                    if (r >= n) continue;
                    const size_t at = (size_t)r * CO + co;
                    if (groups > 1) {
                        part[((size_t)group * kSplitRows + r) * CO + co] = acc[rt][ct][j];
                        continue;
                    }
                    float v = acc[rt][ct][j] + b;
                    if (identity.hi) v += (float)identity.hi[at] + (float)identity.lo[at];
                    if (relu) v = fmaxf(v, 0.0f);
                    if (out32) out32[at] = v;
                    else split_store(v, out.hi + at, out.lo + at);
                }
        }
        __syncthreads();  // LDS is rewritten by the next row group
    }
}

// Sum of the tap groups' partials in group order, then bias, residual and
// ReLU; nothing to do when the conv ran unsplit.
template <int CO>
__global__ __launch_bounds__(256) void split_reduce_kernel(
    const unsigned *__restrict__ count, int launched, const float *__restrict__ part,
    const float *__restrict__ bias, Feat identity, int relu, Feat out, float *__restrict__ out32) {
    const unsigned n = *count;
    const int groups = tap_groups(n, launched);
    if (groups == 1) return;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < (size_t)n * CO;
         e += (size_t)gridDim.x * 256) {
        const int co = (int)(e % CO);
        float v = 0.0f;
        for (int gi = 0; gi < groups; ++gi) v += part[(size_t)gi * kSplitRows * CO + e];
        v += bias[co];
        if (identity.hi) v += (float)identity.hi[e] + (float)identity.lo[e];
        if (relu) v = fmaxf(v, 0.0f);
        if (out32) out32[e] = v;
        else split_store(v, out.hi + e, out.lo + e);
    }
}

// Gather GEMM for the 16-channel-input layers of the finest level: there
// is little math per tap, so the time is the latency of each tap's gather.
// A workgroup owns 32 rows x all CO; its four waves take the active taps in
// turn (wave w: list entries w, w + 4, ...), each keeping the next tap's
// feature and weight fragments in flight while it multiplies the current
// one; the weights ([co][ci] per tap, a few KB) stay in L1/L2.  The four
// partial sums meet in LDS and are added in wave order (deterministic), then
// bias, residual and ReLU are applied on coalesced rows.
template <int CI, int CO>
__global__ __launch_bounds__(256) void sparse_conv_split_kernel(
    const int *__restrict__ nbr, const unsigned *__restrict__ count, int taps, Feat in,
    const _Float16 *__restrict__ w_hi, const _Float16 *__restrict__ w_lo,
    const float *__restrict__ bias, Feat identity, int relu, Feat out,
    float *__restrict__ out32) {
    using K = KOp<CI>;
    typedef typename K::frag frag;
    constexpr int CT = CO / 16, KC = CI / K::kb, R = 32;
    __shared__ int snbr[R * kTaps];
    __shared__ int stap[2 + kTaps];
    __shared__ float part[4][R][CO + 1];
    const unsigned n = *count;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 15, g = lane >> 4;

    struct Frags {
        frag ah[2][KC], al[2][KC], bh[CT][KC], bl[CT][KC];
        bool live;
    };
    auto load = [&](int t, Frags &f) {
        f.live = false;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int src = snbr[(16 * rt + col) * kTaps + t];
            f.live |= src >= 0;
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) {
                const int k0 = kc * K::kb + g * K::per_lane;
                if (src >= 0) {
                    f.ah[rt][kc] = *(const frag *)&in.hi[(size_t)src * CI + k0];
                    f.al[rt][kc] = *(const frag *)&in.lo[(size_t)src * CI + k0];
                } else {
                    f.ah[rt][kc] = frag{};
                    f.al[rt][kc] = frag{};
                }
            }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) {
                const size_t wo = ((size_t)t * CO + 16 * ct + col) * CI + kc * K::kb + g * K::per_lane;
                f.bh[ct][kc] = *(const frag *)&w_hi[wo];
                f.bl[ct][kc] = *(const frag *)&w_lo[wo];
            }
    };

    for (unsigned base = blockIdx.x * R; base < n; base += gridDim.x * R) {
        if (tid == 0) stap[0] = 0;
        __syncthreads();
        unsigned used = 0;
        for (int i = tid; i < R * taps; i += 256) {
            const int r = i / taps, t = i - r * taps;
            const int v = base + r < n ? nbr[(size_t)(base + r) * kTaps + t] : kEmpty;
            snbr[r * kTaps + t] = v;
            if (v >= 0) used |= 1u << t;
        }
        for (int o = 32; o > 0; o >>= 1) used |= __shfl_xor(used, o);
        if (lane == 0) atomicOr(reinterpret_cast<unsigned *>(stap), used);
        __syncthreads();
        if (tid == 0) {
            const unsigned m = (unsigned)stap[0];
            int c = 0;
            for (int t = 0; t < taps; ++t)
                if (m >> t & 1u) stap[2 + c++] = t;
            stap[1] = c;
        }
        __syncthreads();
        const int active = stap[1];

        f32x4 acc[2][CT];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        Frags cur, nxt;
        if (wave < active) load(stap[2 + wave], cur);
        for (int i = wave; i < active; i += 4) {
            const bool more = i + 4 < active;
            if (more) load(stap[2 + i + 4], nxt);
            if (__ballot(cur.live)) {
#pragma unroll
                for (int kc = 0; kc < KC; ++kc)
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                        for (int rt = 0; rt < 2; ++rt) {
                            acc[rt][ct] = K::mfma(cur.al[rt][kc], cur.bh[ct][kc], acc[rt][ct]);
                            acc[rt][ct] = K::mfma(cur.ah[rt][kc], cur.bl[ct][kc], acc[rt][ct]);
                            acc[rt][ct] = K::mfma(cur.ah[rt][kc], cur.bh[ct][kc], acc[rt][ct]);
                        }
            }
            if (more) cur = nxt;
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int j = 0; j < 4; ++j) part[wave][16 * rt + 4 * g + j][16 * ct + col] = acc[rt][ct][j];
        __syncthreads();
        for (int e = tid; e < R * CO; e += 256) {
            const int r = e / CO, co = e - r * CO;
            const unsigned row = base + r;
            if (row >= n) continue;
            const size_t at = (size_t)row * CO + co;
            float v = part[0][r][co] + part[1][r][co] + part[2][r][co] + part[3][r][co] + bias[co];
            if (identity.hi) v += (float)identity.hi[at] + (float)identity.lo[at];
            if (relu) v = fmaxf(v, 0.0f);
            if (out32) out32[at] = v;
            else split_store(v, out.hi + at, out.lo + at);
        }
        __syncthreads();  // LDS is rewritten by the next row group
    }
}

// dense[b][c][z][y][x] = row features of the site at (b, z, y, x), else 0.
// A workgroup takes 64 consecutive cells of one batch: the sites' 128-float
// rows are read whole into LDS and written back channel by channel, so both
// the row reads and the channel-major writes are contiguous.
__global__ __launch_bounds__(256) void dense_kernel(const int *__restrict__ grid, Grid g,
                                                    const float *__restrict__ feat,
                                                    float *__restrict__ dense) {
    __shared__ float tile[64][129];
    __shared__ int rows[64];
    const size_t plane = (size_t)g.d * g.h * g.w;
    const size_t tiles = (plane + 63) / 64;
    for (size_t bt = blockIdx.x; bt < (size_t)g.b * tiles; bt += gridDim.x) {
        const size_t b = bt / tiles, cell0 = (bt % tiles) * 64;
        if (threadIdx.x < 64) {
            const size_t cell = cell0 + threadIdx.x;
            rows[threadIdx.x] = cell < plane ? grid[b * plane + cell] : kEmpty;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < 64 * 128; e += 256) {
            const int k = e >> 7, c = e & 127, idx = rows[k];
            tile[k][c] = idx >= 0 ? feat[(size_t)idx * 128 + c] : 0.0f;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < 64 * 128; e += 256) {
            const int c = e >> 6, k = e & 63;
            const size_t cell = cell0 + k;
            if (cell < plane) dense[(b * 128 + c) * plane + cell] = tile[k][c];
        }
        __syncthreads();
    }
}

struct Conv {
    const _Float16 *w_hi, *w_lo;
    const float *w32, *bias;
    int ci, co, taps;
    Geom q;
};

}  // namespace

struct bf_cuda_lidar_backbone {
    size_t batches, capacity, resident_bytes;
    Grid lv[5];
    long long cells[5];
    int max_chunks;
    unsigned char *params, *work;
    Conv input, res[4][2][2], down[3], out;
    int *grid[5], *nbr;
    bf_coord4 *coords[5];
    unsigned *counts, *chunk_counts;
    unsigned char *marks;
    Feat feat[3];
    float *out32, *part;
};

namespace {

int fold_layer(const bf_model *m, const char *wname, const char *bn, int ci, int co, int kd,
               int kh, int kw, std::vector<float> &w, std::vector<float> &b, char *error,
               size_t cap) {
    const float *src = bind_f32(m, wname, {(uint32_t)kd, (uint32_t)kh, (uint32_t)kw,
                                          (uint32_t)ci, (uint32_t)co}, error, cap);
    if (!src) return 0;
    static const char *suffix[4] = {"weight", "bias", "running_mean", "running_var"};
    const float *p[4];
    char name[192];
    for (int i = 0; i < 4; ++i) {
        std::snprintf(name, sizeof(name), "%s.%s", bn, suffix[i]);
        if (!(p[i] = bind_f32(m, name, {(uint32_t)co}, error, cap))) return 0;
    }
    const int taps = kd * kh * kw;
    w.assign((size_t)taps * ci * co, 0.0f);
    b.assign(co, 0.0f);
    for (int o = 0; o < co; ++o) {
        // Eval BN folded as the reference GPU path (cuda_lidar.cu:41-43).
        const float f = p[0][o] / std::sqrt(p[3][o] + kBnEps);
        b[o] = p[1][o] - p[2][o] * f;
        for (int t = 0; t < taps; ++t)
            for (int i = 0; i < ci; ++i) w[((size_t)t * ci + i) * co + o] = src[((size_t)t * ci + i) * co + o] * f;
    }
    return 1;
}

int axis_out(int in, int k, int s, int p) { return in + 2 * p >= k ? (in + 2 * p - k) / s + 1 : 0; }

int build(bf_cuda_lidar_backbone *n, const bf_model *m, char *error, size_t cap) {
    struct Spec {
        Conv *dst;
        std::string w, bn;
        int ci, co, kd, kh, kw, sd, sh, sw, pd, ph, pw;
    };
    std::vector<Spec> specs;
    specs.push_back({&n->input, "backbone_3d.conv_input.0.weight", "backbone_3d.conv_input.1", 5,
                     16, 3, 3, 3, 1, 1, 1, 1, 1, 1});
    static const int ch[4] = {16, 32, 64, 128};
    char w[160], bn[160];
    for (int s = 0; s < 4; ++s)
        for (int blk = 0; blk < 2; ++blk)
            for (int c = 0; c < 2; ++c) {
                // Layer table of reference cuda_lidar.cu:96-100.
                std::snprintf(w, sizeof(w), "backbone_3d.conv%d.%d.conv%d.weight", s + 1,
                              blk + (s ? 1 : 0), c + 1);
                std::snprintf(bn, sizeof(bn), "backbone_3d.conv%d.%d.bn%d", s + 1,
                              blk + (s ? 1 : 0), c + 1);
                specs.push_back({&n->res[s][blk][c], w, bn, ch[s], ch[s], 3, 3, 3, 1, 1, 1, 1, 1, 1});
            }
    for (int t = 0; t < 3; ++t) {
        std::snprintf(w, sizeof(w), "backbone_3d.conv%d.0.0.weight", t + 2);
        std::snprintf(bn, sizeof(bn), "backbone_3d.conv%d.0.1", t + 2);
        specs.push_back({&n->down[t], w, bn, ch[t], ch[t + 1], 3, 3, 3, 2, 2, 2, t == 2 ? 0 : 1, 1, 1});
    }
    specs.push_back({&n->out, "backbone_3d.conv_out.0.weight", "backbone_3d.conv_out.1", 128, 128,
                     3, 1, 1, 2, 1, 1, 0, 0, 0});
    ParamArena pa;
    struct Off {
        size_t w, w_lo, b;
        bool f32;
    };
    std::vector<Off> offs;
    for (const Spec &sp : specs) {
        std::vector<float> wf, bf;
        if (!fold_layer(m, sp.w.c_str(), sp.bn.c_str(), sp.ci, sp.co, sp.kd, sp.kh, sp.kw, wf, bf,
                        error, cap))
            return 0;
        const int taps = sp.kd * sp.kh * sp.kw;
        Off o{};
        o.f32 = sp.ci == 5;
        if (o.f32) {
            o.w = pa.add_f32(wf);  // [tap][ci][co]
        } else {
            std::vector<float> t((size_t)taps * sp.co * sp.ci);  // [tap][co][ci]
            for (int k = 0; k < taps; ++k)
                for (int i = 0; i < sp.ci; ++i)
                    for (int c = 0; c < sp.co; ++c)
                        t[((size_t)k * sp.co + c) * sp.ci + i] = wf[((size_t)k * sp.ci + i) * sp.co + c];
            // Split pair: hi = fp16(w), lo = fp16(w - hi).
            std::vector<float> lo(t.size());
            for (size_t i = 0; i < t.size(); ++i)
                lo[i] = t[i] - (float)(_Float16)t[i];
            o.w = pa.add_f16(t);
            o.w_lo = pa.add_f16(lo);
        }
        o.b = pa.add_f32(bf);
        offs.push_back(o);
        *sp.dst = Conv{nullptr, nullptr, nullptr, nullptr, sp.ci, sp.co, taps,
                       Geom{sp.kd, sp.kh, sp.kw, sp.sd, sp.sh, sp.sw, sp.pd, sp.ph, sp.pw}};
    }
    if (!hip_ok(hipMalloc((void **)&n->params, pa.host.size()), error, cap,
                "allocate LiDAR weights") ||
        !hip_ok(hipMemcpy(n->params, pa.host.data(), pa.host.size(), hipMemcpyHostToDevice), error,
                cap, "upload LiDAR weights"))
        return 0;
    n->resident_bytes += pa.host.size();
    for (size_t i = 0; i < specs.size(); ++i) {
        Conv &c = *specs[i].dst;
        if (offs[i].f32) c.w32 = (const float *)(n->params + offs[i].w);
        else {
            c.w_hi = (const _Float16 *)(n->params + offs[i].w);
            c.w_lo = (const _Float16 *)(n->params + offs[i].w_lo);
        }
        c.bias = (const float *)(n->params + offs[i].b);
    }
    // Work buffers.
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~size_t(255);
        return at;
    };
    size_t o_grid[5], o_coords[5];
    long long max_cells = 0;
    for (int l = 0; l < 5; ++l) {
        o_grid[l] = take((size_t)n->cells[l] * sizeof(int));
        o_coords[l] = take(n->capacity * sizeof(bf_coord4));
        max_cells = std::max(max_cells, l ? n->cells[l] : 0);
    }
    n->max_chunks = (int)((max_cells + kChunk - 1) / kChunk);
    const size_t o_nbr = take(n->capacity * kTaps * sizeof(int));
    const size_t o_counts = take(8 * sizeof(unsigned));
    const size_t o_chunks = take((size_t)std::max(n->max_chunks, 1) * sizeof(unsigned));
    const size_t mark_bytes = (size_t)std::max(n->max_chunks, 1) * kChunk;  // whole chunks
    const size_t o_marks = take(mark_bytes);
    size_t o_feat[3];
    for (int i = 0; i < 3; ++i) o_feat[i] = take(2 * n->capacity * 128 * sizeof(_Float16));
    const size_t o_out = take(n->capacity * 128 * sizeof(float));
    const size_t o_part = take((size_t)kTapGroups * kSplitRows * 128 * sizeof(float));
    if (!hip_ok(hipMalloc((void **)&n->work, off), error, cap, "allocate LiDAR workspace"))
        return 0;
    n->resident_bytes += off;
    unsigned char *a = n->work;
    for (int l = 0; l < 5; ++l) {
        n->grid[l] = (int *)(a + o_grid[l]);
        n->coords[l] = (bf_coord4 *)(a + o_coords[l]);
        // Every index grid is -1 between forwards.
        if (!hip_ok(hipMemset(n->grid[l], 0xff, (size_t)n->cells[l] * sizeof(int)), error, cap,
                    "clear LiDAR index grid"))
            return 0;
    }
    n->nbr = (int *)(a + o_nbr);
    n->counts = (unsigned *)(a + o_counts);
    n->chunk_counts = (unsigned *)(a + o_chunks);
    n->marks = a + o_marks;
    // The mark map is clear between strided convs: each compaction clears it.
    if (!hip_ok(hipMemset(n->marks, 0, mark_bytes), error, cap, "clear LiDAR mark map"))
        return 0;
    for (int i = 0; i < 3; ++i) {
        n->feat[i].hi = (_Float16 *)(a + o_feat[i]);
        n->feat[i].lo = n->feat[i].hi + n->capacity * 128;
    }
    n->out32 = (float *)(a + o_out);
    n->part = (float *)(a + o_part);
    return 1;
}

unsigned nbr_blocks(const bf_cuda_lidar_backbone *n) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>(16384, (n->capacity * kTaps + 255) / 256));
}

unsigned row_blocks(size_t capacity, int rows_per_block) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>(2048, (capacity + rows_per_block - 1) / rows_per_block));
}

void launch_conv(const bf_cuda_lidar_backbone *n, const Conv &c, const unsigned *count,
                 Feat in, Feat identity, int relu, Feat out, float *out32, hipStream_t s) {
    const unsigned blocks = row_blocks(n->capacity, kRowsPerGroup);
    const unsigned split_blocks =
        (unsigned)std::max<size_t>(1, std::min<size_t>(16384, (n->capacity + 31) / 32));
#define BF_SPLIT(CI, CO)                                                                       \
    if (c.ci == CI && c.co == CO) {                                                            \
        sparse_conv_split_kernel<CI, CO><<<split_blocks, 256, 0, s>>>(                         \
            n->nbr, count, c.taps, in, c.w_hi, c.w_lo, c.bias, identity, relu, out, out32);    \
        return;                                                                                \
    }
    BF_SPLIT(16, 16)
    BF_SPLIT(16, 32)
#undef BF_SPLIT
#define BF_CONV(CI, CO)                                                                        \
    if (c.ci == CI && c.co == CO) {                                                            \
        using S = ConvShape<CI, CO>;                                                           \
        const int groups = CI >= 64 ? kTapGroups : 1;                                          \
        sparse_conv_kernel<CI, CO, S::COW, S::BUFS, S::TPB>                                            \
            <<<dim3(blocks, groups, CO / S::COW), 256, ConvLds<CI, S::COW, S::BUFS, S::TPB>::BYTES,    \
               s>>>(n->nbr, count, c.taps, in, c.w_hi, c.w_lo, c.bias, identity, relu, out,    \
                    out32, n->part);                                                           \
        if (groups > 1)                                                                        \
            split_reduce_kernel<CO><<<1024, 256, 0, s>>>(count, groups, n->part, c.bias,       \
                                                         identity, relu, out, out32);          \
        return;                                                                                \
    }
    BF_CONV(32, 32)
    BF_CONV(32, 64)
    BF_CONV(64, 64)
    BF_CONV(64, 128)
    BF_CONV(128, 128)
#undef BF_CONV
}

// Marks and compacts the output sites of strided conv `c` from level l into
// level l + 1, then builds its output -> input neighbour table.
void strided_sites(bf_cuda_lidar_backbone *n, const Conv &c, int l, const bf_coord4 *in_coords,
                   hipStream_t s) {
    const unsigned rb = row_blocks(n->capacity, 256);
    mark_kernel<<<rb, 256, 0, s>>>(in_coords, n->counts + l, n->lv[l + 1], c.q, n->marks);
    const int chunks = (int)((n->cells[l + 1] + kChunk - 1) / kChunk);
    const long long words = (n->cells[l + 1] + 31) / 32;
    compact_count_kernel<<<chunks, 256, 0, s>>>(n->marks, words, n->chunk_counts);
    compact_write_kernel<<<chunks, 256, 0, s>>>(n->marks, words, n->chunk_counts, chunks,
                                                (unsigned)n->capacity, n->lv[l + 1], n->grid[l + 1],
                                                n->coords[l + 1], n->counts + l + 1);
    down_neighbors_kernel<<<nbr_blocks(n), 256, 0, s>>>(n->coords[l + 1], n->counts + l + 1,
                                                        n->lv[l], c.q, n->grid[l], n->nbr);
}

void forward_impl(bf_cuda_lidar_backbone *n, const bf_coord4 *coords, const float *feats,
                  const unsigned *count_dev, unsigned count_host, float *dense, hipStream_t s) {
    const unsigned rb = row_blocks(n->capacity, 256);
    count_init_kernel<<<1, 1, 0, s>>>(count_dev, count_host, (unsigned)n->capacity, n->counts);
    index_kernel<<<rb, 256, 0, s>>>(coords, n->counts, n->lv[0], n->grid[0]);
    subm_neighbors_kernel<<<nbr_blocks(n), 256, 0, s>>>(coords, n->counts, n->lv[0], n->grid[0],
                                                        n->nbr);
    conv_input_kernel<<<rb, 256, 0, s>>>(n->nbr, n->counts, feats, n->input.w32, n->input.bias,
                                         n->feat[0].hi, n->feat[0].lo);
    const Feat none{nullptr, nullptr};
    int x = 0;
    const bf_coord4 *level_coords = coords;
    for (int st = 0; st < 4; ++st) {
        const unsigned *cnt = n->counts + st;
        if (st) {
            strided_sites(n, n->down[st - 1], st - 1, level_coords, s);
            const int y = (x + 1) % 3;
            launch_conv(n, n->down[st - 1], cnt, n->feat[x], none, 1, n->feat[y], nullptr, s);
            x = y;
            level_coords = n->coords[st];
            subm_neighbors_kernel<<<nbr_blocks(n), 256, 0, s>>>(level_coords, cnt, n->lv[st],
                                                                n->grid[st], n->nbr);
        }
        for (int blk = 0; blk < 2; ++blk) {
            const int y = (x + 1) % 3, z = (x + 2) % 3;
            launch_conv(n, n->res[st][blk][0], cnt, n->feat[x], none, 1, n->feat[y], nullptr, s);
            launch_conv(n, n->res[st][blk][1], cnt, n->feat[y], n->feat[x], 1, n->feat[z], nullptr,
                        s);
            x = z;
        }
    }
    strided_sites(n, n->out, 3, level_coords, s);
    launch_conv(n, n->out, n->counts + 4, n->feat[x], none, 1, none, n->out32, s);
    const size_t dense_tiles = (size_t)n->lv[4].b * (((size_t)n->cells[4] / n->lv[4].b + 63) / 64);
    dense_kernel<<<(unsigned)std::min<size_t>(16384, dense_tiles), 256, 0, s>>>(
        n->grid[4], n->lv[4], n->out32, dense);
    LevelGrids lg;
    for (int l = 0; l < 5; ++l) {
        lg.coords[l] = l ? n->coords[l] : coords;
        lg.count[l] = n->counts + l;
        lg.grid[l] = n->grid[l];
        lg.g[l] = n->lv[l];
    }
    clear_kernel<<<dim3(rb, 5), 256, 0, s>>>(lg);
}

}  // namespace

extern "C" void bf_cuda_lidar_backbone_destroy(bf_cuda_lidar_backbone *n) {
    if (!n) return;
    if (n->params) (void)hipFree(n->params);
    if (n->work) (void)hipFree(n->work);
    std::free(n);
}

extern "C" size_t bf_cuda_lidar_backbone_resident_bytes(const bf_cuda_lidar_backbone *n) {
    return n ? n->resident_bytes : 0;
}

namespace {

template <int CI, int CO>
int allow_lds(char *error, size_t cap) {
    using S = ConvShape<CI, CO>;
    return hip_ok(hipFuncSetAttribute(
                      reinterpret_cast<const void *>(&sparse_conv_kernel<CI, CO, S::COW, S::BUFS, S::TPB>),
                      hipFuncAttributeMaxDynamicSharedMemorySize,
                      (int)ConvLds<CI, S::COW, S::BUFS, S::TPB>::BYTES),
                  error, cap, "set LiDAR conv LDS size");
}

}  // namespace

extern "C" int bf_cuda_lidar_backbone_create(const bf_model *model, size_t batches, size_t d,
                                             size_t h, size_t w, size_t capacity,
                                             bf_cuda_lidar_backbone **out, char *error,
                                             size_t cap) {
    if (out) *out = nullptr;
    if (!model || !out || !batches || !d || !h || !w || !capacity || batches > INT_MAX ||
        d > INT_MAX || h > INT_MAX || w > INT_MAX || capacity > UINT_MAX)
        return fail(error, cap, "invalid HIP LiDAR contract");
    if (capacity > (size_t)INT_MAX / kTaps)
        return fail(error, cap, "HIP LiDAR capacity is too large");
    bf_cuda_lidar_backbone *n = (bf_cuda_lidar_backbone *)std::calloc(1, sizeof(*n));
    if (!n) return fail(error, cap, "HIP LiDAR allocation failed");
    n->batches = batches;
    n->capacity = capacity;
    // Level shapes (lidar_backbone.c:147-162).
    Grid g{(int)batches, (int)d, (int)h, (int)w};
    n->lv[0] = g;
    static const int pz[3] = {1, 1, 0};
    for (int l = 1; l < 4; ++l) {
        g = Grid{g.b, axis_out(g.d, 3, 2, pz[l - 1]), axis_out(g.h, 3, 2, 1), axis_out(g.w, 3, 2, 1)};
        n->lv[l] = g;
    }
    n->lv[4] = Grid{g.b, axis_out(g.d, 3, 2, 0), g.h, g.w};
    for (int l = 0; l < 5; ++l) {
        if (n->lv[l].d <= 0 || n->lv[l].h <= 0 || n->lv[l].w <= 0) {
            bf_cuda_lidar_backbone_destroy(n);
            return fail(error, cap, "invalid HIP LiDAR output shape");
        }
        n->cells[l] = (long long)n->lv[l].b * n->lv[l].d * n->lv[l].h * n->lv[l].w;
    }
    if (!allow_lds<32, 32>(error, cap) || !allow_lds<32, 64>(error, cap) ||
        !allow_lds<64, 64>(error, cap) || !allow_lds<64, 128>(error, cap) ||
        !allow_lds<128, 128>(error, cap) || !build(n, model, error, cap)) {
        bf_cuda_lidar_backbone_destroy(n);
        return 0;
    }
    *out = n;
    return 1;
}

extern "C" int bf_cuda_lidar_backbone_forward(bf_cuda_lidar_backbone *n, const bf_coord4 *coords,
                                              const float *feats, size_t count, float *dense,
                                              void *stream, char *error, size_t cap) {
    if (!n || !coords || !feats || !count || count > n->capacity || !dense)
        return fail(error, cap, "invalid HIP LiDAR buffers");
    forward_impl(n, coords, feats, nullptr, (unsigned)count, dense,
                 reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "HIP LiDAR launch");
}

extern "C" int bf_cuda_lidar_backbone_forward_count_device(bf_cuda_lidar_backbone *n,
                                                           const bf_coord4 *coords,
                                                           const float *feats,
                                                           const unsigned *count, float *dense,
                                                           void *stream, char *error,
                                                           size_t cap) {
    if (!n || !coords || !feats || !count || !dense)
        return fail(error, cap, "invalid device-count HIP LiDAR buffers");
    forward_impl(n, coords, feats, count, 0u, dense, reinterpret_cast<hipStream_t>(stream));
    return launch_ok(error, cap, "HIP LiDAR launch");
}
