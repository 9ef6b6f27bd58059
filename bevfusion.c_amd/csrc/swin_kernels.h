// Swin-T building blocks on gfx950: the stage-output LayerNorm with
// NHWC->NCHW store and batched shifted-window attention on MFMA (the patch
// merges run as LN-folded GEMMs, ln_fold.h).  The Swin path's 16-bit operands (LayerNorm
// outputs, QKV, attention terms and output, MLP hidden, weights) are fp16
// words held in the bf16 container type, multiplied on the fp16 MFMA with
// fp32 accumulation.
#pragma once

#include "hip_common.h"
#include "ln_fold.h"

namespace bfhip {

__device__ __forceinline__ void store4(float *p, float a, float b, float c, float d) {
    *reinterpret_cast<float4 *>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void store4(bf16 *p, float a, float b, float c, float d) {
    bf16x4 v;  // fp16 words
    v[0] = to_half(a); v[1] = to_half(b); v[2] = to_half(c); v[3] = to_half(d);
    *reinterpret_cast<bf16x4 *>(p) = v;
}

// Stage output: LayerNorm over C = 64 G channels of tokens [n, hw, C], stored
// NCHW (reference store_output, swin_backbone.c:265-276).  The row statistics
// are the (mean, M2) partials per 64-channel group that the stage's last
// residual writer left in `stats` (row r: stats[r * G + g]), so a block can
// own a kR-token x 64-channel tile: it reads the tile as 256-byte row
// segments, normalises it into LDS transposed, and writes kR-token runs of
// each of its 64 channel planes, as float4 when `vec` (hw % 4 == 0 and out
// 16-byte aligned: four tokens from a multiple of 4 never straddle two
// images), else per element.  block() is tile (bx, by) with THREADS threads
// on `smem` (kSmem bytes); out_ln_kernel runs grid (ceil(rows / kR), G) of
// them with 256 threads, and a kernel that fuses it with other work calls
// block() for part of its grid.
struct OutLnArgs {
    const float *x;
    const float2 *stats;
    float *out;
    const float *g, *b;
    int rows, hw;
    bool vec;
};

template <int G, int kR, int THREADS>
struct OutLn {
    static constexpr int C = G * kStatCols;
    static constexpr int kPass = THREADS / 16;  // rows per pass of the tile load
    static_assert(kR % 16 == 0 && kR <= THREADS && kR % kPass == 0, "tile rows");
    static constexpr size_t kTileBytes = (size_t)kStatCols * (kR + 1) * sizeof(float);
    static constexpr size_t kSmem = kTileBytes + (size_t)kR * sizeof(float2);

    __device__ __forceinline__ static void block(const OutLnArgs &a, int bx, int by, unsigned char *smem) {
        float(*tile)[kR + 1] = reinterpret_cast<float(*)[kR + 1]>(smem);
        float2 *norm = reinterpret_cast<float2 *>(smem + kTileBytes);
        const int tid = threadIdx.x;
        const int row0 = bx * kR, c0 = by * kStatCols;
        // The x tile and the statistics are loaded together, then combined.
        constexpr int kPer = kR / kPass;  // rows per thread: tid / 16, + kPass, ...
        const int q = 4 * (tid & 15), r0 = tid >> 4;
        float4 v[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int row = row0 + r0 + kPass * i;
            v[i] = row < a.rows ? *reinterpret_cast<const float4 *>(a.x + (size_t)row * C + c0 + q)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (tid < kR) {
            const int row = row0 + tid;
            float2 p[G];
#pragma unroll
            for (int k = 0; k < G; ++k)
                p[k] = row < a.rows ? a.stats[(size_t)row * G + k] : make_float2(0.0f, 0.0f);
            const RowLn<G> l = ln_combine<G>(p);
            norm[tid] = make_float2(l.mean, l.r);
        }
        const float4 gv = *reinterpret_cast<const float4 *>(a.g + c0 + q);
        const float4 bv = *reinterpret_cast<const float4 *>(a.b + c0 + q);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int r = r0 + kPass * i;
            const float2 m = norm[r];
            tile[q + 0][r] = (v[i].x - m.x) * m.y * gv.x + bv.x;
            tile[q + 1][r] = (v[i].y - m.x) * m.y * gv.y + bv.y;
            tile[q + 2][r] = (v[i].z - m.x) * m.y * gv.z + bv.z;
            tile[q + 3][r] = (v[i].w - m.x) * m.y * gv.w + bv.w;
        }
        __syncthreads();
        if (a.vec) {
            constexpr int kQ = kR / 4;
            for (int e = tid; e < kStatCols * kQ; e += THREADS) {
                const int c = e / kQ, r = 4 * (e - c * kQ), row = row0 + r;
                if (row >= a.rows) continue;
                const int n = row / a.hw, p = row - n * a.hw;
                *reinterpret_cast<float4 *>(a.out + ((size_t)n * C + c0 + c) * a.hw + p) =
                    make_float4(tile[c][r], tile[c][r + 1], tile[c][r + 2], tile[c][r + 3]);
            }
        } else {
            for (int e = tid; e < kStatCols * kR; e += THREADS) {
                const int c = e / kR, r = e - c * kR, row = row0 + r;
                if (row >= a.rows) continue;
                const int n = row / a.hw, p = row - n * a.hw;
                a.out[((size_t)n * C + c0 + c) * a.hw + p] = tile[c][r];
            }
        }
    }
};

template <int G, int kR>
__global__ __launch_bounds__(256) void out_ln_kernel(OutLnArgs a) {
    using LN = OutLn<G, kR, 256>;
    __shared__ __attribute__((aligned(16))) unsigned char smem[LN::kSmem];
    LN::block(a, (int)blockIdx.x, (int)blockIdx.y, smem);
}

// ------------------------------------------------------- window attention
// Window token t of window (n, wy, wx) reads padded, cyclically shifted source
// ((wy*7 + t/7 + shift) mod Hp, (wx*7 + t%7 + shift) mod Wp) (reference
// gather_windows_kernel cuda_swin.cu:120-131, cyclic_source swin.c:106-110).
// Returns the token row, -1 for a zero-padded source (q/k/v = qkv bias), -2
// for the MFMA padding rows t >= 49.  shift < 7 <= Hp, Wp, so one conditional
// subtraction is the modulo.
__device__ __forceinline__ int window_token(int t, int n, int wy, int wx, int H, int W, int Hp,
                                            int Wp, int shift) {
    if (t >= 49) return -2;
    const int ty = t / 7;
    int sy = wy * 7 + ty + shift, sx = wx * 7 + (t - 7 * ty) + shift;
    sy -= sy >= Hp ? Hp : 0;
    sx -= sx >= Wp ? Wp : 0;
    return (sy < H && sx < W) ? (n * H + sy) * W + sx : -1;
}

// Shifted-window region label 3*ry + rx of padded position (py, px)
// (reference mask_region, swin.c:112-117; cuda_swin.cu:132-134).
__host__ __device__ __forceinline__ int window_label(int t, int wy, int wx, int Hp, int Wp,
                                                     int shift) {
    const int py = wy * 7 + t / 7, px = wx * 7 + t % 7;
    const int ry = py < Hp - 7 ? 0 : (py < Hp - shift ? 1 : 2);
    const int rx = px < Wp - 7 ? 0 : (px < Wp - shift ? 1 : 2);
    return 3 * ry + rx;
}

// Index-map probe: the window_token / window_label values of every window
// token, as the attention kernel computes them.
static __global__ __launch_bounds__(256) void window_map_kernel(int *token, int *label, int batches,
                                                              int H, int W, int wy_n, int wx_n,
                                                              int shift) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= batches * wy_n * wx_n * 49) return;
    const int t = idx % 49, win = idx / 49;
    const int wx = win % wx_n, t1 = win / wx_n, wy = t1 % wy_n, n = t1 / wy_n;
    token[idx] = window_token(t, n, wy, wx, H, W, wy_n * 7, wx_n * 7, shift);
    label[idx] = window_label(t, wy, wx, wy_n * 7, wx_n * 7, shift);
}

// The region labels of a window depend only on whether it is in the last
// window row and/or column: type = 2*(wy == wy_n-1) + (wx == wx_n-1).  An
// unshifted block has a single type (no mask).
__host__ __device__ __forceinline__ int window_type(int wy, int wx, int wy_n, int wx_n, int shift) {
    return shift ? 2 * (wy == wy_n - 1) + (wx == wx_n - 1) : 0;
}
__host__ __device__ constexpr int window_types(int shift) { return shift ? 4 : 1; }

// Additive score term of the attention kernel, in the order its accumulators
// hold scores, pre-multiplied by log2(e) (softmax runs on exp2):
//   lane l, value v = 16*jb + 4*ib + e  ->  query i = 16*ib + (l & 15),
//                                           key   j = 16*jb + 4*(l >> 4) + e
//   term = rel_bias[h][i][j] - 100 * (label(i) != label(j))  for i, j < 49,
//          0 for padded queries (i >= 49), -inf for padded keys (j >= 49).
// Stored per (type, head) as 8 chunks of [64 lanes][8] fp16, so chunk c is one
// coalesced 16-byte load per lane.  A representative window of each type
// supplies the labels (bias_mat is [heads][49][49] fp32).
static __global__ __launch_bounds__(64) void attn_term_kernel(const float *__restrict__ bias_mat,
                                                              bf16 *__restrict__ term, int heads,
                                                              int wy_n, int wx_n, int shift) {
    const int lane = threadIdx.x, c = blockIdx.x & 7, th = blockIdx.x >> 3;
    const int h = th % heads, type = th / heads;
    const int wy = (type & 2) ? wy_n - 1 : 0, wx = (type & 1) ? wx_n - 1 : 0;
    const int Hp = wy_n * 7, Wp = wx_n * 7;
    constexpr float kLog2e = 1.4426950408889634f;
    bf16x8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int v = 8 * c + k, jb = v >> 4, ib = (v >> 2) & 3, e = v & 3;
        const int i = 16 * ib + (lane & 15), j = 16 * jb + 4 * (lane >> 4) + e;
        float t;
        if (j >= 49) {
            t = -INFINITY;
        } else if (i >= 49) {
            t = 0.0f;
        } else {
            t = bias_mat[((size_t)h * 49 + i) * 49 + j];
            if (shift && window_label(i, wy, wx, Hp, Wp, shift) != window_label(j, wy, wx, Hp, Wp, shift))
                t -= 100.0f;
            t *= kLog2e;
        }
        o[k] = to_half(t);
    }
    *reinterpret_cast<bf16x8 *>(term + ((size_t)(th * 8 + c) * 64 + lane) * 8) = o;
}

constexpr size_t attn_term_elems(int heads, int shift) {
    return (size_t)window_types(shift) * heads * 8 * 64 * 8;
}

// Independent (window, head) waves per workgroup: two spread the waves over
// the CUs more evenly than four (stage 2: 1512 waves) and measured 4.9 us per
// frame faster on MI355X; one was 1 us slower than four.
constexpr int kAttnWaves = 2;
constexpr int kAttnVS = 72;  // LDS row stride of V^T (16-bit words)

// Scores, softmax and O = P V of one (window, head) whose Q and K fragments
// are in registers (lane l: slot 16b + (l&15), the 8 k-slots of lane group
// l>>4, any channel order both operands share), whose V^T sits in this wave's
// LDS slice Vt[channel * kAttnVS + slot] (written by this wave), and whose score
// terms are in add[]; stores the output row of every real slot (tok >= 0).
__device__ __forceinline__ void attend_store(const bf16x8 (&qf)[4], const bf16x8 (&kf)[4],
                                             const bf16x8 (&add)[8], const bf16 *Vt,
                                             const int (&tok)[4], bf16 *out,
                                             int C, int h, int lane) {
    constexpr int VS = kAttnVS;
    const int l16 = lane & 15, g = lane >> 4;
    // S^T[j][i] blocks: s[jb][ib][e] = S[i = 16ib + l16][j = 16jb + 4g + e].
    f32x4 s[4][4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) s[jb][ib] = mfma16_f16(kf[jb], qf[ib], f32x4{0, 0, 0, 0});

    // Softmax in base 2: scores and terms carry log2(e).
    const float scale = 0.17677669529663687f * 1.4426950408889634f;  // log2(e) / sqrt(32)
    float inv[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
        float m = -INFINITY;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 16 * jb + 4 * ib + e;
                const float x = fmaf(s[jb][ib][e], scale, half_to_f32(add[v >> 3][v & 7]));
                s[jb][ib][e] = x;
                m = fmaxf(m, x);
            }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        float sum = 0.0f;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = __builtin_amdgcn_exp2f(s[jb][ib][e] - m);  // -inf -> 0
                s[jb][ib][e] = p;
                sum += p;
            }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        inv[ib] = 1.0f / sum;
    }

    // V^T was written by this wave only; LDS accesses of one wave complete in
    // order, so a compiler-level fence is all the reads below need.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // O^T = V^T P^T over two 32-key chunks; k-slot e of lane group g is key
    // 32c + 16*(e>>2) + 4g + (e&3) in both operands.
    f32x4 o[2][4];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) o[db][ib] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        bf16x8 pf[4], vf[2];
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
#pragma unroll
            for (int e = 0; e < 8; ++e) pf[ib][e] = to_half(s[2 * c + (e >> 2)][ib][e & 3]);
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const bf16 *r = Vt + (16 * db + l16) * VS + 32 * c + 4 * g;
            const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(r);
            const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(r + 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vf[db][e] = lo[e];
                vf[db][4 + e] = hi[e];
            }
        }
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) o[db][ib] = mfma16_f16(vf[db], pf[ib], o[db][ib]);
    }
    // o[db][ib][e] = O[i = 16ib + l16][d = 16db + 4g + e] (unnormalised).
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
        if (tok[ib] < 0) continue;
        bf16 *dst = out + (size_t)tok[ib] * C + h * 32 + 4 * g;
#pragma unroll
        for (int db = 0; db < 2; ++db)
            store4(dst + 16 * db, o[db][ib][0] * inv[ib], o[db][ib][1] * inv[ib],
                   o[db][ib][2] * inv[ib], o[db][ib][3] * inv[ib]);
    }
}

// One wave64 per (window, head) with head dim 32.  Window slot r = 16b + (l&15)
// (b = 0..3, 49 tokens padded to 64) is lane l's row in every operand: the
// S^T = K Q^T MFMAs take K and Q fragments (8 channels 8*(l>>4).. of that row)
// straight from global memory, V goes through LDS once to become V^T, and the
// output row of slot r is stored by the same lane.  The fp32 softmax over keys
// runs on the accumulator registers (the 64 keys of a query sit in 16
// registers x 4 lanes), and O^T = V^T P^T takes P straight from those
// registers as the B operand (the key order of the k-slots is a permutation
// shared by both operands).  Scores are q.k/sqrt(32) + rel_bias[h][i][j]
// (- 100 across shifted regions), the latter read as one precomputed fp16 term
// per accumulator (attn_term_kernel); keys t >= 49 get -inf.  Each wave works
// on its own LDS slice, so waves never synchronise.
static __global__ __launch_bounds__(256) void window_attention_kernel(
    const bf16 *__restrict__ qkv, const float *__restrict__ qkv_bias,
    const bf16 *__restrict__ term, bf16 *__restrict__ out, int H, int W, int C, int heads,
    int wy_n, int wx_n, int shift, int items) {
    constexpr int VS = kAttnVS;
    __shared__ __attribute__((aligned(16))) bf16 sV[kAttnWaves][32 * VS];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int item = blockIdx.x * kAttnWaves + wave;
    if (item >= items) return;  // no workgroup barrier follows
    const int h = item % heads, win = item / heads;
    const int wx = win % wx_n, t1 = win / wx_n, wy = t1 % wy_n, n = t1 / wy_n;
    const int Hp = wy_n * 7, Wp = wx_n * 7;
    const size_t ld = 3 * (size_t)C;
    const int l16 = lane & 15, g = lane >> 4;

    // This window type's score terms: 8 coalesced 16-byte loads per lane.
    const bf16 *tp = term + ((size_t)(window_type(wy, wx, wy_n, wx_n, shift) * heads + h) * 512 + lane) * 8;
    bf16x8 add[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) add[c] = *reinterpret_cast<const bf16x8 *>(tp + c * 512);

    // Every slot's q / k / v and the bias row are loaded unconditionally (a
    // slot without a token reads token row 0), so all of them are in flight
    // together; the selects below pick the token row, the qkv bias for a
    // zero-padded source, or zeros for the MFMA padding rows.
    int tok[4];
    bf16x8 qr[4], kr[4], vr[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        tok[b] = window_token(16 * b + l16, n, wy, wx, H, W, Hp, Wp, shift);
        const bf16 *src = qkv + (size_t)(tok[b] < 0 ? 0 : tok[b]) * ld + h * 32 + 8 * g;
        qr[b] = *reinterpret_cast<const bf16x8 *>(src);
        kr[b] = *reinterpret_cast<const bf16x8 *>(src + C);
        vr[b] = *reinterpret_cast<const bf16x8 *>(src + 2 * C);
    }
    bf16x8 qb, kb, vb;
    {
        const float *bq = qkv_bias + h * 32 + 8 * g;
        float fq[8], fk[8], fv[8];
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            *reinterpret_cast<float4 *>(fq + e) = *reinterpret_cast<const float4 *>(bq + e);
            *reinterpret_cast<float4 *>(fk + e) = *reinterpret_cast<const float4 *>(bq + C + e);
            *reinterpret_cast<float4 *>(fv + e) = *reinterpret_cast<const float4 *>(bq + 2 * C + e);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qb[e] = to_half(fq[e]);
            kb[e] = to_half(fk[e]);
            vb[e] = to_half(fv[e]);
        }
    }
    bf16x8 qf[4], kf[4];
    bf16 *Vt = sV[wave];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const bf16x8 zero = {};
        const bool real = tok[b] >= 0, pad = tok[b] == -1;
        qf[b] = real ? qr[b] : pad ? qb : zero;
        kf[b] = real ? kr[b] : pad ? kb : zero;
        const bf16x8 v = real ? vr[b] : pad ? vb : zero;
#pragma unroll
        for (int e = 0; e < 8; ++e) Vt[(8 * g + e) * VS + 16 * b + l16] = v[e];
    }

    attend_store(qf, kf, add, Vt, tok, out, C, h, lane);
}

// Fused window MSA for the small-channel stages: QKV projection + attention in
// one workgroup per window, one wave per head (C = 32 * heads).  The window's
// 64 slots of LayerNorm-1 output (zero rows for padded and t >= 49 slots) are
// gathered into LDS once; each wave projects its head's q, k and v with the
// weights read from L2, then runs the same scores / softmax / AV tail as
// window_attention_kernel.  The projection is computed transposed,
// Y^T[32 ch][64 slots] = W_h X^T, so that a lane holds one slot (16b + (l&15))
// and channels {4g + i, 16 + 4g + i} (g = l>>4, i < 4): eight channels per
// slot, in one k-slot order that Q and K share, which is all the S = Q K^T
// MFMAs need; V^T goes to LDS as before.  Every projected value is the fp32
// MFMA sum over the input channels in ascending 32-wide steps plus the bias,
// rounded once to fp16 (the separate QKV GEMM's computation), so a zero
// (padded) row yields the bias, as in the unfused path.  The q, k, v rows
// never reach HBM.
template <int C>
__global__ __launch_bounds__(64 * (C / 32)) __attribute__((amdgpu_waves_per_eu(C == 96 ? 3 : 2))) void window_msa_kernel(
    const bf16 *xn, const bf16 *__restrict__ wqkv, const float *__restrict__ bqkv,
    const bf16 *__restrict__ term, bf16 *out, int H, int W, int wy_n, int wx_n, int shift) {
    // xn and out may be the same buffer: a window's rows are all read (into
    // LDS, before the barrier) by the workgroup that later writes them, and
    // windows own disjoint token rows, so neither pointer is __restrict__.
    constexpr int HEADS = C / 32, KS = C / 32, XS = C + 8;  // XS: LDS row stride (words)
    constexpr int VS = kAttnVS;
    __shared__ __attribute__((aligned(16))) bf16 sX[64 * XS];
    __shared__ __attribute__((aligned(16))) bf16 sV[HEADS][32 * VS];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = wave;
    const int win = blockIdx.x;
    const int wx = win % wx_n, t1 = win / wx_n, wy = t1 % wy_n, n = t1 / wy_n;
    const int Hp = wy_n * 7, Wp = wx_n * 7;
    const int l16 = lane & 15, g = lane >> 4;

    // The window's rows, 16 bytes per thread and step: all four steps' loads
    // are issued before any is stored (a slot without a token reads row 0
    // and stores zeros), so their latencies overlap.
    constexpr int kSteps = 64 * (C / 8) / (64 * HEADS);
    static_assert(kSteps * 64 * HEADS == 64 * (C / 8), "whole steps");
    bf16x8 xv[kSteps];
    int xt[kSteps];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
        const int c = threadIdx.x + i * 64 * HEADS, r = c / (C / 8), q = c - r * (C / 8);
        xt[i] = window_token(r, n, wy, wx, H, W, Hp, Wp, shift);
        xv[i] = *reinterpret_cast<const bf16x8 *>(xn + (size_t)(xt[i] < 0 ? 0 : xt[i]) * C + 8 * q);
    }
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
        const int c = threadIdx.x + i * 64 * HEADS, r = c / (C / 8), q = c - r * (C / 8);
        const bf16x8 zero = {};
        *reinterpret_cast<bf16x8 *>(sX + r * XS + 8 * q) = xt[i] >= 0 ? xv[i] : zero;
    }

    int tok[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) tok[b] = window_token(16 * b + l16, n, wy, wx, H, W, Hp, Wp, shift);
    __syncthreads();

    // Y^T for matrix m (0 q, 1 k, 2 v) of head h: acc[cb][b] holds channels
    // 16cb + 4g + i of slot 16b + l16.
    auto project = [&](int m, f32x4 (&acc)[2][4]) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[cb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        // All of this matrix's weight fragments are read before the first
        // MFMA, so the L2 reads overlap.
        bf16x8 wa[KS][2];
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                wa[s][cb] = *reinterpret_cast<const bf16x8 *>(
                    wqkv + (size_t)(m * C + h * 32 + 16 * cb + l16) * C + 32 * s + 8 * g);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            bf16x8 xb[4];
#pragma unroll
            for (int b = 0; b < 4; ++b)
                xb[b] = *reinterpret_cast<const bf16x8 *>(sX + (16 * b + l16) * XS + 32 * s + 8 * g);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[cb][b] = mfma16_f16(wa[s][cb], xb[b], acc[cb][b]);
        }
    };
    // fp16 words of Y^T + bias in k-slot order: e < 4 -> channel 4g + e,
    // e >= 4 -> channel 16 + 4g + (e - 4).
    auto words = [&](int m, const f32x4 (&acc)[2][4], bf16x8 (&f)[4]) {
        const float *bm = bqkv + m * C + h * 32 + 4 * g;
        const float4 b0 = *reinterpret_cast<const float4 *>(bm);
        const float4 b1 = *reinterpret_cast<const float4 *>(bm + 16);
        const float bias[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 8; ++e) f[b][e] = to_half(acc[e >> 2][b][e & 3] + bias[e]);
    };

    f32x4 acc[2][4];
    bf16x8 qf[4], kf[4], vf[4];
    project(0, acc);
    words(0, acc, qf);
    project(1, acc);
    words(1, acc, kf);
    project(2, acc);
    words(2, acc, vf);
    bf16 *Vt = sV[wave];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int ch = (e < 4 ? 0 : 16) + 4 * g + (e & 3);
            Vt[ch * VS + 16 * b + l16] = vf[b][e];
        }
    // Score terms of this window type and head, loaded only now so that their
    // 32 registers are not held through the projections (three waves per
    // SIMD need the kernel under 168 VGPRs).
    const bf16 *tp = term + ((size_t)(window_type(wy, wx, wy_n, wx_n, shift) * HEADS + h) * 512 + lane) * 8;
    bf16x8 add[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) add[c] = *reinterpret_cast<const bf16x8 *>(tp + c * 512);
    attend_store(qf, kf, add, Vt, tok, out, C, h, lane);
}


}  // namespace bfhip
