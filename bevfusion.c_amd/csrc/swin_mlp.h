// Fused Swin block tail for the wide, shallow stage 0 (C = 96):
//   [x += proj(a) + b_proj]                      (PROJ: a = attention output)
//   x += fc2(GELU(fc1(LN2(x)) + b1)) + b2
//   xn = LN1'(x)                                  (optional: next block's LN1)
//   or xh = fp16(x - mean), stats = (mean, M2) of x (optional: for a
//                                                  consumer that folds its
//                                                  LayerNorm)
// in one launch: x is read and written once, the 4C-wide hidden layer never
// leaves the chip.
//
// Transposed formulation on v_mfma_f32_16x16x32_f16 (A = weights, B = tokens;
// fp16 words, fp32 accumulation).
// Every lane owns token (l & 15) of its 16-token fragment and, in the fp32
// accumulator ("C") layout, channels 16j + 4(l>>4) + e (j < C/16, e < 4): the
// residual row, the proj output, LN2, the fc2 output and LN1' all live in
// that layout, so x is loaded and stored as float4s and never shuffled.
//   proj:  y^T[c, tok]   = Wp[c, k] . a^T[k, tok]       (a rows as B operand)
//   fc1:   H^T[hid, tok] = W1[hid, c] . LN2(x)^T[c, tok]
//   fc2:   y^T[c, tok]   = W2[c, hid] . GELU(H^T + b1)[hid, tok]
// An operand that comes out of an accumulator is used in place: k-slot e of
// lane group g stands for index 16(e>>2) + 4g + (e&3) of the 32-wide k-step,
// so LN2(x) feeds fc1 and GELU(H) feeds fc2 straight from registers; W1 and
// W2 columns are packed in that order at create.
//
// Weights are packed in MFMA-fragment order: a 1 KiB fragment is the 64 lanes'
// 16-byte operands, lane-major, so one LDS-DMA instruction per fragment fills
// LDS and each fragment read is one conflict-free ds_read_b128.  Chunk q (32
// hidden units) of the packed MLP buffer holds
//   W1 fragments (f = 0,1; s < C/32): lane l, element e ->
//       W1[32q + 16f + (l&15)][32s + 16(e>>2) + 4(l>>4) + (e&3)]
//   W2 fragments (j < C/16): lane l, element e ->
//       W2[16j + (l&15)][32q + 16(e>>2) + 4(l>>4) + (e&3)]
// and the proj buffer holds fragments (j < C/16, s < C/32): lane l, element e
//   -> Wp[16j + (l&15)][32s + 8(l>>4) + e].
// Chunks stream through NBUF LDS buffers (one barrier per chunk); proj
// fragments are read once per wave straight from global memory (L1/L2).
// LayerNorm statistics are fp32 over the 4 lanes that share a token (two-pass,
// eps 1e-5).
#pragma once

#include "gemm_core.h"

#include <cstring>

namespace bfhip {

template <int C_, int TF_, int WAVES_, int NBUF_, bool PROJ_>
struct MlpCfg {
    static constexpr int C = C_, TF = TF_, kWaves = WAVES_, kBufs = NBUF_;
    static constexpr bool kProj = PROJ_;
    static constexpr int kHid = 4 * C;
    static constexpr int kChunks = kHid / 32;
    static constexpr int kKs = C / 32;            // k-steps over channels
    static constexpr int kCf = C / 16;            // output-channel fragments
    static constexpr int kFrags = 2 * kKs + kCf;  // 1 KiB weight fragments per chunk
    // A chunk is its weight fragments followed by the fc1 bias of its 32
    // hidden units (fp32, in accumulator order: [g][f][r] -> 32q+16f+4g+r).
    static constexpr int kBiasBytes = 32 * 4;
    static constexpr int kChunkBytes = kFrags * 1024 + kBiasBytes;
    static constexpr int kTokens = kWaves * TF * 16;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kPerWave = kFrags / kWaves + 1;  // DMA instructions per wave per chunk
    static constexpr int kBiasLanes = kBiasBytes / 16 / kWaves;  // bias DMA lanes per wave
    static_assert(C % 32 == 0, "channels must be a multiple of 32");
    static_assert(kFrags % kWaves == 0, "chunk fragments must split evenly over the waves");
    static_assert(kBiasLanes * 16 * kWaves == kBiasBytes, "bias block must split evenly over the waves");
    static_assert(kBufs >= 2 && kBufs <= kChunks, "2 .. kChunks chunk buffers");
};

// Hidden / channel index of k-slot e of lane group g within a 32-wide k-step.
constexpr int kslot(int g, int e) { return 16 * (e >> 2) + 4 * g + (e & 3); }

// Host-side packing of W1 [4C][C] and W2 [C][4C] (fp32, PyTorch [out, in])
// into the chunked fragment order above, as fp16 bit patterns, each chunk
// followed by its fp32 fc1 bias block (dst holds kChunks * kChunkBytes bytes).
template <class Cfg, class ToWord>
void pack_mlp_weights(const float *w1, const float *w2, const float *b1, uint16_t *dst,
                      ToWord to_word_bits) {
    constexpr int C = Cfg::C, H = Cfg::kHid;
    size_t o = 0;
    for (int q = 0; q < Cfg::kChunks; ++q) {
        for (int f = 0; f < 2; ++f)
            for (int s = 0; s < Cfg::kKs; ++s)
                for (int l = 0; l < 64; ++l)
                    for (int e = 0; e < 8; ++e)
                        dst[o++] = to_word_bits(w1[(size_t)(32 * q + 16 * f + (l & 15)) * C + 32 * s + kslot(l >> 4, e)]);
        for (int j = 0; j < Cfg::kCf; ++j)
            for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 8; ++e)
                    dst[o++] = to_word_bits(w2[(size_t)(16 * j + (l & 15)) * H + 32 * q + kslot(l >> 4, e)]);
        for (int g = 0; g < 4; ++g)
            for (int f = 0; f < 2; ++f)
                for (int r = 0; r < 4; ++r) {
                    const float b = b1[32 * q + 16 * f + 4 * g + r];
                    std::memcpy(dst + o, &b, 4);
                    o += 2;
                }
    }
}

// Host-side packing of the proj weight Wp [C][C] (fragment (j, s) order).
template <class Cfg, class ToWord>
void pack_proj_weights(const float *wp, uint16_t *dst, ToWord to_word_bits) {
    constexpr int C = Cfg::C;
    size_t o = 0;
    for (int j = 0; j < Cfg::kCf; ++j)
        for (int s = 0; s < Cfg::kKs; ++s)
            for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 8; ++e)
                    dst[o++] = to_word_bits(wp[(size_t)(16 * j + (l & 15)) * C + 32 * s + 8 * (l >> 4) + e]);
}

template <class Cfg>
__global__ __launch_bounds__(Cfg::kThreads) __attribute__((amdgpu_waves_per_eu(4))) void swin_mlp_kernel(
    float *__restrict__ x, const bf16 *attn, const bf16 *__restrict__ wproj,
    const float *__restrict__ bproj, const float *__restrict__ ln_g, const float *__restrict__ ln_b,
    const bf16 *__restrict__ wpk, const float *__restrict__ b1, const float *__restrict__ b2,
    const float *__restrict__ next_g, const float *__restrict__ next_b, bf16 *xn, int T,
    bf16 *xh, float2 *__restrict__ stats) {
    // attn may be the same buffer as xn (the next block's LN1 overwrites the
    // attention rows) or as xh (the stage's last block writes the fp16 copy
    // over them): each row is read (prologue) by the lane group that later
    // writes it (epilogue), so none of the three is __restrict__.
    constexpr int C = Cfg::C, TF = Cfg::TF, KS = Cfg::kKs, CF = Cfg::kCf;
    constexpr int NB = Cfg::kBufs, P = Cfg::kPerWave;
    // The chunk buffers are the kernel's only LDS object: a second __shared__
    // array makes the compiler attach alias scopes to LDS accesses and then
    // wait for every chunk DMA in flight before any chunk read, serialising
    // the weight stream with the MFMAs.  The fc1 bias therefore travels inside
    // each chunk.
    __shared__ __attribute__((aligned(1024))) bf16 sw[NB][Cfg::kChunkBytes / 2];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int tok0 = blockIdx.x * Cfg::kTokens + wave * TF * 16;

    const __amdgpu_buffer_rsrc_t rsrc =
        buffer_rsrc(wpk, (uint32_t)Cfg::kChunks * (uint32_t)Cfg::kChunkBytes);
    // Chunk q into buffer q % NB: P - 1 weight fragments per wave, then the
    // wave's share of the bias block (kBiasLanes lanes of 16 bytes).  Past the
    // last chunk the offsets are out of range, so the DMA only zero-fills that
    // (free) buffer; issuing it anyway keeps every iteration's vmcnt
    // arithmetic the same.
    auto issue = [&](int q) {
        const bool in = q < Cfg::kChunks;
#pragma unroll
        for (int p = 0; p < P - 1; ++p) {
            const int frag = p * Cfg::kWaves + wave;
            dma16(rsrc, sw[q % NB] + frag * 512,
                  in ? (uint32_t)(q * Cfg::kChunkBytes + frag * 1024 + lane * 16) : kDmaOutOfRange);
        }
        if (lane < Cfg::kBiasLanes) {
            const int at = Cfg::kFrags * 1024 + wave * Cfg::kBiasLanes * 16;
            dma16(rsrc, sw[q % NB] + at / 2,
                  in ? (uint32_t)(q * Cfg::kChunkBytes + at + lane * 16) : kDmaOutOfRange);
        }
    };

    // Global loads first (x rows in the C layout, attention rows, proj
    // fragments, b1), then the first NB-1 weight chunks, so that waiting for
    // the former (in-order vmcnt) never waits for the weight stream.
    float4 xr[TF][CF];
    bf16x8 af[TF][KS];
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        const int t = tok0 + 16 * i + l16;
        const bool ok = t < T;
        const size_t row = (size_t)(ok ? t : 0) * C;
#pragma unroll
        for (int j = 0; j < CF; ++j)
            xr[i][j] = ok ? *reinterpret_cast<const float4 *>(x + row + 16 * j + 4 * g)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (Cfg::kProj)
#pragma unroll
            for (int k = 0; k < KS; ++k)
                af[i][k] = ok ? *reinterpret_cast<const bf16x8 *>(attn + row + 32 * k + 8 * g) : bf16x8{};
    }
    if constexpr (Cfg::kProj) {
        // x += proj(a) + b_proj, accumulated in the C layout.
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float4 bp = *reinterpret_cast<const float4 *>(bproj + 16 * j + 4 * g);
            f32x4 pa[TF];
#pragma unroll
            for (int i = 0; i < TF; ++i) pa[i] = f32x4{bp.x, bp.y, bp.z, bp.w};
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const bf16x8 w = *reinterpret_cast<const bf16x8 *>(wproj + ((j * KS + k) * 64 + lane) * 8);
#pragma unroll
                for (int i = 0; i < TF; ++i) pa[i] = mfma16_f16(w, af[i][k], pa[i]);
            }
#pragma unroll
            for (int i = 0; i < TF; ++i) {
                xr[i][j].x += pa[i][0]; xr[i][j].y += pa[i][1];
                xr[i][j].z += pa[i][2]; xr[i][j].w += pa[i][3];
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NB - 1; ++q) issue(q);

    // LN2 in the C layout, then into fc1 B operands (k-slot order).
    bf16x8 xf[TF][KS];
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) s += (xr[i][j].x + xr[i][j].y) + (xr[i][j].z + xr[i][j].w);
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const float mean = s * (1.0f / C);
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float a = xr[i][j].x - mean, b = xr[i][j].y - mean, c = xr[i][j].z - mean,
                        d = xr[i][j].w - mean;
            q += (a * a + b * b) + (c * c + d * d);
        }
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        const float rstd = rsqrtf(q * (1.0f / C) + 1e-5f);
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float4 gg = *reinterpret_cast<const float4 *>(ln_g + 16 * j + 4 * g);
            const float4 bb = *reinterpret_cast<const float4 *>(ln_b + 16 * j + 4 * g);
            const int k = j >> 1, e0 = 4 * (j & 1);
            xf[i][k][e0 + 0] = to_half((xr[i][j].x - mean) * rstd * gg.x + bb.x);
            xf[i][k][e0 + 1] = to_half((xr[i][j].y - mean) * rstd * gg.y + bb.y);
            xf[i][k][e0 + 2] = to_half((xr[i][j].z - mean) * rstd * gg.z + bb.z);
            xf[i][k][e0 + 3] = to_half((xr[i][j].w - mean) * rstd * gg.w + bb.w);
        }
    }

    f32x4 acc[CF][TF];
#pragma unroll
    for (int j = 0; j < CF; ++j) {
        const float4 bj = *reinterpret_cast<const float4 *>(b2 + 16 * j + 4 * g);
#pragma unroll
        for (int i = 0; i < TF; ++i) acc[j][i] = f32x4{bj.x, bj.y, bj.z, bj.w};
    }

    // fc1 bias of hidden rows 32q + 16f + 4g + r, from chunk q's bias block.
    // Read before the next chunk's DMA is issued: the compiler makes this read
    // wait for every chunk DMA in flight.
    auto bias_of = [&](int q, float4 (&bq)[2]) {
#pragma unroll
        for (int f = 0; f < 2; ++f)
            bq[f] = __builtin_bit_cast(
                float4, *reinterpret_cast<const bf16x8 *>(sw[q % NB] + (Cfg::kFrags * 1024 + g * 32 + f * 16) / 2));
    };
    // fc1 of chunk q; the accumulators start at the bias (one VALU add per
    // hidden element saved).
    auto fc1_of = [&](int q, const float4 (&bq)[2], f32x4 (&h)[2][TF]) {
        const bf16 *wb = sw[q % NB] + lane * 8;
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int i = 0; i < TF; ++i) h[f][i] = f32x4{bq[f].x, bq[f].y, bq[f].z, bq[f].w};
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(wb + (f * KS + k) * 512);
#pragma unroll
                for (int i = 0; i < TF; ++i) h[f][i] = mfma16_f16(a, xf[i][k], h[f][i]);
            }
    };
    // GELU(H + b1) of chunk q -> fc2 B operands (k-slot order), then fc2.
    auto gelu_fc2 = [&](int q, const f32x4 (&h)[2][TF]) {
        const bf16 *wb = sw[q % NB] + lane * 8;
        bf16x8 hb[TF];
#pragma unroll
        for (int i = 0; i < TF; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) hb[i][e] = to_half(gelu(h[e >> 2][i][e & 3]));
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(wb + (2 * KS + j) * 512);
#pragma unroll
            for (int i = 0; i < TF; ++i) acc[j][i] = mfma16_f16(a, hb[i], acc[j][i]);
        }
    };

    // Software pipeline over the chunks: iteration q runs fc1 of chunk q + 1
    // before GELU and fc2 of chunk q, so the matrix cores have independent
    // work while the GELU runs.  Chunk q + NB - 1 is issued at iteration q
    // into the buffer of chunk q - 1, whose last reader (fc2, iteration
    // q - 1) every wave has passed at the iteration's barrier; chunk q + 1,
    // issued NB - 2 iterations earlier, must have landed by then.
    static_assert(NB >= 3, "fc1 runs one chunk ahead");
    DmaWait<NB - 2>::template stages<P>(NB - 2);  // chunk 0 (chunks 1 .. NB - 2 in flight)
    __syncthreads();
    f32x4 h[2][TF];
    {
        float4 bq[2];
        bias_of(0, bq);
        fc1_of(0, bq, h);
    }
    for (int q = 0; q < Cfg::kChunks; ++q) {
        const bool more = q + 1 < Cfg::kChunks;
        f32x4 hn[2][TF];
        if (more) {
            // Chunks 0 .. q + NB - 2 were issued: NB - 3 after chunk q + 1.
            DmaWait<NB - 3>::template stages<P>(NB - 3);
            lds_barrier();
            float4 bq[2];
            bias_of(q + 1, bq);
            issue(q + NB - 1);
            fc1_of(q + 1, bq, hn);
        }
        gelu_fc2(q, h);
        if (more) {
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int i = 0; i < TF; ++i) h[f][i] = hn[f][i];
        }
    }

    // Residual, then one of (uniform for the whole launch):
    //   xn = LN1'(x) of the next block, with x stored fp32;
    //   xh = fp16 words of x - mean and stats[t] = (mean, M2) over the row, for
    //   a consumer that folds the next LayerNorm (the patch merge), x not
    //   stored;
    //   x stored fp32 only.
    // acc[j][i][e] is channel 16j + 4g + e.
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        const int t = tok0 + 16 * i + l16;
        const bool ok = t < T;
        float *row = x + (size_t)(ok ? t : 0) * C + 4 * g;
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            xr[i][j].x += acc[j][i][0];
            xr[i][j].y += acc[j][i][1];
            xr[i][j].z += acc[j][i][2];
            xr[i][j].w += acc[j][i][3];
            if (ok && !xh) *reinterpret_cast<float4 *>(row + 16 * j) = xr[i][j];
            s += (xr[i][j].x + xr[i][j].y) + (xr[i][j].z + xr[i][j].w);
        }
        if (!xn && !xh) continue;
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const float mean = s * (1.0f / C);
        float qs = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float a = xr[i][j].x - mean, b = xr[i][j].y - mean, c = xr[i][j].z - mean,
                        d = xr[i][j].w - mean;
            qs += (a * a + b * b) + (c * c + d * d);
        }
        qs += __shfl_xor(qs, 16);
        qs += __shfl_xor(qs, 32);
        if (xh) {
            if (!ok) continue;
            if (g == 0) stats[t] = make_float2(mean, qs);
            // The copy is centred on the token mean (ln_fold.h).
#pragma unroll
            for (int j = 0; j < CF; ++j) {
                bf16x4 o;
                o[0] = to_half(xr[i][j].x - mean);
                o[1] = to_half(xr[i][j].y - mean);
                o[2] = to_half(xr[i][j].z - mean);
                o[3] = to_half(xr[i][j].w - mean);
                *reinterpret_cast<bf16x4 *>(xh + (size_t)t * C + 16 * j + 4 * g) = o;
            }
            continue;
        }
        const float rstd = rsqrtf(qs * (1.0f / C) + 1e-5f);
        if (!ok) continue;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const int c = 16 * j + 4 * g;
            const float4 gg = *reinterpret_cast<const float4 *>(next_g + c);
            const float4 bb = *reinterpret_cast<const float4 *>(next_b + c);
            bf16x4 o;
            o[0] = to_half((xr[i][j].x - mean) * rstd * gg.x + bb.x);
            o[1] = to_half((xr[i][j].y - mean) * rstd * gg.y + bb.y);
            o[2] = to_half((xr[i][j].z - mean) * rstd * gg.z + bb.z);
            o[3] = to_half((xr[i][j].w - mean) * rstd * gg.w + bb.w);
            *reinterpret_cast<bf16x4 *>(xn + (size_t)t * C + c) = o;
        }
    }
}

// xn (with next_g / next_b) or xh (with stats) selects the epilogue above;
// at most one of them is set.
template <class Cfg>
inline void launch_swin_mlp(float *x, const bf16 *attn, const bf16 *wproj, const float *bproj,
                            const float *ln_g, const float *ln_b, const bf16 *wpk,
                            const float *b1, const float *b2, const float *next_g,
                            const float *next_b, bf16 *xn, int T, hipStream_t s,
                            bf16 *xh = nullptr, float2 *stats = nullptr) {
    hipLaunchKernelGGL((swin_mlp_kernel<Cfg>), dim3((T + Cfg::kTokens - 1) / Cfg::kTokens),
                       dim3(Cfg::kThreads), 0, s, x, attn, wproj, bproj, ln_g, ln_b, wpk, b1, b2,
                       next_g, next_b, xn, T, xh, stats);
}

}  // namespace bfhip
