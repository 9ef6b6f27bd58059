// Fused Swin MLP for the wide, shallow stages (C = 96, 192):
//   x += fc2(GELU(fc1(LN2(x))))          and optionally  xn = LN1'(x)
// in one launch, with the 4C-wide hidden layer never leaving the chip.
//
// Transposed formulation on v_mfma_f32_16x16x32_bf16 (A = weights, B = tokens):
//   fc1:  H^T[hid, tok] = W1[hid, c] . LN2(x)^T[c, tok]
//   fc2:  y^T[c, tok]   = W2[c, hid] . GELU(H^T + b1)[hid, tok]
// The fc1 accumulator of lane l holds hidden rows 4*(l>>4)+r of token l&15,
// which is exactly the k-slot set the fc2 B operand wants from that lane if the
// hidden index of k-slot e is 16*(e>>2) + 4*(l>>4) + (e&3): GELU(H) feeds fc2
// straight from registers.  W2's columns are packed in that order at create.
//
// Weights are packed per 32-wide hidden chunk in MFMA-fragment order: a 1 KiB
// fragment is the 64 lanes' 16-byte operands, lane-major, so one LDS-DMA
// instruction per fragment fills LDS and each fragment read is one
// conflict-free ds_read_b128.  Chunk q of the packed buffer holds
//   W1 fragments (f = 0,1; s = 0..C/32-1): lane l, element e ->
//       W1[32q + 16f + (l&15)][32s + 8(l>>4) + e]
//   W2 fragments (j = 0..C/16-1): lane l, element e ->
//       W2[16j + (l&15)][32q + 16(e>>2) + 4(l>>4) + (e&3)]
// Chunks stream through NBUF LDS buffers (one barrier per chunk) while every
// wave keeps its tokens' LN2 rows (the fc1 B operand) and fc2 accumulators in
// registers.  Each wave owns 16*TF tokens; LayerNorm statistics are fp32 over
// the 4 lanes that share a token (two-pass, eps 1e-5).
#pragma once

#include "gemm_core.h"

namespace bfhip {

template <int C_, int TF_, int WAVES_, int NBUF_>
struct MlpCfg {
    static constexpr int C = C_, TF = TF_, kWaves = WAVES_, kBufs = NBUF_;
    static constexpr int kHid = 4 * C;
    static constexpr int kChunks = kHid / 32;
    static constexpr int kKs = C / 32;          // fc1 k-steps
    static constexpr int kCf = C / 16;          // fc2 output-channel fragments
    static constexpr int kFrags = 2 * kKs + kCf;  // 1 KiB fragments per chunk
    static constexpr int kChunkBytes = kFrags * 1024;
    static constexpr int kTokens = kWaves * TF * 16;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kPerWave = kFrags / kWaves;  // DMA instructions per wave per chunk
    static_assert(C % 32 == 0, "channels must be a multiple of 32");
    static_assert(kFrags % kWaves == 0, "chunk fragments must split evenly over the waves");
    static_assert(kBufs >= 2 && kBufs <= kChunks, "2 .. kChunks chunk buffers");
};

// Host-side packing of W1 [4C][C] and W2 [C][4C] (fp32, PyTorch [out, in])
// into the chunked fragment order above, as bf16 bit patterns.
template <class Cfg, class ToBf16>
void pack_mlp_weights(const float *w1, const float *w2, uint16_t *dst, ToBf16 to_bf16_bits) {
    constexpr int C = Cfg::C, H = Cfg::kHid;
    size_t o = 0;
    for (int q = 0; q < Cfg::kChunks; ++q) {
        for (int f = 0; f < 2; ++f)
            for (int s = 0; s < Cfg::kKs; ++s)
                for (int l = 0; l < 64; ++l)
                    for (int e = 0; e < 8; ++e)
                        dst[o++] = to_bf16_bits(w1[(size_t)(32 * q + 16 * f + (l & 15)) * C + 32 * s + 8 * (l >> 4) + e]);
        for (int j = 0; j < Cfg::kCf; ++j)
            for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 8; ++e)
                    dst[o++] = to_bf16_bits(
                        w2[(size_t)(16 * j + (l & 15)) * H + 32 * q + 16 * (e >> 2) + 4 * (l >> 4) + (e & 3)]);
    }
}

template <class Cfg>
__global__ __launch_bounds__(Cfg::kThreads) void swin_mlp_kernel(
    float *__restrict__ x, const float *__restrict__ ln_g, const float *__restrict__ ln_b,
    const bf16 *__restrict__ wpk, const float *__restrict__ b1, const float *__restrict__ b2,
    const float *__restrict__ next_g, const float *__restrict__ next_b, bf16 *__restrict__ xn,
    int T) {
    constexpr int C = Cfg::C, TF = Cfg::TF, KS = Cfg::kKs, CF = Cfg::kCf;
    constexpr int NB = Cfg::kBufs, P = Cfg::kPerWave;
    __shared__ __attribute__((aligned(1024))) bf16 sw[NB][Cfg::kChunkBytes / 2];
    __shared__ float sb1[Cfg::kHid];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, l16 = lane & 15;
    const int tok0 = blockIdx.x * Cfg::kTokens + wave * TF * 16;

    const __amdgpu_buffer_rsrc_t rsrc =
        buffer_rsrc(wpk, (uint32_t)Cfg::kChunks * (uint32_t)Cfg::kChunkBytes);
    auto issue = [&](int q) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int frag = p * Cfg::kWaves + wave;
            dma16(rsrc, sw[q % NB] + frag * 512, (uint32_t)(q * Cfg::kChunkBytes + frag * 1024 + lane * 16));
        }
    };

    // LN2 of this wave's tokens into fc1 B operands: lane holds token
    // tok0 + 16i + l16, channels 32s + 8g + e.
    // x rows first, then the first NB-1 weight chunks, so that waiting for
    // x (in-order vmcnt) does not also wait for the weight stream.
    float4 xv[TF][KS][2];
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        const int t = tok0 + 16 * i + l16;
        const bool ok = t < T;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float *src = x + (size_t)(ok ? t : 0) * C + 32 * k + 8 * g;
            xv[i][k][0] = ok ? *reinterpret_cast<const float4 *>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[i][k][1] = ok ? *reinterpret_cast<const float4 *>(src + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float bias1[(Cfg::kHid + Cfg::kThreads - 1) / Cfg::kThreads];
#pragma unroll
    for (int r = 0; r < (Cfg::kHid + Cfg::kThreads - 1) / Cfg::kThreads; ++r) {
        const int i = threadIdx.x + r * Cfg::kThreads;
        bias1[r] = i < Cfg::kHid ? b1[i] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < NB - 1; ++q) issue(q);
#pragma unroll
    for (int r = 0; r < (Cfg::kHid + Cfg::kThreads - 1) / Cfg::kThreads; ++r) {
        const int i = threadIdx.x + r * Cfg::kThreads;
        if (i < Cfg::kHid) sb1[i] = bias1[r];
    }

    bf16x8 xf[TF][KS];
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        float v[KS][8];
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float4 a = xv[i][k][0], b = xv[i][k][1];
            v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
            v[k][4] = b.x; v[k][5] = b.y; v[k][6] = b.z; v[k][7] = b.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) s += v[k][e];
        }
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const float mean = s * (1.0f / C);
        float q = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) q += (v[k][e] - mean) * (v[k][e] - mean);
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        const float rstd = rsqrtf(q * (1.0f / C) + 1e-5f);
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int c = 32 * k + 8 * g;
            const float4 ga = *reinterpret_cast<const float4 *>(ln_g + c);
            const float4 gb = *reinterpret_cast<const float4 *>(ln_g + c + 4);
            const float4 ba = *reinterpret_cast<const float4 *>(ln_b + c);
            const float4 bb = *reinterpret_cast<const float4 *>(ln_b + c + 4);
            const float gg[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
            const float bbv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[i][k][e] = to_bf16((v[k][e] - mean) * rstd * gg[e] + bbv[e]);
        }
    }

    f32x4 acc[CF][TF];
#pragma unroll
    for (int j = 0; j < CF; ++j)
#pragma unroll
        for (int i = 0; i < TF; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int q = 0; q < Cfg::kChunks; ++q) {
        // Chunks issued after q: min(NB - 2, kChunks - 1 - q); wait for q only.
        DmaWait<NB - 2>::template stages<P>(min(NB - 2, Cfg::kChunks - 1 - q));
        // Every wave's part of chunk q landed, and buffer (q - 1) % NB is no
        // longer read by anyone.  (sb1 was written before the first barrier.)
        if (q == 0) __syncthreads(); else lds_barrier();
        if (q + NB - 1 < Cfg::kChunks) issue(q + NB - 1);
        const bf16 *wb = sw[q % NB] + lane * 8;

        // fc1 accumulators start at the bias of their hidden rows 32q + 16f + 4g + r.
        f32x4 h[2][TF];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const float4 bq = *reinterpret_cast<const float4 *>(sb1 + 32 * q + 16 * f + 4 * g);
#pragma unroll
            for (int i = 0; i < TF; ++i) h[f][i] = f32x4{bq.x, bq.y, bq.z, bq.w};
        }
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(wb + (f * KS + k) * 512);
#pragma unroll
                for (int i = 0; i < TF; ++i) h[f][i] = mfma16(a, xf[i][k], h[f][i]);
            }
        // GELU(H + b1) -> fc2 B operands (k-slot e = hidden 16(e>>2) + 4g + (e&3)).
        bf16x8 hb[TF];
#pragma unroll
        for (int i = 0; i < TF; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) hb[i][e] = to_bf16(gelu(h[e >> 2][i][e & 3]));
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(wb + (2 * KS + j) * 512);
#pragma unroll
            for (int i = 0; i < TF; ++i) acc[j][i] = mfma16(a, hb[i], acc[j][i]);
        }
    }

    // Residual: acc[j][i][e] is y[token tok0 + 16i + l16][channel 16j + 4g + e].
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        const int t = tok0 + 16 * i + l16;
        const bool ok = t < T;
        float *row = x + (size_t)(ok ? t : 0) * C + 4 * g;
        float4 y[CF];
#pragma unroll
        for (int j = 0; j < CF; ++j)
            y[j] = ok ? *reinterpret_cast<const float4 *>(row + 16 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float4 bj = *reinterpret_cast<const float4 *>(b2 + 16 * j + 4 * g);
            y[j].x += acc[j][i][0] + bj.x;
            y[j].y += acc[j][i][1] + bj.y;
            y[j].z += acc[j][i][2] + bj.z;
            y[j].w += acc[j][i][3] + bj.w;
            if (ok) *reinterpret_cast<float4 *>(row + 16 * j) = y[j];
            s += (y[j].x + y[j].y) + (y[j].z + y[j].w);
        }
        if (!xn) continue;  // uniform: the next LayerNorm is fused or not for the whole launch
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const float mean = s * (1.0f / C);
        float qs = 0.0f;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const float a = y[j].x - mean, b = y[j].y - mean, c = y[j].z - mean, d = y[j].w - mean;
            qs += (a * a + b * b) + (c * c + d * d);
        }
        qs += __shfl_xor(qs, 16);
        qs += __shfl_xor(qs, 32);
        const float rstd = rsqrtf(qs * (1.0f / C) + 1e-5f);
        if (!ok) continue;
#pragma unroll
        for (int j = 0; j < CF; ++j) {
            const int c = 16 * j + 4 * g;
            const float4 gg = *reinterpret_cast<const float4 *>(next_g + c);
            const float4 bb = *reinterpret_cast<const float4 *>(next_b + c);
            bf16x4 o;
            o[0] = to_bf16((y[j].x - mean) * rstd * gg.x + bb.x);
            o[1] = to_bf16((y[j].y - mean) * rstd * gg.y + bb.y);
            o[2] = to_bf16((y[j].z - mean) * rstd * gg.z + bb.z);
            o[3] = to_bf16((y[j].w - mean) * rstd * gg.w + bb.w);
            *reinterpret_cast<bf16x4 *>(xn + (size_t)t * C + c) = o;
        }
    }
}

template <class Cfg>
inline void launch_swin_mlp(float *x, const float *ln_g, const float *ln_b, const bf16 *wpk,
                            const float *b1, const float *b2, const float *next_g,
                            const float *next_b, bf16 *xn, int T, hipStream_t s) {
    hipLaunchKernelGGL((swin_mlp_kernel<Cfg>), dim3((T + Cfg::kTokens - 1) / Cfg::kTokens),
                       dim3(Cfg::kThreads), 0, s, x, ln_g, ln_b, wpk, b1, b2, next_g, next_b, xn, T);
}

}  // namespace bfhip
