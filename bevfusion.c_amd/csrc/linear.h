// fp16 x fp16 linear layers for the Swin context: Y = X W^T (+ epilogue),
// X [M, K] fp16 row-major, W [N, K] fp16 (the PyTorch [out, in] layout), fp32
// accumulation on the fp16 MFMA.
//
// Operands stream into LDS through buffer_load ... lds (DmaRowsBf16).  The
// tile per layer comes from a sweep of this core over the Swin-T layer shapes
// at 6 x 256 x 704 on MI355X (all 19 (N, K) pairs: qkv, proj, fc1, fc2 per
// stage and the three patch merges).  The grids are small (1-6 rounds of
// 64 x 64 tiles on 256 CUs), so more workgroups in flight mostly beat larger
// per-wave tiles: 64 x 64 is the default, K = 96 layers run three 32-deep
// steps and the N = 768, K >= 768 reductions one more stage of 128.  Where a
// wider tile measured faster it is listed by (N, K): 128 x 64 for stage-1
// qkv / fc2 and the first merge (M = 16896), 64 x 128 for stage-2 qkv and
// stage-3 fc1; stage-1 fc1 (1584 tiles of 64 x 128) as 32-deep k-steps in
// three stages, whose 36 KiB of LDS let four workgroups share a CU (1.55
// rounds instead of 2.06 at three: 18.9 vs 19.7 us).  (N, K)
// identifies the layer, so the table holds for any camera count; other shapes
// take the 64-deep default.
//
// Four layers measured faster on the wave-specialised pipeline
// (gemm_spec_kernel: loader waves issue every DMA, so the compute waves'
// MFMAs never wait behind a stalled DMA issue), each with four loader waves
// (one wave's 63 in-flight DMA instructions cap its workgroup's fetch):
// stage-2 fc1 (128 x 128 x 64, eight compute waves, two stages: 12.7 vs 14.0
// us as 128 x 128 on the plain core), stage-2 fc2 (64 x 64 x 64, four stages:
// 11.5 vs 11.9 us with one loader wave), stage-3 fc2 (64 x 64 x 128, three
// stages: 12.8 vs 14.2 us with one loader wave, 16.3 us plain) and stage-3
// proj (64 x 64 x 128, three stages: 5.6 vs 6.4 us as 32 x 64 with one).
//
// Stage-3 fc1 (M = 1056 tokens at six cameras, W 3072 x 768) deals its tiles
// to the XCDs as 2 row groups x 4 column groups (XcdBlocks): each XCD's L2
// then fetches a quarter of W instead of all of it (plain fp16 stores: 11.7
// -> 10.3 us; with its epilogue 13.4 -> 11.9 us alone, 0.5 us per frame in
// the frame).  The same order measured no faster, or slower by up to 1 us,
// for the other stage-3 linears and the stage-2 -> 3 merge: their repeated
// weight reads are served by the memory-side cache, and the per-CU fetch
// rate, not the HBM, bounds them.
#pragma once

#include <cstdint>

#include "gemm_core.h"

namespace bfhip {

template <class T, class Epi>
inline void linear_tile(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    DmaRowsBf16<T::BM, T::BK, T::kThreads> al{x, K, M, K};
    DmaRowsBf16<T::BN, T::BK, T::kThreads> bl{w, K, N, K};
    launch_gemm_dma<T>(al, bl, epi, M, N, K, s);
}

template <class T, int LW = 1, class Epi>
inline void linear_spec(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    DmaRowsBf16<T::BM, T::BK, LW * kWave> al{x, K, M, K};
    DmaRowsBf16<T::BN, T::BK, LW * kWave> bl{w, K, N, K};
    launch_gemm_spec<T>(al, bl, epi, M, N, K, s);
}

enum LinearTile { kK32, kK64, kK128, kTall, kWide, kWideXcd2, kWide32, kSpecBig, kSpec64, kSpec128 };

inline LinearTile pick_linear_tile(int N, int K) {
    struct Entry { int n, k; LinearTile t; };
    static const Entry table[] = {
        {768, 3072, kSpec128}, {384, 1536, kSpec64}, {768, 768, kSpec128}, {768, 1536, kK128},
        {576, 192, kTall}, {192, 768, kTall},  {192, 384, kTall},
        {768, 192, kWide32}, {1152, 384, kWide}, {3072, 768, kWideXcd2},
        {1536, 384, kSpecBig},
    };
    for (const Entry &e : table)
        if (e.n == N && e.k == K) return e.t;
    return K <= 96 ? kK32 : kK64;
}

// Buffer-resource offsets are 32-bit: both operands must span < 2 GiB, rows
// start 16-byte aligned and K is a multiple of 8 (true of every layer here;
// checked by the callers' contexts at create).
inline bool linear_operands_ok(const void *x, const void *w, int M, int N, int K) {
    return K % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
           (uint64_t)M * K * 2 < (1ull << 31) && (uint64_t)N * K * 2 < (1ull << 31);
}

template <class Epi>
inline void linear_f16(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    switch (pick_linear_tile(N, K)) {
        case kK32: linear_tile<DmaTile<64, 64, 32, 2, 2, 2, true>>(x, w, M, N, K, epi, s); break;
        case kK64: linear_tile<DmaTile<64, 64, 64, 2, 2, 2, true>>(x, w, M, N, K, epi, s); break;
        case kK128: linear_tile<DmaTile<64, 64, 128, 2, 2, 3, true>>(x, w, M, N, K, epi, s); break;
        case kTall: linear_tile<DmaTile<128, 64, 64, 2, 2, 2, true>>(x, w, M, N, K, epi, s); break;
        case kWide: linear_tile<DmaTile<64, 128, 64, 2, 2, 2, true>>(x, w, M, N, K, epi, s); break;
        case kWideXcd2:
            linear_tile<XcdBlocks<DmaTile<64, 128, 64, 2, 2, 2, true>, 2>>(x, w, M, N, K, epi, s);
            break;
        case kWide32: linear_tile<DmaTile<64, 128, 32, 2, 2, 3, true>>(x, w, M, N, K, epi, s); break;
        case kSpecBig: linear_spec<DmaTile<128, 128, 64, 2, 4, 2, true>, 4>(x, w, M, N, K, epi, s); break;
        case kSpec64: linear_spec<DmaTile<64, 64, 64, 2, 2, 4, true>, 4>(x, w, M, N, K, epi, s); break;
        case kSpec128: linear_spec<DmaTile<64, 64, 128, 2, 2, 3, true>, 4>(x, w, M, N, K, epi, s); break;
    }
}

}  // namespace bfhip
