// bf16 x bf16 linear layers for the Swin context: Y = X W^T (+ epilogue),
// X [M, K] bf16 row-major, W [N, K] bf16 (the PyTorch [out, in] layout).
//
// The tile shape per layer comes from a sweep of this GEMM core over the
// Swin-T layer shapes at 6 x 256 x 704 on MI355X (all 19 (N, K) pairs: qkv,
// proj, fc1, fc2 per stage and the three patch merges).  Small M favours
// 64 x 64 tiles (more workgroups in flight); K = 96 layers run the whole
// reduction in three 32-deep steps.  (N, K) identifies the layer, so the
// table holds for any camera count; other shapes take the 64 x 64 default.
#pragma once

#include "gemm_core.h"

namespace bfhip {

template <class T, class Epi>
inline void linear_tile(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    LoadRowsBf16<T::BM, T::BK, T::kThreads> al{x, K, M, K};
    LoadRowsBf16<T::BN, T::BK, T::kThreads> bl{w, K, N, K};
    launch_gemm<T>(al, bl, epi, M, N, K, s);
}

enum LinearTile { kT64x96k32, kT64x64k32, kT64x96k64, kT64x64k64, kT128x64k64, kT128x128w8, kT32x64k64 };

inline LinearTile pick_linear_tile(int N, int K) {
    struct Entry { int n, k; LinearTile t; };
    static const Entry table[] = {
        {288, 96, kT64x96k32},   {96, 96, kT64x96k32},    {384, 96, kT64x64k32},
        {96, 384, kT64x96k64},   {576, 192, kT64x64k64},  {192, 192, kT64x64k64},
        {768, 192, kT64x64k32},  {192, 768, kT128x64k64}, {1152, 384, kT64x64k64},
        {384, 384, kT64x64k64},  {1536, 384, kT128x128w8}, {384, 1536, kT64x64k64},
        {2304, 768, kT64x64k64}, {768, 768, kT32x64k64},  {3072, 768, kT128x64k64},
        {768, 3072, kT32x64k64}, {192, 384, kT128x64k64}, {384, 768, kT64x64k64},
        {768, 1536, kT32x64k64},
    };
    for (const Entry &e : table)
        if (e.n == N && e.k == K) return e.t;
    return K <= 96 ? kT64x64k32 : kT64x64k64;
}

template <class Epi>
inline void linear_bf16(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    switch (pick_linear_tile(N, K)) {
        case kT64x96k32: linear_tile<Tile<64, 96, 32, 2, 2>>(x, w, M, N, K, epi, s); break;
        case kT64x64k32: linear_tile<Tile<64, 64, 32, 2, 2>>(x, w, M, N, K, epi, s); break;
        case kT64x96k64: linear_tile<Tile<64, 96, 64, 2, 2>>(x, w, M, N, K, epi, s); break;
        case kT64x64k64: linear_tile<Tile<64, 64, 64, 2, 2>>(x, w, M, N, K, epi, s); break;
        case kT128x64k64: linear_tile<Tile<128, 64, 64, 2, 2>>(x, w, M, N, K, epi, s); break;
        case kT128x128w8: linear_tile<Tile<128, 128, 64, 4, 2>>(x, w, M, N, K, epi, s); break;
        case kT32x64k64: linear_tile<Tile<32, 64, 64, 2, 2>>(x, w, M, N, K, epi, s); break;
    }
}

}  // namespace bfhip
