// bf16 x bf16 linear layers for the Swin context: Y = X W^T (+ epilogue),
// X [M, K] bf16 row-major, W [N, K] bf16 (the PyTorch [out, in] layout).
// Tile shape is picked per call from a small fixed set: 96-wide column
// tiles for the C = 96k widths of Swin-T, 128 otherwise; BK 32 for K = 96,
// 64 above; 64-row tiles when 128-row tiles would leave the chip under-filled.
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

template <class Epi>
inline void linear_bf16(const bf16 *x, const bf16 *w, int M, int N, int K, const Epi &epi,
                        hipStream_t s) {
    const bool n96 = N % 96 == 0 && N <= 576;
    const int bn = n96 ? 96 : 128;
    const long long tiles128 = ((M + 127LL) / 128) * ((N + bn - 1) / bn);
    const bool small_m = tiles128 < 512;
    if (K <= 96) {
        if (n96) linear_tile<Tile<128, 96, 32, 2, 2>>(x, w, M, N, K, epi, s);
        else linear_tile<Tile<128, 128, 32, 2, 2>>(x, w, M, N, K, epi, s);
    } else if (small_m) {
        if (n96) linear_tile<Tile<64, 96, 64, 2, 2>>(x, w, M, N, K, epi, s);
        else linear_tile<Tile<64, 128, 64, 2, 2>>(x, w, M, N, K, epi, s);
    } else {
        if (n96) linear_tile<Tile<128, 96, 64, 2, 2>>(x, w, M, N, K, epi, s);
        else linear_tile<Tile<128, 128, 64, 2, 2>>(x, w, M, N, K, epi, s);
    }
}

}  // namespace bfhip
