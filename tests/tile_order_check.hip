// Host-side check of the workgroup -> tile maps of hip_common.h: for every
// grid up to 48 x 48 tiles and every XCD row-group count, xcd_swizzle and
// xcd_block_tile must be permutations of [0, tiles), and xcd_block_tile must
// give each XCD its own rectangle of rows and columns wherever the grid
// divides evenly.  Prints "ok" and exits 0, or names the first failure.
#include "hip_common.h"

#include <cstdio>
#include <vector>

int main() {
    using bfhip::xcd_block_tile;
    using bfhip::xcd_swizzle;
    for (int tm = 1; tm <= 48; ++tm)
        for (int tn = 1; tn <= 48; ++tn) {
            const int count = tm * tn;
            std::vector<int> seen(count, 0);
            for (int b = 0; b < count; ++b) {
                const int t = xcd_swizzle(b, count);
                if (t < 0 || t >= count || seen[t]++) {
                    std::printf("xcd_swizzle %dx%d: bid %d -> %d\n", tm, tn, b, t);
                    return 1;
                }
            }
            for (int gm = 1; gm <= 8; gm *= 2) {
                std::vector<int> hit(count, 0);
                std::vector<int> xcd_of(count, -1);
                for (int b = 0; b < count; ++b) {
                    const int t = xcd_block_tile(b, tm, tn, gm);
                    if (t < 0 || t >= count || hit[t]++) {
                        std::printf("xcd_block_tile %dx%d gm %d: bid %d -> %d\n", tm, tn, gm, b, t);
                        return 1;
                    }
                    xcd_of[t] = b % 8;
                }
                // Even grids: tile (r, c) sits on XCD (r / (tm/gm)) * gn + c / (tn/gn).
                const int gn = 8 / gm;
                if (count >= 16 && tm % gm == 0 && tn % gn == 0)
                    for (int t = 0; t < count; ++t) {
                        const int r = t / tn, c = t % tn;
                        const int want = (r / (tm / gm)) * gn + c / (tn / gn);
                        if (xcd_of[t] != want) {
                            std::printf("xcd_block_tile %dx%d gm %d: tile %d on XCD %d, want %d\n",
                                        tm, tn, gm, t, xcd_of[t], want);
                            return 1;
                        }
                    }
            }
        }
    std::printf("ok\n");
    return 0;
}
