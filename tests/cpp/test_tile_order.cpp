// The fp8 wide GEMM's workgroup -> tile order (reciprocating-engine_amd/csrc/tile_order.h):
// on every grid up to 64 x 256 tiles and each tile size the launcher uses, the
// workgroups 0 .. tiles-1 reach every tile exactly once, with or without the
// 2-D XCD blocks wide_mapm picks; and the picks on the Qwen2.5-32B prefill shapes.
#include <cstdio>
#include <vector>

#include "../../reciprocating-engine_amd/csrc/tile_order.h"

using reng::wide_mapm;
using reng::wide_tile_of;

int main() {
    long grids = 0, blocks2d = 0, failed = 0;
    const uint32_t bms[] = {64, 128, 256}, bns[] = {64, 128, 160, 256};
    for (uint32_t tm = 1; tm <= 64; ++tm)
        for (uint32_t tn = 1; tn <= 256; ++tn)
            for (uint32_t bm : bms)
                for (uint32_t bn : bns) {
                    const uint32_t mapm = wide_mapm(tm, tn, bm, bn), tiles = tm * tn;
                    std::vector<unsigned char> seen(tiles, 0);
                    bool ok = true;
                    for (uint32_t b = 0; b < tiles && ok; ++b) {
                        uint32_t mt = 0, nt = 0;
                        wide_tile_of(b, tm, tiles, mapm, mt, nt);
                        if (mt >= tm || nt >= tn || seen[nt * tm + mt]++) ok = false;
                    }
                    if (!ok) {
                        std::printf("FAILED: %u x %u tiles of %u x %u, mapm %u\n", tm, tn, bm, bn, mapm);
                        ++failed;
                    }
                    ++grids;
                    blocks2d += mapm != 0;
                }
    // [M, N] / tile -> (tiles_m, tiles_n): kv 64 x 64, [5120, 5120] 128 x 160,
    // [27648, 5120] 256 x 256, [5120, 27648] 256 x 128.
    struct Case { uint32_t tm, tn, bm, bn, want; } cases[] = {
        {16, 16, 64, 64, 4}, {8, 32, 128, 160, 0}, {4, 108, 256, 256, 0}, {4, 40, 256, 128, 0}};
    for (const Case &c : cases) {
        const uint32_t got = wide_mapm(c.tm, c.tn, c.bm, c.bn);
        if (got != c.want) {
            std::printf("FAILED: wide_mapm(%u, %u, %u, %u) = %u, want %u\n", c.tm, c.tn, c.bm, c.bn, got, c.want);
            ++failed;
        }
    }
    std::printf("%ld grids, %ld with 2-D XCD blocks, %ld failed\n", grids, blocks2d, failed);
    return failed ? 1 : 0;
}
