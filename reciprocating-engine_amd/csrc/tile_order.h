// tile_order.h - which output tile a workgroup of gemm_fp8_wide computes
// (csrc/gemm_fp8.hip). Plain C++ so that the host tests can check the
// mapping (tests/cpp/test_tile_order.cpp) with the same code the kernel runs.
//
// Workgroups are dealt to the 8 XCDs round-robin (workgroup b runs on XCD
// b % 8), and each XCD takes a contiguous run of the tiles: XCD x holds run
// [x per + min(x, rem), + per + (x < rem)) of tiles = 8 per + rem. Within a run
// the tiles go m fastest, or, with mapm > 0, as a block of mapm m-tiles by
// per / mapm n-tiles: the blocks of the 8 XCDs are laid out tiles_m / mapm
// along m and 8 / (tiles_m / mapm) along n. wide_mapm picks mapm.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define RENG_HD __host__ __device__
#else
#define RENG_HD
#endif

namespace reng {

constexpr uint32_t TILE_XCDS = 8;

// Tile (mt, nt) of workgroup b.
RENG_HD inline void wide_tile_of(uint32_t b, uint32_t tiles_m, uint32_t tiles, uint32_t mapm, uint32_t &mt,
                                 uint32_t &nt) {
    const uint32_t x = b % TILE_XCDS, l = b / TILE_XCDS;
    const uint32_t per = tiles / TILE_XCDS, rem = tiles % TILE_XCDS;
    const uint32_t tile = x * per + (x < rem ? x : rem) + l;
    mt = tile % tiles_m;
    nt = tile / tiles_m;
    if (mapm) {
        const uint32_t rgm = tiles_m / mapm, gn = per / mapm;
        mt = (x % rgm) * mapm + l % mapm;
        nt = (x / rgm) * gn + l / mapm;
    }
}

// The number of m-tiles per XCD block (0 keeps the m-fastest runs): the block
// that reads the fewest operand rows per XCD (mapm bm rows of a plus
// per / mapm bn rows of b), among blocks that tile the grid exactly (8 equal
// runs, mapm dividing the run and tiles_m, the XCD blocks 8 / (tiles_m / mapm)
// wide in n), and only if it reads fewer than the m-fastest run does.
inline uint32_t wide_mapm(uint32_t tiles_m, uint32_t tiles_n, uint32_t bm, uint32_t bn) {
    const uint32_t tiles = tiles_m * tiles_n;
    if (tiles % TILE_XCDS) return 0;
    const uint32_t per = tiles / TILE_XCDS;
    // The m-fastest run: the m-tiles it touches (at most tiles_m) and its n-columns (at most).
    const uint32_t cm = per < tiles_m ? per : tiles_m;
    const uint32_t cn = (per + tiles_m - 1) / tiles_m + (per % tiles_m ? 1 : 0);
    uint64_t best = (uint64_t)cm * bm + (uint64_t)cn * bn;
    uint32_t pick = 0;
    for (uint32_t m = 1; m <= tiles_m && m <= per; ++m) {
        if (tiles_m % m || per % m) continue;
        const uint32_t rgm = tiles_m / m;
        if (TILE_XCDS % rgm || (TILE_XCDS / rgm) * (per / m) != tiles_n) continue;
        const uint64_t c = (uint64_t)m * bm + (uint64_t)(per / m) * bn;
        if (c < best) best = c, pick = m;
    }
    return pick;
}

}  // namespace reng
