// polar_schedule.hpp — work assignment of the DMA-fed stage kernels: which
// output tile and which K-steps a workgroup computes, and where a stream-K
// contributor keeps its fp32 partial.
//
// Host and device share these functions: the kernels call them to pick their
// work, and the host-side plan check (polar_capi.cpp, muon_polar_plan_extents)
// walks every workgroup of a launch with the same code to bound the memory each
// one stores to.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "polar_kernels.h"

namespace muon_polar {

// Output tile (tm, tn) of linear tile index t within one batch matrix for the
// triangular stages: row-major walk over the upper tiles tn >= tm of an nt x nt grid.
__host__ __device__ __forceinline__ void upper_tile_of(int t, int nt, int &tm, int &tn) {
    int row = 0, len = nt;
    while (t >= len) {
        t -= len;
        ++row;
        --len;
    }
    tm = row;
    tn = row + t;
}

// The same tiles walked in B x B super-blocks: super-blocks (I, J >= I) row-major,
// the tiles of each row-major inside it (tn >= tm in a diagonal one).  A run of
// consecutive tiles then covers a compact block of the triangle, whose row and
// column panels (blocks of X rows for gram, of A rows for poly) are few and shared
// in one XCD's L2.  B <= 1: the row-major walk.
__host__ __device__ __forceinline__ void upper_tile_blocked(int t, int nt, int b, int &tm,
                                                            int &tn) {
    if (b <= 1) {
        upper_tile_of(t, nt, tm, tn);
        return;
    }
    const int ns = (nt + b - 1) / b;
    tm = tn = 0;
    for (int bi = 0; bi < ns; ++bi) {
        const int rows = b < nt - bi * b ? b : nt - bi * b;
        const int diag = rows * (rows + 1) / 2;
        if (t < diag) {
            int r, c;
            upper_tile_of(t, rows, r, c);
            tm = bi * b + r;
            tn = bi * b + c;
            return;
        }
        t -= diag;
        for (int bj = bi + 1; bj < ns; ++bj) {
            const int cols = b < nt - bj * b ? b : nt - bj * b;
            if (t < rows * cols) {
                tm = bi * b + t / cols;
                tn = bj * b + t % cols;
                return;
            }
            t -= rows * cols;
        }
    }
}

// The off-diagonal tiles (tn > tm) in the order of upper_tile_blocked with the
// diagonal tiles left out.
__host__ __device__ __forceinline__ void strict_upper_tile_blocked(int t, int nt, int b, int &tm,
                                                                   int &tn) {
    if (b <= 1) b = nt;  // row by row: one super-block
    const int ns = (nt + b - 1) / b;
    tm = tn = 0;
    for (int bi = 0; bi < ns; ++bi) {
        const int rows = b < nt - bi * b ? b : nt - bi * b;
        const int above = rows * (rows - 1) / 2;
        if (t < above) {
            int r = 0, len = rows - 1;
            while (t >= len) {
                t -= len;
                ++r;
                --len;
            }
            tm = bi * b + r;
            tn = bi * b + r + 1 + t;
            return;
        }
        t -= above;
        for (int bj = bi + 1; bj < ns; ++bj) {
            const int cols = b < nt - bj * b ? b : nt - bj * b;
            if (t < rows * cols) {
                tm = bi * b + t / cols;
                tn = bj * b + t % cols;
                return;
            }
            t -= rows * cols;
        }
    }
}

// Units of one batch matrix of a triangular stage (g.diag_pairs: off-diagonal
// tiles, then diagonal pairs; else its upper tiles).
__host__ __device__ __forceinline__ int sym_units(int nt, bool diag_pairs) {
    return diag_pairs ? nt * (nt - 1) / 2 + (nt + 1) / 2 : nt * (nt + 1) / 2;
}

// Whether unit t of a batch matrix is a pair of diagonal tiles (2p, 2p) and
// (2p + 1, 2p + 1); tile_coords gives it (tm, tn) = (2p, 2p + 1), the tile whose
// row and column panels are the two tiles' panels.
__host__ __device__ __forceinline__ bool is_diag_pair(const GemmArgs &g, int t) {
    if (!g.diag_pairs) return false;
    const int off = g.tiles_m * (g.tiles_m - 1) / 2;
    return t >= off && 2 * (t - off) + 1 < g.tiles_m;
}

// Tile (tm, tn) of linear tile t of one batch matrix.  Triangular stages: the
// super-block walk above (with g.diag_pairs, the unit order above: a diagonal
// pair gives (2p, 2p + 1), a last diagonal tile alone (2p, 2p)).  Others: runs
// of group_n column tiles walked row by row, so the tiles an XCD holds at once
// share few row- and column-operand panels.
__host__ __device__ __forceinline__ void tile_coords(const GemmArgs &g, bool symmetric, int t,
                                                     int &tm, int &tn) {
    if (symmetric) {
        if (g.diag_pairs) {
            const int off = g.tiles_m * (g.tiles_m - 1) / 2;
            if (t < off) {
                strict_upper_tile_blocked(t, g.tiles_m, g.group_n, tm, tn);
            } else {
                tm = 2 * (t - off);
                tn = tm + 1 < g.tiles_m ? tm + 1 : tm;
            }
            return;
        }
        upper_tile_blocked(t, g.tiles_m, g.group_n, tm, tn);
        return;
    }
    const int gn = g.group_n;
    const int span = gn * g.tiles_m;
    const int grp = t / span, r = t - grp * span;
    const int width = gn < g.tiles_n - grp * gn ? gn : g.tiles_n - grp * gn;
    tm = r / width;
    tn = grp * gn + r % width;
}

// Stream-K bookkeeping (all values uniform across the workgroup).
// Range of unit u: iterations [sk_bound(u), sk_bound(u + 1)).
__host__ __device__ __forceinline__ int64_t sk_bound(const GemmArgs &g, int u) {
    return int64_t(u) * g.sk_iters / g.sk_units;
}
// Unit whose range holds iteration i: the largest u with sk_bound(u) <= i.
__host__ __device__ __forceinline__ int sk_unit_of(const GemmArgs &g, int64_t i) {
    const int64_t u = ((i + 1) * g.sk_units - 1) / g.sk_iters;
    return u < g.sk_units ? static_cast<int>(u) : g.sk_units - 1;
}
// Partial slot of unit u for stream-K tile st (tiles counted from dp_tiles).
// Units cover contiguous iteration ranges in order, so for units u < u' every
// tile of u is <= every tile of u': u + st is distinct for every (unit, tile)
// pair that exists, and the slots number sk_units + (stream-K tiles) - 1.
__host__ __device__ __forceinline__ int sk_slot(int u, int st) { return u + st; }

// Number of partial slots a launch of the split can touch.
inline int64_t sk_slots(int64_t sk_units, int64_t sk_tiles) {
    return sk_units > 0 ? sk_units + sk_tiles - 1 : 0;
}

// Work of workgroup w: iterations [it_lo, it_hi) of tiles tile_base + i / k_steps,
// and its stream-K unit (-1 for a whole tile).  Workgroup w runs on XCD w % 8;
// each XCD gets a contiguous run of whole tiles (workgroups [0, 8 * per_xcd),
// dispatched first, so full rounds start together and tiles that share operand
// panels stay in step) and of stream-K units (the rest, which fill the last
// round as CUs free up).  Returns false when the workgroup has no work.
__host__ __device__ __forceinline__ bool workgroup_range(const GemmArgs &g, int w, int &unit,
                                                         int &tile_base, int64_t &it_lo,
                                                         int64_t &it_hi) {
    const int dp_grid = 8 * g.per_xcd;
    if (w >= dp_grid) {
        const int ws = w - dp_grid;
        unit = (ws & 7) * (g.sk_units >> 3) + (ws >> 3);
        tile_base = g.dp_tiles;
        it_lo = sk_bound(g, unit);
        it_hi = sk_bound(g, unit + 1);
        return true;
    }
    unit = -1;
    tile_base = (w & 7) * g.per_xcd + (w >> 3);
    it_lo = 0;
    it_hi = g.k_steps;
    return tile_base < g.dp_tiles;
}

}  // namespace muon_polar
