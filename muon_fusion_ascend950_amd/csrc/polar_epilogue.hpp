// polar_epilogue.hpp — register epilogues of the three stages (shared by the
// register-staged and the DMA-streamed kernels).
//
// Accumulator layout: acc[i][j] is the 32x32 MFMA block (i: output-row block,
// j: output-column block) of a wave sub-tile whose origin is (row0 + wr*BM/2,
// col0 + wc*BN/2).  Lane l owns output row (lane%32) of each row block and, for
// q = 0..3, the 4 consecutive columns 8q + 4*(lane/32) .. +3 (acc elements 4q..4q+3).
//
//   gram : A = bf16(acc)                                   + mirrored store
//   poly : P = bf16(b·A + c·acc)  (fp32, b·A first, then fma) + mirrored store
//   apply: Y = bf16(a·X + acc)    (one fp32 fma, one rounding)
//
// Reference epilogues: gram RNE cast .asc:407 and mirror .asc:414-468;
// poly .asc:929-973; apply .asc:1454-1492 (the reference rounds P·X and a·X to
// bf16 separately and adds in bf16; here a·X + P·X is rounded once).
#pragma once

#include "polar_kernels.h"
#include "polar_tile.hpp"

namespace muon_polar {

// bf16 pair helpers for the 8-byte (4 x bf16) epilogue vectors.
__device__ __forceinline__ void unpack4(u32x2 v, float (&f)[4]) {
    f[0] = bf16_bits_to_f32(v[0] & 0xffffu);
    f[1] = bf16_bits_to_f32(v[0] >> 16);
    f[2] = bf16_bits_to_f32(v[1] & 0xffffu);
    f[3] = bf16_bits_to_f32(v[1] >> 16);
}
__device__ __forceinline__ u32x2 pack4(const uint16_t (&h)[4]) {
    return u32x2{uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
}

// Epilogue values of one output row-block i: 4 consecutive columns per (j, q).
template <Stage S>
__device__ __forceinline__ void epilogue_values(const f32x16 &acc, int q, const float (&e)[4],
                                                const GemmArgs &g, uint16_t (&h)[4]) {
    constexpr Stage E = StageTraits<S>::kEpilogue;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float v = acc[4 * q + t];
        if constexpr (E == Stage::Apply)
            h[t] = f32_to_bf16_bits(fmaf(g.s_epi, e[t], v));  // a·X + P·X  (a·X + X·P)
        else if constexpr (E == Stage::Poly)
            h[t] = f32_to_bf16_bits(fmaf(g.s_acc, v, g.s_epi * e[t]));  // b·A + c·A²
        else
            h[t] = f32_to_bf16_bits(v);
    }
}

// Symmetric stages write A or P as [mp, mp] (row stride ld_out = mp) from a grid
// of tiles_n x tiles_n tiles of T rows; mp is the larger of the two symmetric
// stages' tile extents, so a stage with the smaller tile stops short of it.  The
// last column tile of each tile row then also writes zeros into its T rows past
// the grid and into the mirrored rows (the last tile row covers the corner), so
// the padding holds exact zeros whichever stage has the larger tile.
template <int T>
__device__ __forceinline__ void zero_past_grid(const GemmArgs &g, uint16_t *out, int tm, int tn,
                                               int tid, int nthreads) {
    const int ext = g.tiles_n * T;
    const int w = g.ld_out - ext;  // a multiple of 64
    if (w <= 0 || tn != g.tiles_n - 1) return;
    const int row0 = tm * T;
    const u32x4 z{0u, 0u, 0u, 0u};
    const int wch = w >> 3;  // 16-byte chunks per row of the strip
    for (int idx = tid; idx < T * wch; idx += nthreads) {
        const int r = idx / wch, c = idx - r * wch;
        *reinterpret_cast<u32x4 *>(out + (row0 + r) * g.ld_out + ext + 8 * c) = z;
    }
    const int cch = (tm == g.tiles_m - 1 ? T + w : T) >> 3;
    for (int idx = tid; idx < w * cch; idx += nthreads) {
        const int r = idx / cch, c = idx - r * cch;
        *reinterpret_cast<u32x4 *>(out + (ext + r) * g.ld_out + row0 + 8 * c) = z;
    }
}

template <int BM, int BN, Stage S, bool VEC>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[BM / 64][BN / 64], const GemmArgs &g,
                                           int bt, int row0, int col0, bool diag_tile, int lane,
                                           int wr, int wc) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int SM = WM / 32, SN = WN / 32;
    uint16_t *out = g.out + bt * g.sb_out;
    const uint16_t *epi = g.epi + bt * g.sb_epi;
    const bool diag = (S != Stage::Apply) && diag_tile;
    const int rbase = row0 + wr * WM + (lane & 31);          // + i*32
    const int cbase = col0 + wc * WN + 4 * (lane >> 5);      // + j*32 + 8q

    // ---- interior fast path: no masks; the epilogue operand of row-block i+1 is
    // loaded while row-block i is converted and stored.
    const bool interior = (S != Stage::Apply) ||
                          (VEC && row0 + BM <= g.out_rows && col0 + BN <= g.out_cols);
    if (interior && !diag) {
        constexpr bool kLoads = (S != Stage::Gram);
        u32x2 ev[2][SN][4];
        auto load_block = [&](int i, u32x2 (&dst)[SN][4]) {
            if constexpr (kLoads) {
                const uint16_t *er = epi + (rbase + i * 32) * g.ld_epi + cbase;
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        dst[j][q] = *reinterpret_cast<const u32x2 *>(er + j * 32 + 8 * q);
            }
        };
        load_block(0, ev[0]);
#pragma unroll
        for (int i = 0; i < SM; ++i) {
            if (i + 1 < SM) load_block(i + 1, ev[(i + 1) & 1]);
            const int r = rbase + i * 32;
            uint16_t *orow = out + r * g.ld_out + cbase;
#pragma unroll
            for (int j = 0; j < SN; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float e[4] = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (kLoads) unpack4(ev[i & 1][j][q], e);
                    uint16_t h[4];
                    epilogue_values<S>(acc[i][j], q, e, g, h);
                    *reinterpret_cast<u32x2 *>(orow + j * 32 + 8 * q) = pack4(h);
                    if constexpr (S != Stage::Apply) {
                        const int c = cbase + j * 32 + 8 * q;
#pragma unroll
                        for (int t = 0; t < 4; ++t) out[(c + t) * g.ld_out + r] = h[t];
                    }
                }
            }
        }
        return;
    }

    // ---- edge / diagonal path: per-element masks.
#pragma unroll
    for (int i = 0; i < SM; ++i) {
        const int r = rbase + i * 32;
#pragma unroll
        for (int j = 0; j < SN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = cbase + j * 32 + 8 * q;
                if constexpr (S == Stage::Apply) {
                    if (r < g.out_rows) {
                        const uint16_t *xr = epi + r * g.ld_epi + c;
                        uint16_t *yr = out + r * g.ld_out + c;
                        float e[4];
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            e[t] = (c + t < g.out_cols) ? bf16_bits_to_f32(xr[t]) : 0.0f;
                        uint16_t h[4];
                        epilogue_values<S>(acc[i][j], q, e, g, h);
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            if (c + t < g.out_cols) yr[t] = h[t];
                    }
                } else {
                    float e[4] = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (S == Stage::Poly)
                        unpack4(*reinterpret_cast<const u32x2 *>(epi + r * g.ld_epi + c), e);
                    uint16_t h[4];
                    epilogue_values<S>(acc[i][j], q, e, g, h);
                    uint16_t *orow = out + r * g.ld_out + c;
                    // Diagonal tile: the element with row <= col is the single source
                    // of both (r, c) and (c, r), so A and P are bitwise symmetric.
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (!diag || r <= c + t) {
                            orow[t] = h[t];
                            out[(c + t) * g.ld_out + r] = h[t];
                        }
                    }
                }
            }
        }
    }
}

}  // namespace muon_polar
