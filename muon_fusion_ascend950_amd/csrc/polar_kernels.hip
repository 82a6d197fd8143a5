// polar_kernels.hip — the three gfx950 kernels of one Polar Express step.
//
//   stage 1 "gram"  : A = X·Xᵀ          upper-triangle tiles only, mirrored store
//   stage 2 "poly"  : P = b·A + c·A·A    upper-triangle tiles only, mirrored store,
//                                        polynomial fused into the register epilogue
//   stage 3 "apply" : Y = a·X + P·X      a·X fused into the register epilogue
//
// Reference counterparts (behaviour, not structure):
//   stage 1  csrc/muon_polar_unified_ascend950.asc:38-517   (MuonGramLowLevelFused)
//   stage 2  csrc/muon_polar_unified_ascend950.asc:520-1035 (MuonCube2PFused)
//   stage 3  csrc/muon_polar_unified_ascend950.asc:1038-1540 (MuonCube3FusedLowLevel)
//
// One templated kernel serves the three stages.  A workgroup owns one BM x BN
// output tile of one batch matrix; 4 waves in a 2x2 layout each own a
// (BM/2) x (BN/2) sub-tile of 32x32 MFMA blocks.  The K loop stages 64-deep
// panels of both operands through LDS with a register prefetch of the next panel.
//
// Scratch layout: A and P are [batch][mp][mp] bf16 with mp the larger of the
// stage-1/2 tile extents; rows/columns >= m are computed from zero-filled X rows
// (or written as zeros past a stage's tile grid) and are therefore exact zeros, so
// stages 2 and 3 need no K masking on A or P.
#include "polar_kernels.h"
#include "polar_schedule.hpp"
#include "polar_tile.hpp"
#include "polar_epilogue.hpp"

namespace muon_polar {

namespace {

template <int BM, int BN, Stage S, bool VEC>
__global__ __launch_bounds__(256) void polar_gemm_kernel(GemmArgs g) {
    constexpr int NT = 256;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int SM = WM / 32, SN = WN / 32;
    static_assert(SM >= 1 && SN >= 1, "tile too small");
    static_assert(S == Stage::Apply || BM == BN, "triangular stages need square tiles");
    // X-side accesses use VEC; A and P (library scratch) are always 16-byte aligned.
    constexpr bool kRowVec = (S != Stage::Gram) || VEC;
    constexpr bool kColVec = (S == Stage::Poly) || VEC;

    __shared__ __attribute__((aligned(16))) uint16_t lds_row[BM * kBK];
    __shared__ __attribute__((aligned(16))) uint16_t lds_col[BN * kBK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave & 1, wc = wave >> 1;

    const int bt = blockIdx.x / g.tiles_per_batch;
    const int t = blockIdx.x - bt * g.tiles_per_batch;
    int tm, tn;
    if constexpr (S == Stage::Apply) {
        tm = t % g.tiles_m;
        tn = t / g.tiles_m;
    } else {
        upper_tile_of(t, g.tiles_m, tm, tn);
    }
    const int row0 = tm * BM, col0 = tn * BN;

    const uint16_t *rowop = g.rowop + bt * g.sb_row;
    const uint16_t *colop = g.colop + bt * g.sb_col;

    KContigTile<BM, NT, kRowVec> ta;
    using ColTile = typename std::conditional<S == Stage::Apply, NContigTile<BN, NT, kColVec>,
                                              KContigTile<BN, NT, kColVec>>::type;
    ColTile tb;

    auto load_stage = [&](int k0) {
        ta.load(rowop, g.ld_row, row0, g.row_rows, k0, g.row_k, tid);
        if constexpr (S == Stage::Apply)
            tb.load(colop, g.ld_col, k0, g.col_k, col0, g.col_rows, tid);
        else
            tb.load(colop, g.ld_col, col0, g.col_rows, k0, g.col_k, tid);
    };

    f32x16 acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int nk = g.k_loop / kBK;
    load_stage(0);
    ta.store(lds_row, tid);
    tb.store(lds_col, tid);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) load_stage((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            bf16x8 fr[SM], fc[SN];
#pragma unroll
            for (int i = 0; i < SM; ++i)
                fr[i] = frag_kc(lds_row, wr * WM + i * 32 + (lane & 31), kk, lane);
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                if constexpr (S == Stage::Apply)
                    fc[j] = frag_nc_tr<BN>(lds_col, wc * WN + j * 32 + ((lane >> 4) & 1) * 16, kk,
                                           lane);
                else
                    fc[j] = frag_kc(lds_col, wc * WN + j * 32 + (lane & 31), kk, lane);
            }
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j) acc[i][j] = mfma_32x32x16(fc[j], fr[i], acc[i][j]);
        }
        __syncthreads();
        if (kt + 1 < nk) {
            ta.store(lds_row, tid);
            tb.store(lds_col, tid);
            __syncthreads();
        }
    }

    // ---------------------------------------------------------------- epilogue
    store_tile<BM, BN, S, VEC>(acc, g, bt, row0, col0, tm == tn, lane, wr, wc);
    if constexpr (S != Stage::Apply) zero_past_grid<BM>(g, g.out + bt * g.sb_out, tm, tn, tid, NT);
}

template <int BM, int BN, Stage S, bool VEC>
hipError_t launch_one(const GemmArgs &g, int grid, hipStream_t stream) {
    GemmArgs copy = g;
    void *args[] = {&copy};
    return hipLaunchKernel(reinterpret_cast<const void *>(&polar_gemm_kernel<BM, BN, S, VEC>),
                           dim3(grid), dim3(256), args, 0, stream);
}

template <Stage S, bool VEC>
hipError_t launch_by_tile(int bm, int bn, const GemmArgs &g, int grid, hipStream_t stream) {
    if (bm == 64 && bn == 64) return launch_one<64, 64, S, VEC>(g, grid, stream);
    if (bm == 128 && bn == 128) return launch_one<128, 128, S, VEC>(g, grid, stream);
    if (bm == 256 && bn == 256) return launch_one<256, 256, S, VEC>(g, grid, stream);
    if constexpr (S != Stage::Apply) {
        if (bm == 192 && bn == 192) return launch_one<192, 192, S, VEC>(g, grid, stream);
    }
    if constexpr (S == Stage::Apply) {
        if (bm == 128 && bn == 256) return launch_one<128, 256, S, VEC>(g, grid, stream);
        if (bm == 256 && bn == 128) return launch_one<256, 128, S, VEC>(g, grid, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool tile_supported(Stage s, int bm, int bn) {
    if (bm == bn && (bm == 64 || bm == 128 || bm == 256)) return true;
    if (s != Stage::Apply && bm == 192 && bn == 192) return true;
    if (s == Stage::Apply && ((bm == 128 && bn == 256) || (bm == 256 && bn == 128))) return true;
    return false;
}

hipError_t launch_gemm(Stage s, int bm, int bn, bool vec, const GemmArgs &g, int grid,
                       hipStream_t stream) {
    switch (s) {
        case Stage::Gram:
            return vec ? launch_by_tile<Stage::Gram, true>(bm, bn, g, grid, stream)
                       : launch_by_tile<Stage::Gram, false>(bm, bn, g, grid, stream);
        case Stage::Poly:
            return launch_by_tile<Stage::Poly, true>(bm, bn, g, grid, stream);
        case Stage::Apply:
            return vec ? launch_by_tile<Stage::Apply, true>(bm, bn, g, grid, stream)
                       : launch_by_tile<Stage::Apply, false>(bm, bn, g, grid, stream);
        case Stage::GramT:
        case Stage::ApplyR:
            // right-Gram stages exist only as DMA-fed kernels (the host never
            // routes them here)
            return hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

}  // namespace muon_polar
