// polar_kernels.h — host-visible interface of the gfx950 stage kernels
// (internal to the library; the public C ABI is include/muon_polar.h).
#pragma once

#include <hip/hip_runtime_api.h>
#include <cstddef>
#include <cstdint>

namespace muon_polar {

// The three stages of a step on X [m, n] with m <= n (A = X·Xᵀ, P = b·A + c·A·A,
// Y = a·X + P·X), and the right-Gram forms for m > n: G = Xᵀ·X (GramT) and
// Y = a·X + X·P (ApplyR), which need no transposed copy of X.
enum class Stage : int { Gram = 0, Poly = 1, Apply = 2, GramT = 3, ApplyR = 4 };

// Compile-time properties of a stage.
template <Stage S>
struct StageTraits {
    // upper-triangle tiles of a symmetric output, mirrored (square tiles)
    static constexpr bool kSymmetric = S == Stage::Gram || S == Stage::Poly || S == Stage::GramT;
    // operand panels stored [K][rows] (N-contiguous), read with transposing LDS reads
    static constexpr bool kRowNC = S == Stage::GramT;
    static constexpr bool kColNC = S == Stage::Apply || S == Stage::GramT;
    // the epilogue reads a tile of `epi` (A for poly, X for apply)
    static constexpr bool kEpiOperand = S == Stage::Poly || S == Stage::Apply || S == Stage::ApplyR;
    // epilogue arithmetic: gram (round), poly (b·A + c·acc) or apply (a·X + acc)
    static constexpr Stage kEpilogue =
        S == Stage::GramT ? Stage::Gram : (S == Stage::ApplyR ? Stage::Apply : S);
};

// Kernel arguments, passed by value (no device-side tiling buffer).
// Element offsets inside one batch matrix are 32-bit (the host rejects matrices
// of 2^31 elements or more); batch offsets are 64-bit.
struct GemmArgs {
    const uint16_t *rowop;  // K-contiguous operand whose rows index output rows
    const uint16_t *colop;  // gram/poly: K-contiguous, rows index output cols;
                            // apply: [K][cols] N-contiguous (X)
    const uint16_t *epi;    // epilogue input: A (poly) or X (apply); unused by gram
    uint16_t *out;
    int64_t sb_row, sb_col, sb_epi, sb_out;  // batch strides in elements
    int32_t ld_row, ld_col, ld_epi, ld_out;  // leading dimensions in elements
    int32_t row_rows, row_k;                 // extents of rowop present in memory
    int32_t col_rows, col_k;                 // gram/poly: rows x K of colop; apply: cols x K
    int32_t k_loop;                          // K extent iterated (multiple of 64)
    int32_t out_rows, out_cols;              // store extent (apply only)
    int32_t out_vec;  // 1: out rows take 16-byte stores; 2 (rows of an even number of
                      // elements from a 4-byte aligned out): 16-byte stores at 4-byte aligned
                      // addresses for chunks inside the row, 2-byte stores for the chunk
                      // that ends it; 3 (an odd number of elements, 4-byte aligned out): as
                      // 2 on the rows that start on a 4-byte boundary (even element offset),
                      // 2-byte stores on the others; 0: 2-byte stores
    int32_t out_cpol;                       // DMA-fed kernels' output stores: 0 plain, 1 nt,
                                             // 2 sc1, 3 nt sc1, 4 sc0 sc1
    int32_t tiles_m, tiles_n, tiles_per_batch;
    float s_epi, s_acc;  // poly: b, c;  apply: a, 1
    // streaming kernels only
    int32_t total_tiles, per_xcd;   // batch * tiles_per_batch; ceil(dp_tiles / 8)
    uint32_t bytes_row, bytes_col;  // byte extent of one batch matrix of rowop / colop
    uint32_t bytes_epi;             // byte extent of one batch matrix of epi
    int32_t group_n;                // apply: column tiles per raster group; gram and
                                    // poly: super-block side of the tile walk
    // Stream-K split of the streaming kernels.  Tiles [0, dp_tiles) run one per
    // workgroup (the first 8 * per_xcd workgroups); tiles [dp_tiles, total_tiles)
    // form sk_iters = (total_tiles - dp_tiles) * k_steps (tile, K-step)
    // iterations cut into sk_units equal contiguous ranges, one per workgroup
    // after those.  A tile cut between ranges is summed from fp32 partials by the
    // last contributor to arrive.
    int32_t k_steps;                // k_loop / 64
    int32_t dp_tiles;               // == total_tiles when stream-K is off
    int32_t sk_units;               // 0 or a multiple of 8
    int64_t sk_iters;
    float *partials;                // sk_units + (total_tiles - dp_tiles) - 1 slots of
                                    // BM * BN floats (sk_slot, polar_schedule.hpp)
    // One arrival word per stream-K tile: (token << 32) | count.  A word holding
    // another launch's token counts as zero, so the words need no clearing; the
    // last contributor leaves (token << 32) | 0, which a replay of the same
    // launch (a captured graph keeps its token) reads as zero too.
    uint64_t *counters;
    uint32_t token;                 // this launch's token
    // Apply stages (DMA-fed, 256x256 tiles with 8 waves): 2 or 3 = the tiles past
    // dp_tiles run as two 256x128 column halves each, one per workgroup after the
    // whole tiles, with that many ring slots, sk_units = the number of halves (no
    // partials, no arrival words); 0 = the stream-K split above.
    int32_t halves;
    // Triangular stages (DMA-fed, 64x64 tiles with 4 waves, no stream-K split):
    // 1 = the tiles_per_batch units of a batch matrix are its tiles_m (tiles_m - 1)
    // / 2 off-diagonal tiles (the super-block walk without the diagonal), then
    // (tiles_m + 1) / 2 diagonal units, unit p holding the diagonal tiles 2p and
    // 2p + 1 (2p alone when it is the last), so that fewer workgroups run the
    // same tiles (diagonal tiles read one panel each; a pair reads the two panels
    // an off-diagonal tile reads).  0 = every upper tile a unit of its own.
    int32_t diag_pairs;
};

bool tile_supported(Stage s, int bm, int bn);

// Register-staged kernels: any shape and alignment (element-masked edges).
hipError_t launch_gemm(Stage s, int bm, int bn, bool vec, const GemmArgs &g, int grid,
                       hipStream_t stream);

// DMA-fed kernels: X rows of 16-byte chunks (n % 8 == 0, 16-byte aligned X) or of an
// even number of elements from a 4-byte aligned X.  Grid is g.sk_units + 8 * g.per_xcd;
// `waves` per workgroup as returned by stream_waves; `depth` LDS ring slots (one K-step
// each), a combination stream_depth_supported accepts.  k_mask (gram and apply-right):
// 1 = the K-contiguous operands' rows end inside the last K-step (X rows of n % 64 != 0
// elements read in place), so the K-masked variant loads that step's chunks past row_k /
// col_k as zeros; 2 (gram only) = as 1, rows of n % 8 != 0 elements: the chunk that
// straddles n also has its positions past n zeroed in LDS.
hipError_t launch_stream(Stage s, int bm, int bn, int waves, int depth, const GemmArgs &g,
                         hipStream_t stream, int k_mask = 0);

// Whether a DMA-fed kernel exists for (s, bm, bn, waves, depth).
bool stream_depth_supported(Stage s, int bm, int bn, int waves, int depth);

// Waves per workgroup the DMA-fed kernel of a bm x bn tile runs with, given the
// requested count (8 is available for 256x256, 192x192 (the wave pairs) and
// 128x128 tiles; 4 otherwise).
int stream_waves(int bm, int bn, int requested);

// Workgroups of the DMA-fed kernel for (s, bm, bn, waves, depth) resident per CU
// (0 on error).
int stream_blocks_per_cu(Stage s, int bm, int bn, int waves, int depth);


// Per-matrix normalisation y = x / (‖x‖_F·1.01 + 1e-6) of `batch` matrices of mn
// elements (reference recipe rounding points; polar_norm.hip).  `partial` holds
// batch * norm_chunks(batch, mn) floats; vec: mn % 8 == 0 and 16-byte aligned x and y.
// Elements per partial sum (a power of two from 4096 to 2^20) and partial sums per
// matrix for `batch` matrices of mn elements.
int64_t norm_chunk(int64_t batch, int64_t mn);
int64_t norm_chunks(int64_t batch, int64_t mn);
hipError_t launch_normalize(const uint16_t *x, uint16_t *y, float *partial, int64_t batch,
                            int64_t mn, bool vec, hipStream_t stream);
// The scale pass alone, from partial sums already in `partial`.
hipError_t launch_norm_scale(const uint16_t *x, uint16_t *y, const float *partial,
                             int64_t batch, int64_t mn, bool vec, hipStream_t stream);

// Muon update passes (polar_norm.hip).  Momentum: buf ← lerp(buf, g, w),
// g' = nesterov ? lerp(g, buf, beta) : buf, x0 = bf16(g'), and x0's per-chunk
// sums of squares into `partial` in launch_normalize's order (ready for
// launch_norm_scale).  vec: mn % 8 == 0 and 16-byte aligned g, buf, x0.
hipError_t launch_muon_momentum(const float *g, float *buf, uint16_t *x0, float *partial,
                                int64_t batch, int64_t mn, float w, float beta, bool nesterov,
                                bool vec, hipStream_t stream);
// Xp [rows, np] = X [rows, n] with zero columns n .. np-1 (np >= n, np % 8 == 0,
// 16-byte aligned xp).
hipError_t launch_pad_rows(const uint16_t *x, uint16_t *xp, int64_t rows, int64_t n, int64_t np,
                           hipStream_t stream);

// p ← p·decay + alpha·O over `total` elements; vec: total % 8 == 0, 16-byte aligned.
hipError_t launch_muon_param_update(float *p, const uint16_t *o, int64_t total, float decay,
                                    float alpha, bool vec, hipStream_t stream);

// Scratch of the allocation-free step (polar_noalloc.hip): a device array of
// kNoAllocScratchBytes per GPU.  noalloc_scratch returns its address on
// `device`, which must be the current device (looked up once per device).
constexpr size_t kNoAllocScratchBytes = size_t(192) << 20;
hipError_t noalloc_scratch(int device, void **ptr);

}  // namespace muon_polar
