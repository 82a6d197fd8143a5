// polar_stream.hip — DMA-fed variant of the three stage kernels.
//
// Same tiles, MFMA layout and arithmetic as the register-staged kernels in
// polar_kernels.hip; what changes is how data moves:
//
//   * global -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging, no
//     ds_write), 1 KiB per wave instruction, swizzle applied on the global side;
//   * an LDS ring of D K-step slots (2 for 256x256 tiles; up to 8 for the
//     latency-bound small tiles): panels k+1 .. k+D-1 stream in while step k is
//     multiplied; one barrier per K-step, placed so that the MFMA pipe keeps a
//     k16 slice of work queued across it, and the DMA instructions of the next
//     panel are interleaved one by one with that slice's MFMAs;
//   * MFMA operand fragments double-buffered in registers: the LDS reads of
//     slice s+1 are in flight while slice s is multiplied (with one MFMA per
//     slice, 64x64 tiles, a whole K-step's reads run one step ahead instead);
//   * stream-K: an under-full last round is cut into equal K ranges, one per
//     workgroup, and summed from fp32 partials by the last contributor;
//   * edge masking by out-of-range buffer offsets (the hardware returns zeros);
//   * an LDS-staged epilogue: the epilogue operand tile (X or A) is DMA'd into
//     the freed ring, each lane combines it with its accumulators in place, and
//     the tile leaves LDS as coalesced 16-byte row chunks (plus the mirrored tile
//     for the symmetric stages);
//   * XCD-aware tile order: workgroup w runs on XCD w % 8, so each XCD gets a
//     contiguous run of tiles that share operand panels in its L2 (apply: runs
//     of column tiles walked row by row; gram and poly: super-blocks of tiles).
//
// Used when X's rows can be read as 16-byte chunks: n % 8 == 0 with X 16-byte
// aligned, or an even n with X 4-byte aligned (the chunk that straddles a row's
// end is masked; see KT below); odd rows reach these kernels through a
// zero-padded copy, and the register-staged kernels cover calls without room
// for one.
#include "polar_epilogue.hpp"
#include "polar_kernels.h"
#include "polar_schedule.hpp"
#include "polar_tile.hpp"

#include <type_traits>

namespace muon_polar {

namespace {

// NW waves per workgroup in a 2 x NW/2 grid over the tile: 4 (one wave per
// SIMD, 128x128 wave tiles for a 256x256 tile) or 8 (two waves per SIMD, 128x64
// wave tiles: 1.5x the fragment reads, but one wave's LDS and barrier waits are
// covered by the other's MFMAs).  D = ring depth (LDS slots of one K-step each):
// panels k+1 .. k+D-1 are in flight while step k is multiplied.  Two slots suit
// the MFMA-bound shapes (a third measured slower at 4096 x 14336: more DMA in
// flight competes with the fragment reads); deeper rings serve latency-bound
// launches with few K-steps per workgroup, where each step would otherwise wait
// for one full memory round trip.
template <int BM, int BN, int NW, int D>
struct StreamGeom {
    static constexpr int kThreads = 64 * NW;
    static constexpr int kABytes = BM * kBK * 2;        // row-operand panel per K-step
    static constexpr int kBBytes = BN * kBK * 2;        // col-operand panel per K-step
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kStages = D;
    static constexpr int kLoadsA = kABytes / 1024 / NW;  // DMA instructions per wave
    static constexpr int kLoadsB = kBBytes / 1024 / NW;
    static constexpr int kLoads = kLoadsA + kLoadsB;
    static constexpr int kTileBytes = BM * BN * 2;       // bf16 output tile (epilogue)
    static constexpr int kEpiLoads = kTileBytes / 1024 / NW;
    // The epilogue operand tile fits one ring slot (BM, BN <= 128): it is fetched
    // into the first slot the K loop stops refilling, so its latency overlaps the
    // last K-steps instead of following them.
    static constexpr bool kEpiInSlot = kTileBytes <= kStageBytes && D >= 3;
    static_assert(D >= 2 && D <= 8, "ring depth");
    static_assert((D - 1) * kLoads + kEpiLoads <= 63, "vmcnt range");
    static_assert(kLoadsA >= 1 && kLoadsB >= 1 && kABytes % (1024 * NW) == 0 &&
                      kBBytes % (1024 * NW) == 0,
                  "panels must split into whole 1 KiB DMA blocks per wave");
    static_assert(kTileBytes <= kStages * kStageBytes, "epilogue tile must fit the ring");
    static_assert(kTileBytes % (1024 * NW) == 0, "epilogue DMA is whole 1 KiB blocks per wave");
};

// s_waitcnt vmcnt(n * LOADS), workgroup barrier; n < NMAX known only at run time.
template <int LOADS, int NMAX, int EXTRA = 0>
__device__ __forceinline__ void wait_panels_barrier(int n) {
    if constexpr (NMAX <= 1) {
        wait_vm_barrier<EXTRA>();
    } else {
        if (n >= NMAX - 1)
            wait_vm_barrier<(NMAX - 1) * LOADS + EXTRA>();
        else
            wait_panels_barrier<LOADS, NMAX - 1, EXTRA>(n);
    }
}

// Epilogue tile in LDS: [BM][BN] bf16.  BN a power of two: 16-byte chunk c of
// row r is stored at chunk position c ^ ((r ^ (r >> 5)) & (BN/8 - 1)), so 32
// consecutive rows at one chunk (MFMA-layout accesses) and 32 rows spaced 8
// apart (mirror reads) land on distinct positions.  BN = 192 (24 chunks): the
// XOR acts within each group of 8 chunks.  Either way the map is its own
// inverse for a fixed row.
template <int BN>
__device__ __forceinline__ int epi_pos(int row, int chunk) {
    if constexpr ((BN & (BN - 1)) == 0)
        return chunk ^ ((row ^ (row >> 5)) & (BN / 8 - 1));
    else
        return (chunk & ~7) | ((chunk ^ (row ^ (row >> 3))) & 7);
}
template <int BN>
__device__ __forceinline__ int epi_offset(int row, int col) {
    return row * BN + (epi_pos<BN>(row, col >> 3) << 3) + (col & 7);
}

// One segment of a workgroup's work: K-steps [kbeg, kend) of output tile
// tile_base + lt (its stream-K fixup when the tile is cut, and its epilogue when
// this workgroup completes it).  `smem`, `sink` and `s_arrived` are the caller's
// LDS: the ring of D K-step slots, the per-wave DMA sink and one arrival word.
// half >= 0: the segment computes column half `half` (BN wide) of the tile of
// the launch's 2*BN-wide tile grid (the apply stage's last round, see
// polar_stream_halves_kernel).  DG: the unit is a pair of diagonal tiles
// (GemmArgs::diag_pairs; tile (tm, tn) = (2p, 2p + 1) names its two panels).
template <int BM, int BN, Stage S, int NW, int D, int KT, bool DG = false>
__device__ __forceinline__ void stream_segment(const GemmArgs &g, uint16_t *smem, uint16_t *sink,
                                               uint32_t *s_arrived_p, int unit, int tile_base,
                                               int lt, int kbeg, int kend, int half = -1) {
    using Geo = StreamGeom<BM, BN, NW, D>;
    constexpr int kThreads = Geo::kThreads;
    // Wave pairs (8 waves on a 192x192 tile, whose 2 x 4 wave grid would not be
    // made of 32-wide MFMA blocks, or on a 256x128 apply tile, whose 2 x 4 grid
    // would read 5 fragments per 4 MFMAs): the tile is four wave tiles (96x96,
    // 128x64), each computed by two waves — wave w and w + 4 — that split every
    // K-step's four k16 slices between them (slices h and h + 2 for h = w / 4).
    // Each wave pair reads each fragment once, as one wave of a 4-wave kernel
    // does, and the two waves cover each other's LDS and barrier waits.  The
    // halves are added once after the K loop (acc(h = 0) + acc(h = 1)), so each
    // output sums its K terms in two interleaved chains: results differ in
    // rounding from the single-chain kernels.
    constexpr bool kPair = NW == 8 && ((BM == 192 && BN == 192) || (BM == 256 && BN == 128));
    constexpr int kGridWaves = kPair ? 4 : NW;
    // Diagonal pairs (DG, 64x64 tiles with 4 waves): waves 0-1 compute diagonal
    // tile 2p from the row panel, waves 2-3 tile 2p + 1 from the column panel.
    // Of a tile's 32x32 blocks the store needs (0,0), (0,1) and (1,1): wave h
    // (= w & 1) sums its diagonal block (h,h) over every k16 slice and the shared
    // block over its two slices of each K-step (h = 0: block (0,1) over slices
    // 0-1; h = 1: block (1,0), the transpose, over slices 2-3), which h = 0 adds
    // in transposed after the K loop.  Six MFMAs and six fragment reads per wave
    // and K-step, against four and eight for an off-diagonal tile.  Block (0,1)
    // then sums its K terms in two interleaved chains and wave 1 takes its slices
    // in the order 2, 3, 0, 1: results differ in rounding from single tiles.
    static_assert(!DG || (StageTraits<S>::kSymmetric && BM == 64 && BN == 64 && NW == 4),
                  "diagonal pairs: 64x64 tiles of a triangular stage, 4 waves");
    constexpr int WM = BM / 2, WN = DG ? BN : BN / (kGridWaves / 2);
    constexpr int SM = WM / 32, SN = WN / 32;
    constexpr int kMfmaPerSlice = SM * SN;
    // Threads that hold accumulators (the h = 0 waves in pair mode).
    constexpr int kAccThreads = kPair ? kThreads / 2 : kThreads;
    using Tr = StageTraits<S>;
    static_assert(!Tr::kSymmetric || BM == BN, "triangular stages need square tiles");
    static_assert(!Tr::kRowNC || BM % 64 == 0, "N-contiguous panel rows of whole 128 B");
    static_assert(!Tr::kColNC || BN % 64 == 0, "N-contiguous panel rows of whole 128 B");

    constexpr int kStages = Geo::kStages;
    // Apply stages: a·X is added into the accumulators at the K-steps whose operand
    // panel holds this tile's own X values (apply: the X rows of the tile's rows;
    // apply-right: the X columns of the tile's columns), so the epilogue reads no
    // X tile.  Only poly still reads an epilogue operand tile (A).
    // Wave tiles of 128x128 (4 waves on a 256x256 tile) hold 256 accumulator
    // registers per lane, which fit only as AGPRs: code that works on the
    // accumulators with vector ALU instructions inside the K loop (a·X) or with
    // large register buffers (the partial sums of the stream-K fixup) would force
    // them into VGPRs and spill, so these kernels add a·X in the epilogue and read
    // partials in small blocks.
    constexpr bool kBigAcc = (BM / 2) * (BN / (NW / 2)) >= 128 * 128;
    constexpr bool kAxInLoop = Tr::kEpilogue == Stage::Apply && !kBigAcc;
    constexpr bool kEpiLoad = Tr::kEpiOperand && !kAxInLoop;
    // DMA instructions per wave of the epilogue operand tile (two tiles for a
    // diagonal pair, which fill one ring slot)
    constexpr int kEpiLoadsU = DG ? 2 * Geo::kEpiLoads : Geo::kEpiLoads;
    static_assert(!DG || 2 * Geo::kTileBytes <= Geo::kStageBytes, "a pair's tiles fill one slot");
    static_assert((D - 1) * Geo::kLoads + kEpiLoadsU <= 63, "vmcnt range");
    // Fragment schedule: a whole K-step ahead for one MFMA per slice, else one slice.
    constexpr bool kStepFrags = kMfmaPerSlice == 1;
    uint32_t &s_arrived = *s_arrived_p;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wq = kPair ? (wave & 3) : wave;  // wave tile of this wave
    const int wr = wq & 1, wc = DG ? 0 : wq >> 1;
    const int dt = DG ? wave >> 1 : 0;  // diagonal pairs: this wave's tile of the two
    const int hr = DG ? wave & 1 : 0;   // and its row half
    const int kh = kPair ? (wave >> 2) : 0;    // pair mode: which half of the slices
    const bool acc_owner = !kPair || kh == 0;  // holds the tile's sums after the K loop
    const int nk = g.k_steps;
    const uint32_t smem_base = lds_addr(smem);
    const int64_t tstart = int64_t(lt) * nk;
    // The thread index is opaque to the optimizer from here on, so the many
    // per-lane offsets derived from it are formed inside each segment instead
    // of being kept (and spilled) across the segment loop.
    int tid = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;

    const int tlin = tile_base + lt;
    const int bt = tlin / g.tiles_per_batch;
    const int t = tlin - bt * g.tiles_per_batch;
    int tm, tn;
    tile_coords(g, Tr::kSymmetric, t, tm, tn);
    const int row0 = tm * BM, col0 = half >= 0 ? tn * (2 * BN) + half * BN : tn * BN;

    const i32x4 rs_row = make_buffer_rsrc(g.rowop + bt * g.sb_row, g.bytes_row);
    const i32x4 rs_col = make_buffer_rsrc(g.colop + bt * g.sb_col, g.bytes_col);

    // -------------------------------------------------------- DMA geometry
    // Per-lane byte offsets of this wave's DMA chunks at K-step 0 (kOob if the
    // chunk's row/column lies outside the matrix).
    // K-contiguous panel ([rows][64], 8 rows per 1 KiB instruction) or
    // N-contiguous panel ([64][rows], 512 / rows K-rows per instruction).
    // N-contiguous panels [64][rows]: 16-byte chunk q of the panel (q = 64 * DMA
    // instruction + lane, row-major) is K-row q / (rows / 8), position q % (rows / 8).
    constexpr int kAChunksPerKRow = BM / 8, kBChunksPerKRow = BN / 8;
    auto a_row = [&](int i) { return 8 * (wave * Geo::kLoadsA + i) + (lane >> 3); };
    auto a_chunk = [&](int i) { return (lane & 7) ^ kc_swz(a_row(i)); };
    auto a_krow = [&](int i) {  // N-contiguous row operand
        return ((wave * Geo::kLoadsA + i) * 64 + lane) / kAChunksPerKRow;
    };
    auto a_kpos = [&](int i) { return ((wave * Geo::kLoadsA + i) * 64 + lane) % kAChunksPerKRow; };
    auto b_krow = [&](int i) {  // N-contiguous column operand
        return ((wave * Geo::kLoadsB + i) * 64 + lane) / kBChunksPerKRow;
    };
    auto b_kpos = [&](int i) { return ((wave * Geo::kLoadsB + i) * 64 + lane) % kBChunksPerKRow; };
    auto b_row = [&](int i) { return 8 * (wave * Geo::kLoadsB + i) + (lane >> 3); };
    auto b_chunk = [&](int i) { return (lane & 7) ^ kc_swz(b_row(i)); };

    uint32_t off_a[Geo::kLoadsA], off_b[Geo::kLoadsB];
#pragma unroll
    for (int i = 0; i < Geo::kLoadsA; ++i) {
        if constexpr (Tr::kRowNC) {
            const int krow = a_krow(i);
            const int c = a_kpos(i) ^ nc_swz<BM>(krow);
            const int col = row0 + 8 * c;
            off_a[i] =
                col < g.row_rows ? static_cast<uint32_t>((krow * g.ld_row + col) * 2) : kOob;
        } else {
            const int gr = row0 + a_row(i);
            off_a[i] = gr < g.row_rows
                           ? static_cast<uint32_t>((gr * g.ld_row + 8 * a_chunk(i)) * 2)
                           : kOob;
        }
    }
#pragma unroll
    for (int i = 0; i < Geo::kLoadsB; ++i) {
        if constexpr (Tr::kColNC) {
            const int krow = b_krow(i);
            const int c = b_kpos(i) ^ nc_swz<BN>(krow);
            const int col = col0 + 8 * c;
            off_b[i] =
                col < g.col_rows ? static_cast<uint32_t>((krow * g.ld_col + col) * 2) : kOob;
        } else {
            const int gr = col0 + b_row(i);
            off_b[i] = gr < g.col_rows
                           ? static_cast<uint32_t>((gr * g.ld_col + 8 * b_chunk(i)) * 2)
                           : kOob;
        }
    }

    auto a_dst = [&](int slot, int i) {
        return smem_base + slot * Geo::kStageBytes + (wave * Geo::kLoadsA + i) * 1024;
    };
    auto b_dst = [&](int slot, int i) {
        return smem_base + slot * Geo::kStageBytes + Geo::kABytes +
               (wave * Geo::kLoadsB + i) * 1024;
    };
    auto a_step = [&](int k0) -> uint32_t {
        return static_cast<uint32_t>((Tr::kRowNC ? k0 * g.ld_row : k0) * 2);
    };
    auto b_step = [&](int k0) -> uint32_t {
        return static_cast<uint32_t>((Tr::kColNC ? k0 * g.ld_col : k0) * 2);
    };
    // DMA instruction d (0 .. kLoads-1) of K-step `step` into `slot`, or, when
    // `live` is false, out-of-range zeros into this wave's sink block (the same
    // instruction, chosen by scalar operands).  Without KT, K-contiguous operands
    // have rows that extend to a multiple of 64 elements with zeros (A and P, a
    // padded copy of X, or X with n % 64 == 0), and N-contiguous operands end at
    // their buffer's num_records, past which the hardware returns zeros.
    // (An idle instruction whose row is outside the matrix wraps to offset 0:
    // an in-range read, also into the sink.)
    const uint32_t sink_base = lds_addr(sink) + wave * 1024;
    // KT (gram and apply-right reading X rows of n % 64 != 0 elements in place;
    // KT == 2, below, also covers an even n % 8 != 0): chunks at K positions past
    // the operand's K extent
    // (row_k, col_k; only in the last K-step) take an out-of-range offset, so
    // they read the zeros a padded copy of X would hold there, and the sums are
    // the padded copy's bit for bit.
    static_assert(!KT || (!Tr::kRowNC && !Tr::kColNC), "K masks of K-contiguous panels");
    auto dma_one = [&](int d, int step, int slot, bool live) {
        const int k0 = step * kBK;
        if (d < Geo::kLoadsA) {
            const uint32_t koff = live ? a_step(k0) : kOob;
            uint32_t off = off_a[d] + koff;
            if constexpr (KT) off = k0 + 8 * a_chunk(d) < g.row_k ? off : kOob;
            dma_16B(rs_row, live ? a_dst(slot, d) : sink_base, off);
        } else {
            const int i = d - Geo::kLoadsA;
            const uint32_t koff = live ? b_step(k0) : kOob;
            uint32_t off = off_b[i] + koff;
            if constexpr (KT) off = k0 + 8 * b_chunk(i) < g.col_k ? off : kOob;
            dma_16B(rs_col, live ? b_dst(slot, i) : sink_base, off);
        }
    };
    // KT with rows of n % 8 != 0 elements (gram reading X rows of even length in
    // place, 4-byte aligned): on the tile's last K-step the chunk that holds K
    // position n also holds the next row's first values (a matrix's last row:
    // zeros past the buffer).  Once this lane's DMA of that step has landed, its
    // positions >= n are zeroed in LDS before the step's barrier, so the operands
    // hold the zeros a zero-padded copy of X holds there.  tail_rem packs, per DMA
    // instruction d of this lane, the number of valid values (1..7) in its chunk of
    // that step in bits 4d..4d+3 (0: nothing to zero).
    static_assert(Geo::kLoads <= 16, "tail_rem holds 16 instructions");
    const bool tail_fix = KT == 2 && ((g.row_k | g.col_k) & 7) != 0 && kend == nk;
    uint64_t tail_rem = 0;
    if constexpr (KT == 2) {
        if (tail_fix) {
            const int k0 = (nk - 1) * kBK;
#pragma unroll
            for (int d = 0; d < Geo::kLoads; ++d) {
                const int rem = d < Geo::kLoadsA ? g.row_k - (k0 + 8 * a_chunk(d))
                                                 : g.col_k - (k0 + 8 * b_chunk(d - Geo::kLoadsA));
                if (rem > 0 && rem < kChunk) tail_rem |= uint64_t(rem) << (4 * d);
            }
        }
    }
    auto fix_tail = [&](int slot_) {
        if constexpr (KT == 2) {
            // an opaque copy of the wave index keeps this address arithmetic here
            // rather than hoisted out of the K loop (where its values would stay
            // live in scalar registers and spill)
            int wv = wave;
            asm volatile("" : "+s"(wv));
            const uint32_t base = smem_base + slot_ * Geo::kStageBytes + 16 * lane;
#pragma unroll
            for (int d = 0; d < Geo::kLoads; ++d) {
                const uint32_t dst =
                    d < Geo::kLoadsA
                        ? base + (wv * Geo::kLoadsA + d) * 1024
                        : base + Geo::kABytes + (wv * Geo::kLoadsB + d - Geo::kLoadsA) * 1024;
                // keep values 0 .. rem-1 of the chunk (all of it when rem is 0)
                const int rem = static_cast<int>((tail_rem >> (4 * d)) & 15u);
                u32x4 *q = reinterpret_cast<u32x4 *>(smem + (dst - smem_base) / 2);
                u32x4 v = *q;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t keep = rem == 0 || 2 * w + 1 < rem ? 0xffffffffu
                                          : 2 * w < rem              ? 0x0000ffffu
                                                                     : 0u;
                    v[w] &= keep;
                }
                *q = v;
            }
        }
    };
    auto issue_all = [&](int step, int slot) {
#pragma unroll
        for (int d = 0; d < Geo::kLoads; ++d) dma_one(d, step, slot, true);
    };

    // Epilogue operand tile (A for poly, X for apply) -> LDS ring slot `eslot`
    // (the tile may span several slots from slot 0), rows/cols outside the
    // matrix read as zero.  Diagonal pairs: both tiles, the second 8 KiB after
    // the first.
    auto issue_epi = [&](int eslot) {
        if constexpr (kEpiLoad) {
            const i32x4 rs_epi = make_buffer_rsrc(g.epi + bt * g.sb_epi, g.bytes_epi);
            constexpr int kChunksPerRow = BN / 8;
            constexpr int kTileChunks = BM * kChunksPerRow;
#pragma unroll
            for (int d = 0; d < kEpiLoadsU; ++d) {
                // LDS chunk q of the tile (row q / kChunksPerRow, position q %
                // kChunksPerRow) receives global chunk epi_pos(row, position).
                const int blk = wave * kEpiLoadsU + d;
                const int qt = blk * 64 + lane;
                const int et = DG ? qt / kTileChunks : 0;  // which tile of a pair
                const int q = DG ? qt - et * kTileChunks : qt;
                const int row = q / kChunksPerRow;
                const int c = epi_pos<BN>(row, q - row * kChunksPerRow);
                const int er0 = DG ? row0 + et * BM : row0, ec0 = DG ? er0 : col0;
                const int gr = er0 + row, gc = ec0 + 8 * c;
                const uint32_t v = (gr < g.out_rows && gc < g.out_cols)
                                       ? static_cast<uint32_t>((gr * g.ld_epi + gc) * 2)
                                       : kOob;
                dma_16B(rs_epi, smem_base + eslot * Geo::kStageBytes + blk * 1024, v);
            }
        }
    };

    // -------------------------------------------------------- main loop
    f32x16 acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // MFMA operand fragments of one k16 slice, double-buffered in registers.
    // Fragment f of k16 slice kk from `slot`: f < SM row-operand fragment f,
    // else column-operand fragment f - SM.
    auto load_frag = [&](int slot, int kk, int f, bf16x8 (&fr)[SM], bf16x8 (&fc)[SN]) {
        const uint16_t *as = smem + slot * (Geo::kStageBytes / 2);
        const uint16_t *bs = as + Geo::kABytes / 2;
        if (f < SM) {
            if constexpr (Tr::kRowNC)
                fr[f] = frag_nc_tr<BM>(as, wr * WM + f * 32 + ((lane >> 4) & 1) * 16, kk, lane);
            else
                fr[f] = frag_kc(as, wr * WM + f * 32 + (lane & 31), kk, lane);
        } else {
            const int j = f - SM;
            if constexpr (Tr::kColNC)
                fc[j] = frag_nc_tr<BN>(bs, wc * WN + j * 32 + ((lane >> 4) & 1) * 16, kk, lane);
            else
                fc[j] = frag_kc(bs, wc * WN + j * 32 + (lane & 31), kk, lane);
        }
    };
    auto load_frags = [&](int slot, int kk, bf16x8 (&fr)[SM], bf16x8 (&fc)[SN]) {
#pragma unroll
        for (int f = 0; f < SM + SN; ++f) load_frag(slot, kk, f, fr, fc);
    };
    // a·X into the accumulators from the panel of global K-step kg in `slot`,
    // when that step's 64 K-values are 64 of this tile's rows (apply: X rows;
    // the column panel [64][BN] holds X[k][col0 + c]) or columns (apply-right:
    // X columns; the row panel [BM][64] holds X[row0 + r][k]).  Each lane adds
    // the 4 consecutive values its accumulator elements 4q..4q+3 cover, once
    // per output element over the whole K loop.
    auto add_ax = [&](int slot, int kg) {
        if constexpr (kAxInLoop) {
            if (!acc_owner) return;  // wave pairs: a·X goes into the h = 0 half once
            const uint16_t *as = smem + slot * (Geo::kStageBytes / 2);
            const uint16_t *bs = as + Geo::kABytes / 2;
            const float a = g.s_epi;
            auto fma4 = [&](f32x16 &acc_ij, int q, u32x2 v) {
                float x[4];
                unpack4(v, x);
#pragma unroll
                for (int t = 0; t < 4; ++t) acc_ij[4 * q + t] = fmaf(a, x[t], acc_ij[4 * q + t]);
            };
            if constexpr (S == Stage::Apply) {
                const int rel = kg * kBK - row0;  // tile row of the step's first K-row
                if (rel < 0 || rel >= BM) return;
#pragma unroll
                for (int i = 0; i < SM; ++i) {
                    const int rb = wr * WM + 32 * i;
                    if (rb < rel || rb >= rel + kBK) continue;
                    const int kr = rb - rel + (lane & 31);
#pragma unroll
                    for (int j = 0; j < SN; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int c = wc * WN + 32 * j + 8 * q + 4 * (lane >> 5);
                            fma4(acc[i][j], q,
                                 *reinterpret_cast<const u32x2 *>(
                                     bs + nc_offset<BN>(kr, c >> 3) + (c & 7)));
                        }
                }
            } else {
                const int rel = kg * kBK - col0;  // tile column of the step's first K
                if (rel < 0 || rel >= BN) return;
#pragma unroll
                for (int j = 0; j < SN; ++j) {
                    const int cb = wc * WN + 32 * j;
                    if (cb < rel || cb >= rel + kBK) continue;
#pragma unroll
                    for (int i = 0; i < SM; ++i) {
                        const int r = wr * WM + 32 * i + (lane & 31);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int kc = cb - rel + 8 * q + 4 * (lane >> 5);
                            fma4(acc[i][j], q,
                                 *reinterpret_cast<const u32x2 *>(
                                     as + kc_offset(r, kc >> 3) + (kc & 7)));
                        }
                    }
                }
            }
        }
    };
    auto mfmas = [&](const bf16x8 (&fr)[SM], const bf16x8 (&fc)[SN]) {
#pragma unroll
        for (int i = 0; i < SM; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j) acc[i][j] = mfma_32x32x16(fc[j], fr[i], acc[i][j]);
    };
    // Last slice of a step: its MFMAs with the DMA of panel `step` interleaved,
    // about kLoads / kMfmaPerSlice instructions after each MFMA (into the sink
    // when `live` is false: the panel would be past the segment's end; a
    // branch around each DMA instead cost 3-4% of the step at 4096 x 14336),
    // and the next step's slice-0 fragment reads (from slot `nslot`, complete
    // once the step's barrier has passed) issued one after each MFMA too (0.7%
    // faster at 4096 x 14336 than reading them all first).
    auto mfmas_with_dma_frags = [&](const bf16x8 (&fr)[SM], const bf16x8 (&fc)[SN], int step,
                                    int slot_, bool live, int nslot,
                                    bf16x8 (&nfr)[SM], bf16x8 (&nfc)[SN], int nkk) {
#pragma unroll
        for (int m = 0; m < kMfmaPerSlice; ++m) {
            const int i = m / SN, j = m % SN;
            acc[i][j] = mfma_32x32x16(fc[j], fr[i], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
            if (m < SM + SN) load_frag(nslot, nkk, m, nfr, nfc);
#pragma unroll
            for (int d = m * Geo::kLoads / kMfmaPerSlice;
                 d < (m + 1) * Geo::kLoads / kMfmaPerSlice; ++d)
                dma_one(d, step, slot_, live);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int f = kMfmaPerSlice; f < SM + SN; ++f) load_frag(nslot, nkk, f, nfr, nfc);
    };
    static_assert(kBK / 16 == 4, "schedule below is written for four k16 slices per step");

    // Schedule per K-step k (slot k % kStages), slices s0..s3 of 16 K-values:
    //   frags(s1) | mfma(s0) | frags(s2) | mfma(s1) | frags(s3) | mfma(s2) |
    //   wait panel k+1, barrier | frags(next s0) | mfma(s3) + DMA panel k+kStages -> slot
    // Within each "frags | mfma" pair the fragment reads are issued one after
    // each MFMA (1-2% faster than all reads first at 4096 x 14336).
    // The barrier sits where every wave has read all of step k's slot into
    // registers; panels k+2 .. k+kStages-1 may still be in flight there.
    // With the epilogue tile in a slot (kEpiInSlot), the first step that issues
    // no panel (k = nkl - kStages) issues the epilogue operand tile into its
    // slot instead; every later wait lets those loads stay in flight.
    const int nkl = kend - kbeg;
    constexpr bool kEpiPrefetch = kEpiLoad && Geo::kEpiInSlot;
    // The wave pairs add their halves through the ring after the K loop, which
    // would overwrite an epilogue tile fetched into a ring slot during the loop.
    static_assert(!(kPair && kEpiPrefetch), "wave pairs cannot prefetch the epilogue tile");
    const int npro = nkl < kStages ? nkl : kStages;
    for (int i = 0; i < npro; ++i) issue_all(kbeg + i, i);
    int epi_slot = 0;
    if (tail_fix && nkl == 1) {  // the segment is the tile's last K-step alone
        wait_vm<0>();
        fix_tail(0);
    }
    if constexpr (kEpiPrefetch) {
        if (nkl < kStages) {
            epi_slot = nkl;  // a slot the K loop never fills
            issue_epi(epi_slot);
            wait_panels_barrier<Geo::kLoads, kStages, kEpiLoadsU>(npro - 1);
        } else {
            epi_slot = (nkl - kStages) % kStages;
            wait_panels_barrier<Geo::kLoads, kStages>(npro - 1);
        }
    } else {
        wait_panels_barrier<Geo::kLoads, kStages>(npro - 1);
    }
    int slot = 0;
    if constexpr (kPair) {
        // This wave's k16 slices of every K-step: ka = h and kb = h + 2, in the
        // 4-wave kernel's schedule with two slices per step:
        //   frags(kb) | mfma(ka) | wait panel k+1, barrier | frags(next ka) |
        //   mfma(kb) + DMA panel k+kStages -> slot
        const int ka = kh, kb = kh + 2;
        bf16x8 fr0[SM], fc0[SN], fr1[SM], fc1[SN];
        load_frags(0, ka, fr0, fc0);
        for (int k = 0; k < nkl; ++k) {
            const int next = slot + 1 == kStages ? 0 : slot + 1;
            if constexpr (kAxInLoop) add_ax(slot, kbeg + k);
            load_frags(slot, kb, fr1, fc1);
            mfmas(fr0, fc0);
            for (int z = 0; z < kMfmaPerSlice; ++z) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // the waits of the schedule below (panel k+1; later DMA groups in flight)
            const int after = (npro - k - 2 > 0 ? npro - k - 2 : 0) + (k < kStages - 2 ? k : kStages - 2);
            if (tail_fix && k == nkl - 2) {
                wait_vm<0>();
                fix_tail(next);
            }
            wait_panels_barrier<Geo::kLoads, kStages - 1>(after);
            mfmas_with_dma_frags(fr1, fc1, kbeg + k + kStages, slot, k + kStages < nkl, next, fr0,
                                 fc0, ka);
            __builtin_amdgcn_sched_barrier(0);
            slot = next;
        }
    } else if constexpr (DG) {
        // Fragments of one K-step, slices taken in the order s_i = (2h + i) mod 4:
        // o[i] = rows 32h.. (own block), t[i] = rows 32(1-h).. (shared block, i < 2).
        bf16x8 ao[4], at[2], bo[4], bt[2];
        auto frag_of = [&](const uint16_t *ps, int rbase, int kk) {
            if constexpr (Tr::kRowNC)
                return frag_nc_tr<BM>(ps, rbase + ((lane >> 4) & 1) * 16, kk, lane);
            else
                return frag_kc(ps, rbase + (lane & 31), kk, lane);
        };
        auto read_dg = [&](int sl, bf16x8 (&o)[4], bf16x8 (&t)[2]) {
            const uint16_t *ps = smem + sl * (Geo::kStageBytes / 2) + dt * (Geo::kABytes / 2);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kk = (2 * hr + i) & 3;
                o[i] = frag_of(ps, 32 * hr, kk);
                if (i < 2) t[i] = frag_of(ps, 32 - 32 * hr, kk);
            }
        };
        auto step_dg = [&](int k, const bf16x8 (&o)[4], const bf16x8 (&t)[2], bf16x8 (&no)[4],
                           bf16x8 (&nt)[2]) {
            const int next = slot + 1 == kStages ? 0 : slot + 1;
            // the waits of the one-MFMA-per-slice schedule below
            const int after = (npro - k - 2 > 0 ? npro - k - 2 : 0) + (k < kStages - 2 ? k : kStages - 2);
            if (tail_fix && k == nkl - 2) {
                wait_vm<0>();
                fix_tail(next);
            }
            if (kEpiPrefetch && k > nkl - kStages)
                wait_panels_barrier<Geo::kLoads, kStages - 1, kEpiLoadsU>(after);
            else
                wait_panels_barrier<Geo::kLoads, kStages - 1>(after);
            read_dg(next, no, nt);  // stale on the last step, not used
            __builtin_amdgcn_sched_barrier(0);
            constexpr int kM = 6;
            const int dstep = kbeg + k + kStages;
            const bool live = k + kStages < nkl;
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                // m = 0..5: own(0), shared(0), own(1), shared(1), own(2), own(3)
                const int i = m < 4 ? m >> 1 : m - 2;
                if (m < 4 && (m & 1))
                    acc[0][1] = mfma_32x32x16(t[i & 1], o[i], acc[0][1]);
                else
                    acc[0][0] = mfma_32x32x16(o[i], o[i], acc[0][0]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int d = m * Geo::kLoads / kM; d < (m + 1) * Geo::kLoads / kM; ++d)
                    dma_one(d, dstep, slot, live);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (kEpiPrefetch) {
                if (k == nkl - kStages) issue_epi(epi_slot);
            }
            slot = next;
        };
        read_dg(0, ao, at);
        int k = 0;
        for (; k + 1 < nkl; k += 2) {
            step_dg(k, ao, at, bo, bt);
            step_dg(k + 1, bo, bt, ao, at);
        }
        if (k < nkl) step_dg(k, ao, at, bo, bt);
    } else if constexpr (kStepFrags) {
        // One MFMA per k16 slice (32x32 wave tiles): a slice's fragment reads
        // cannot hide behind the single MFMA issued before them, so every slice
        // would wait out the LDS latency.  Instead all fragments of step k+1 are
        // read right after step k's barrier, while step k's MFMAs (on fragments
        // read one step earlier) run.  MFMAs and a·X additions keep the order of
        // the schedule below, so results are the same bits.
        bf16x8 ar[4][SM], ac[4][SN], br[4][SM], bc[4][SN];
        auto read_step = [&](int sl, bf16x8 (&r)[4][SM], bf16x8 (&c)[4][SN]) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) load_frags(sl, kk, r[kk], c[kk]);
        };
        auto step = [&](int k, const bf16x8 (&r)[4][SM], const bf16x8 (&c)[4][SN],
                        bf16x8 (&nr)[4][SM], bf16x8 (&nc)[4][SN]) {
            const int next = slot + 1 == kStages ? 0 : slot + 1;
            // the same waits as the schedule below: panel k+1, before this
            // step's DMA group
            const int after = (npro - k - 2 > 0 ? npro - k - 2 : 0) + (k < kStages - 2 ? k : kStages - 2);
            if (tail_fix && k == nkl - 2) {
                wait_vm<0>();
                fix_tail(next);
            }
            if (kEpiPrefetch && k > nkl - kStages)
                wait_panels_barrier<Geo::kLoads, kStages - 1, kEpiLoadsU>(after);
            else
                wait_panels_barrier<Geo::kLoads, kStages - 1>(after);
            read_step(next, nr, nc);  // stale on the last step, not used
            __builtin_amdgcn_sched_barrier(0);
            constexpr int kM = 4 * kMfmaPerSlice;
            const int dstep = kbeg + k + kStages;
            const bool live = k + kStages < nkl;
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                const int kk = m / kMfmaPerSlice, ij = m % kMfmaPerSlice;
                acc[ij / SN][ij % SN] =
                    mfma_32x32x16(c[kk][ij % SN], r[kk][ij / SN], acc[ij / SN][ij % SN]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int d = m * Geo::kLoads / kM; d < (m + 1) * Geo::kLoads / kM; ++d)
                    dma_one(d, dstep, slot, live);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (kAxInLoop) {
                if (k + 1 < nkl) add_ax(next, kbeg + k + 1);
            }
            if constexpr (kEpiPrefetch) {
                if (k == nkl - kStages) issue_epi(epi_slot);
            }
            slot = next;
        };
        if constexpr (kAxInLoop) add_ax(0, kbeg);
        read_step(0, ar, ac);
        int k = 0;
        for (; k + 1 < nkl; k += 2) {
            step(k, ar, ac, br, bc);
            step(k + 1, br, bc, ar, ac);
        }
        if (k < nkl) step(k, ar, ac, br, bc);
    } else {
        bf16x8 fr0[SM], fc0[SN], fr1[SM], fc1[SN];
        load_frags(0, 0, fr0, fc0);
        for (int k = 0; k < nkl; ++k) {
            const int next = slot + 1 == kStages ? 0 : slot + 1;
            if constexpr (kAxInLoop) add_ax(slot, kbeg + k);
            load_frags(slot, 1, fr1, fc1);
            mfmas(fr0, fc0);
            for (int z = 0; z < kMfmaPerSlice; ++z) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_frags(slot, 2, fr0, fc0);
            mfmas(fr1, fc1);
            for (int z = 0; z < kMfmaPerSlice; ++z) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_frags(slot, 3, fr1, fc1);
            mfmas(fr0, fc0);
            for (int z = 0; z < kMfmaPerSlice; ++z) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // Wait for panel k+1.  The DMA groups issued after it (each step issues
            // one, to the ring or the sink; the prologue issued npro) may stay in
            // flight: prologue panels k+2 .. npro-1 and the groups of steps
            // k+2-kStages .. k-1, at most kStages-2 groups (plus the epilogue tile
            // once issued).  Unconditional, also on the last step (nothing needed is
            // in flight then, and the fragments read from the stale slot are not
            // used): a branch around these LDS reads makes the compiler's wait
            // counts on the join below assume none were issued, and the slice-3
            // MFMAs would then wait for all of them.
            const int after = (npro - k - 2 > 0 ? npro - k - 2 : 0) + (k < kStages - 2 ? k : kStages - 2);
            if (tail_fix && k == nkl - 2) {
                wait_vm<0>();
                fix_tail(next);
            }
            if (kEpiPrefetch && k > nkl - kStages)
                wait_panels_barrier<Geo::kLoads, kStages - 1, kEpiLoadsU>(after);
            else
                wait_panels_barrier<Geo::kLoads, kStages - 1>(after);
            mfmas_with_dma_frags(fr1, fc1, kbeg + k + kStages, slot, k + kStages < nkl, next, fr0,
                                 fc0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kEpiPrefetch) {
                if (k == nkl - kStages) issue_epi(epi_slot);
            }
            slot = next;
        }
    }
    // All waves are done with the ring (and no DMA is outstanding).
    wait_vm_barrier<0>();

    // Diagonal pairs: wave h = 1's block (1,0) over slices 2-3 goes through the ring
    // ([32][33] floats per tile, in a slot the epilogue tile was not fetched into)
    // and is added transposed into wave h = 0's block (0,1): (0,1)[r][c] += (1,0)[c][r].
    if constexpr (DG) {
        const int red_slot = kEpiPrefetch ? (epi_slot + 1) % kStages : 0;
        float *red = reinterpret_cast<float *>(smem + red_slot * (Geo::kStageBytes / 2)) +
                     dt * (32 * 33);
        static_assert(2 * 32 * 33 * 4 <= Geo::kStageBytes, "pair reduction fits a slot");
        if (hr == 1) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    red[(lane & 31) * 33 + 8 * q + 4 * (lane >> 5) + e] = acc[0][1][4 * q + e];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (hr == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[0][1][4 * q + e] += red[(8 * q + 4 * (lane >> 5) + e) * 33 + (lane & 31)];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    // Wave pairs: the h = 1 wave's sums are added into its partner's through the
    // ring, in two rounds of accumulator blocks (each round's buffer fits the
    // ring): f32x4 group e4 of block f of wave tile wq at [wq][f][e4][lane].
    if constexpr (kPair) {
        constexpr int kF = SM * SN;
        constexpr int kF0 = (kF + 1) / 2;
        static_assert(4 * kF0 * 4 * 64 * 16 <= kStages * Geo::kStageBytes,
                      "pair reduction buffer must fit the ring");
        f32x4 *buf = reinterpret_cast<f32x4 *>(smem);
        auto round = [&](auto lo_c, auto hi_c) {
            constexpr int lo = decltype(lo_c)::value, hi = decltype(hi_c)::value;
            if (kh == 1) {
#pragma unroll
                for (int f = lo; f < hi; ++f)
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4) {
                        const f32x16 &a = acc[f / SN][f % SN];
                        buf[((wq * kF0 + (f - lo)) * 4 + e4) * 64 + lane] =
                            f32x4{a[4 * e4], a[4 * e4 + 1], a[4 * e4 + 2], a[4 * e4 + 3]};
                    }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (kh == 0) {
#pragma unroll
                for (int f = lo; f < hi; ++f)
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4) {
                        const f32x4 v = buf[((wq * kF0 + (f - lo)) * 4 + e4) * 64 + lane];
                        f32x16 &a = acc[f / SN][f % SN];
#pragma unroll
                        for (int t = 0; t < 4; ++t) a[4 * e4 + t] = a[4 * e4 + t] + v[t];
                    }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        round(std::integral_constant<int, 0>{}, std::integral_constant<int, kF0>{});
        round(std::integral_constant<int, kF0>{}, std::integral_constant<int, kF>{});
    }

    // -------------------------------------------------------- stream-K fixup
    bool epi_issued = false;
    if (!DG && (kbeg != 0 || kend != nk)) {  // (diagonal pairs are never cut)
        // This tile is cut between units u0 .. u1.  Each contributor but the
        // last stores its fp32 partial and counts itself in; the last one to
        // arrive forms p(u1) + p(u1 - 1) + ... + p(u0) in that fixed order (so
        // results do not depend on arrival order) and runs the epilogue.
        const int u0 = sk_unit_of(g, tstart), u1 = sk_unit_of(g, tstart + nk - 1);
        const uint32_t others = static_cast<uint32_t>(u1 - u0);
        uint64_t *cnt = g.counters + lt;
        const uint64_t tok = uint64_t(g.token) << 32;
        auto count_of = [&](uint64_t w) -> uint32_t {
            return (w & 0xffffffff00000000ull) == tok ? static_cast<uint32_t>(w) : 0u;
        };
        // Partials and counters are accessed device-coherently (sc1 stores and
        // loads, agent-scope atomics), so no whole-cache write-back or
        // invalidate is needed: a contributor's stores are complete before its
        // count is added, and the last contributor reads them after seeing
        // every count.  The L2 contents the other workgroups are streaming
        // from stay intact.
        constexpr int kSc1 = 16;  // cache-policy bits of a device-scope access
        const int64_t slot_bytes = int64_t(BM) * BN * 4;
        const __amdgpu_buffer_rsrc_t rs_part =
            __builtin_amdgcn_make_buffer_rsrc(g.partials, 0, 0x7fffffff, 0x00020000);
        auto lane_base = [&](int u) {
            return static_cast<uint32_t>(int64_t(sk_slot(u, lt)) * slot_bytes) + tid * 16;
        };
        // Slot layout: 16-byte chunk c = (i * SN + j) * 4 + q of every thread that
        // holds accumulators, thread-minor, so each access instruction covers 1 KiB
        // contiguously.
        constexpr uint32_t kChunkStride = kAccThreads * 16;
        auto store_own = [&]() {
            if (!acc_owner) return;
            const uint32_t base = lane_base(unit);
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        __builtin_amdgcn_raw_buffer_store_b128(
                            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                  acc[i][j][4 * q + 3]},
                            rs_part, base + ((i * SN + j) * 4 + q) * kChunkStride, 0, kSc1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        };
        if (tid == 0)
            s_arrived = count_of(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        __syncthreads();
        bool last = __builtin_amdgcn_readfirstlane(s_arrived) == others;
        bool stored = false;
        if (!last) {
            store_own();
            stored = true;
            __syncthreads();
            if (tid == 0) {
                // count this unit in: compare-and-swap, starting from zero when the
                // word holds another launch's token (each failed exchange means
                // another contributor got in, so at most two retries)
                uint64_t old = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                uint32_t before = count_of(old);
                while (!__hip_atomic_compare_exchange_strong(
                    cnt, &old, tok | (before + 1u), __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                    __HIP_MEMORY_SCOPE_AGENT))
                    before = count_of(old);
                s_arrived = before;
            }
            __syncthreads();
            last = __builtin_amdgcn_readfirstlane(s_arrived) == others;
        }
        if (!last) return;
        // Every other contributor has counted itself in: the word is this
        // unit's alone now.  Leave a zero count under this launch's token (a
        // replay of the launch reuses the token).
        if (tid == 0) __hip_atomic_store(cnt, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The epilogue operand tile (poly's A tile, which fills the idle ring) is
        // fetched now, so that its round trip overlaps the partials' reads
        // instead of following them.
        if constexpr (kEpiLoad && !kEpiPrefetch) {
            issue_epi(0);
            epi_issued = true;
        }
        // Own partial first or second in the order: add the others to it in
        // place (x + y == y + x).  Further back: start from p(u1) in memory.
        const bool from_memory = u1 - unit >= 2;
        if (from_memory && !stored) store_own();  // read back by the same lanes
        // Partials are read a row-block (16 chunks per lane) at a time, the
        // next block's loads in flight while the current one is added.
        auto add_partial = [&](int u, bool assign) {
            if (!acc_owner) return;
            const uint32_t base = lane_base(u);
            // blocks of kBlk accumulator tiles (i, j), the next block's loads in
            // flight while one is added (one row-block of SN tiles; one tile
            // for the 256-register accumulators)
            constexpr int kBlk = kBigAcc ? 1 : SN;
            constexpr int kBlocks = SM * SN / kBlk;
            f32x4 x[2][kBlk * 4];
            auto load_block = [&](int blk, f32x4 (&dst)[kBlk * 4]) {
#pragma unroll
                for (int c = 0; c < kBlk * 4; ++c)
                    dst[c] = __builtin_amdgcn_raw_buffer_load_b128(
                        rs_part, base + (blk * kBlk * 4 + c) * kChunkStride, 0, kSc1);
            };
            load_block(0, x[0]);
#pragma unroll
            for (int blk = 0; blk < kBlocks; ++blk) {
                if (blk + 1 < kBlocks) load_block(blk + 1, x[(blk + 1) & 1]);
#pragma unroll
                for (int t = 0; t < kBlk; ++t) {
                    const int ij = blk * kBlk + t, i = ij / SN, j = ij % SN;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[i][j][4 * q + e] = assign ? x[blk & 1][t * 4 + q][e]
                                                          : acc[i][j][4 * q + e] +
                                                                x[blk & 1][t * 4 + q][e];
                }
            }
        };
        if (from_memory) add_partial(u1, true);
        for (int u = from_memory ? u1 - 1 : u1; u >= u0; --u)
            if (from_memory || u != unit) add_partial(u, false);
    }

    // -------------------------------------------------------- epilogue
    uint16_t *tile = smem + epi_slot * (Geo::kStageBytes / 2);
    // element (row, col) of staged output tile ot
    auto at = [&](int ot, int row, int col) -> uint16_t * {
        return tile + ot * (BM * BN) + epi_offset<BN>(row, col);
    };
    uint16_t *out = g.out + bt * g.sb_out;
    const __amdgpu_buffer_rsrc_t rs_out =
        __builtin_amdgcn_make_buffer_rsrc(out, 0, 0x7fffffff, 0x00020000);
    const bool diag = Tr::kSymmetric && (DG || tm == tn);
    constexpr int kOutTiles = DG ? 2 : 1;  // staged [BM][BN] tiles, one after the other

    if constexpr (kEpiLoad && !kEpiPrefetch) {
        if (!epi_issued) issue_epi(0);
        wait_vm_barrier<0>();
    }

    // Each lane turns its accumulators into bf16 results in place (pair mode:
    // the h = 0 waves, which hold the sums).
    if (acc_owner) {
#pragma unroll
        for (int i = 0; i < SM; ++i) {
            const int r = wr * WM + i * 32 + (lane & 31);
#pragma unroll
            for (int j = 0; j < SN; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // diagonal pairs: block (h,h), and (0,1) for h = 0
                    if (DG && hr == 1 && j == 1) continue;
                    const int cb = DG ? (j == 0 ? 32 * hr : 32) : wc * WN + j * 32;
                    const int c = cb + 8 * q + 4 * (lane >> 5);
                    u32x2 *p = reinterpret_cast<u32x2 *>(at(dt, r, c));
                    float e[4] = {0.f, 0.f, 0.f, 0.f};
                    uint16_t h[4];
                    if constexpr (kAxInLoop) {
#pragma unroll
                        for (int t = 0; t < 4; ++t) h[t] = f32_to_bf16_bits(acc[i][j][4 * q + t]);
                    } else {
                        if constexpr (kEpiLoad) unpack4(*p, e);
                        epilogue_values<S>(acc[i][j], q, e, g, h);
                    }
                    *p = pack4(h);
                }
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // The tile's stores, with the cache policy GemmArgs::out_cpol as the constant
    // kAux of the store instructions (the switch below picks one instantiation).
    auto store_out = [&](auto aux_c) {
        constexpr int kAux = decltype(aux_c)::value;
        auto st16 = [&](u32x4 v, int elem) {
            __builtin_amdgcn_raw_buffer_store_b128(v, rs_out, static_cast<uint32_t>(elem * 2), 0,
                                                   kAux);
        };
        // Coalesced store of the tile: 16-byte chunks, consecutive threads along a row.
        constexpr int kChunksPerRow = BN / 8;
        for (int idx = tid; idx < kOutTiles * BM * kChunksPerRow; idx += kThreads) {
            // diagonal pairs: tile ot of the two at (row0 + ot * BM, row0 + ot * BM)
            const int ot = DG ? idx / (BM * kChunksPerRow) : 0;
            const int ti = DG ? idx - ot * (BM * kChunksPerRow) : idx;
            int row = ti / kChunksPerRow;
            const int c = ti % kChunksPerRow;
            // out_vec 3: even rows first, then odd ones, so that the rows a wave stores
            // share one parity and so one store path (row0 is even)
            if (!Tr::kSymmetric && g.out_vec == 3) row = row < BM / 2 ? 2 * row : 2 * row - (BM - 1);
            const int sr0 = DG ? row0 + ot * BM : row0, sc0 = DG ? sr0 : col0;
            const int gr = sr0 + row, gc = sc0 + 8 * c;
            if constexpr (!Tr::kSymmetric) {
                if (gr >= g.out_rows || gc >= g.out_cols) continue;
            }
            u32x4 v;
            if (!diag) {
                v = *reinterpret_cast<const u32x4 *>(at(ot, row, 8 * c));
            } else {
                // Diagonal tile: element (r, c) comes from the upper-triangle source
                // min/max(r, c), so the stored matrix is bitwise symmetric.
                uint32_t hh[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int col = 8 * c + e;
                    hh[e] = row <= col ? *at(ot, row, col) : *at(ot, col, row);
                }
                v = u32x4{hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16), hh[4] | (hh[5] << 16),
                          hh[6] | (hh[7] << 16)};
            }
            // out_vec 3: a row starts on a 4-byte boundary when its element offset from
            // the (4-byte aligned) out, bt * sb_out + gr * ld_out, is even (parities of the
            // products and the sum from the low bits)
            const bool vec_row =
                g.out_vec == 2 ||
                (g.out_vec == 3 && (((bt & g.sb_out) ^ (gr & g.ld_out)) & 1) == 0);
            if (Tr::kSymmetric || g.out_vec == 1 || (vec_row && gc + 8 <= g.out_cols)) {
                st16(v, gr * g.ld_out + gc);
            } else {
                // rows of n % 8 != 0 elements: 2-byte stores up to the last column
                uint16_t *dst = out + gr * g.ld_out + gc;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (gc + e < g.out_cols)
                        dst[e] = static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1)));
            }
        }

        // Mirrored store (symmetric stages, off-diagonal tiles): row c of the
        // mirror tile is column c of this tile; consecutive threads walk along it.
        if constexpr (Tr::kSymmetric) {
            if (!diag) {
                constexpr int kMirrorChunks = BM / 8;  // 16-byte chunks per mirror row
                for (int idx = tid; idx < BN * kMirrorChunks; idx += kThreads) {
                    const int mc = idx / kMirrorChunks, rb = idx % kMirrorChunks;
                    uint32_t hh[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) hh[e] = *at(0, 8 * rb + e, mc);
                    const u32x4 v{hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16),
                                  hh[4] | (hh[5] << 16), hh[6] | (hh[7] << 16)};
                    st16(v, (col0 + mc) * g.ld_out + row0 + 8 * rb);
                }
            }
        }
    };
    switch (g.out_cpol) {
        case 1: store_out(std::integral_constant<int, 2>{}); break;   // nt
        case 2: store_out(std::integral_constant<int, 16>{}); break;  // sc1
        case 3: store_out(std::integral_constant<int, 18>{}); break;  // nt sc1
        case 4: store_out(std::integral_constant<int, 17>{}); break;  // sc0 sc1
        default: store_out(std::integral_constant<int, 0>{}); break;
    }

    if constexpr (Tr::kSymmetric) {
        if constexpr (DG) {
            zero_past_grid<BM>(g, out, tm, tm, tid, kThreads);
            zero_past_grid<BM>(g, out, tm + 1, tm + 1, tid, kThreads);
        } else {
            zero_past_grid<BM>(g, out, tm, tn, tid, kThreads);
        }
    }
}

template <int BM, int BN, Stage S, int NW, int D, int KT>
__global__ __launch_bounds__(64 * NW) void polar_stream_kernel(GemmArgs g) {
    using Geo = StreamGeom<BM, BN, NW, D>;
    constexpr int kStages = Geo::kStages;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kStages * Geo::kStageBytes / 2];
    // 1 KiB per wave that the ring's idle DMA instructions write (out-of-range
    // offsets: zeros, no memory traffic) in the last kStages steps of a segment,
    // so that every step issues the same instructions: no branch around them.
    __shared__ __attribute__((aligned(1024))) uint16_t sink[NW * 512];
    __shared__ uint32_t s_arrived;
    const int nk = g.k_steps;

    // Work of this workgroup: iterations [it_lo, it_hi) of tiles tile_base + i / nk
    // (polar_schedule.hpp: XCD-contiguous whole tiles, then the stream-K units).
    int unit, tile_base;
    int64_t it_lo, it_hi;
    if (!workgroup_range(g, static_cast<int>(blockIdx.x), unit, tile_base, it_lo, it_hi)) return;

    // Segments are taken from the end of the range backwards: a unit first
    // computes the leading K-steps of its last tile (a partial the tile's owner
    // of the final K-steps will need) and ends with the trailing K-steps of its
    // first tile, so the contributor that arrives last usually finds the other
    // partials long written.
    for (int64_t hi = it_hi; hi > it_lo;) {
        const int lt = static_cast<int>((hi - 1) / nk);
        const int64_t tstart = int64_t(lt) * nk;
        const int64_t lo = tstart > it_lo ? tstart : it_lo;
        const int kbeg = static_cast<int>(lo - tstart), kend = static_cast<int>(hi - tstart);
        if (hi != it_hi) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        hi = lo;
        if constexpr (StageTraits<S>::kSymmetric && BM == 64 && BN == 64 && NW == 4) {
            if (is_diag_pair(g, (tile_base + lt) % g.tiles_per_batch)) {
                stream_segment<BM, BN, S, NW, D, KT, true>(g, smem, sink, &s_arrived, unit,
                                                           tile_base, lt, kbeg, kend);
                continue;
            }
        }
        stream_segment<BM, BN, S, NW, D, KT>(g, smem, sink, &s_arrived, unit, tile_base, lt, kbeg,
                                         kend);
    }
}

// Apply stage whose last round of 256x256 tiles would leave most CUs idle:
// whole 256x256 tiles [0, dp_tiles) one per workgroup (the first 8 * per_xcd
// workgroups, XCD-contiguous runs as in polar_stream_kernel), then each tile of
// [dp_tiles, total_tiles) as two 256x128 column halves, one per workgroup
// (g.sk_units = the number of halves, a multiple of 8; XCD-contiguous runs of
// halves).  A half computes its whole K range: no partials, no fix-up.  The
// halves run the wave-pair kernel (two K chains per output).
template <Stage S, int KT, int DH>
__global__ __launch_bounds__(512) void polar_stream_halves_kernel(GemmArgs g) {
    // ring: two 64 KiB slots for the whole tiles, DH 48 KiB slots for the halves
    constexpr int kWhole = 2 * StreamGeom<256, 256, 8, 2>::kStageBytes;
    constexpr int kHalf = DH * StreamGeom<256, 128, 8, DH>::kStageBytes;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[(kWhole > kHalf ? kWhole : kHalf) / 2];
    __shared__ __attribute__((aligned(1024))) uint16_t sink[8 * 512];
    __shared__ uint32_t s_arrived;
    const int w = static_cast<int>(blockIdx.x);
    const int dp_grid = 8 * g.per_xcd;
    if (w < dp_grid) {
        const int tile = (w & 7) * g.per_xcd + (w >> 3);
        if (tile >= g.dp_tiles) return;
        stream_segment<256, 256, S, 8, 2, KT>(g, smem, sink, &s_arrived, -1, tile, 0, 0,
                                              g.k_steps);
    } else {
        const int ws = w - dp_grid;
        const int v = (ws & 7) * (g.sk_units >> 3) + (ws >> 3);
        stream_segment<256, 128, S, 8, DH, KT>(g, smem, sink, &s_arrived, -1,
                                               g.dp_tiles + (v >> 1), 0, 0, g.k_steps, v & 1);
    }
}

// Instantiated (tile, waves, depth) combinations: 256x256 with 8 or 4 waves and
// two slots; 128x128 with 8 or 4 waves and 2 or 4 slots of 32 KiB (8 waves: two
// per SIMD, 64x32 wave tiles; [16,512,2048] 62.5 -> 59.0 us, [1,1024,4096]
// 46.3 -> 43.9 us against 4 waves); 192x192 with 8 waves (the wave pairs) and 2
// or 3 slots of 48 KiB (three by default: [4096,14336] gram 225 -> 212 us, poly
// 75 -> 72 us), or with 4 waves and 2 slots; other tiles with 4 waves and the
// depths their LDS allows (64x64: 2, 4 or 8 of 16 KiB; 128x256 and 256x128: 2 or 3
// of 48 KiB).
template <int BM, int BN>
constexpr bool depth_ok(int waves, int depth) {
    if (BM == 256 && BN == 256) return depth == 2 && (waves == 8 || waves == 4);
    if (BM == 128 && BN == 128) return (waves == 4 || waves == 8) && (depth == 2 || depth == 4);
    if (BM == 192 && BN == 192) return (depth == 2 && waves == 4) || ((depth == 2 || depth == 3) && waves == 8);
    if (waves != 4) return false;
    if (BM == 64 && BN == 64) return depth == 2 || depth == 4 || depth == 8;
    if (BM != BN) return depth == 2 || depth == 3;
    return depth == 2;
}

template <int BM, int BN, Stage S, int NW, int D, int KT>
const void *kernel_ptr() {
    return reinterpret_cast<const void *>(&polar_stream_kernel<BM, BN, S, NW, D, KT>);
}

// Kernel of (BM, BN, S, KT) for the given waves and depth, or null.
template <int BM, int BN, Stage S, int KT>
const void *kernel_for(int waves, int depth) {
    if (!depth_ok<BM, BN>(waves, depth)) return nullptr;
    if constexpr (BM == 256 && BN == 256) {
        return waves == 8 ? kernel_ptr<BM, BN, S, 8, 2, KT>() : kernel_ptr<BM, BN, S, 4, 2, KT>();
    } else if constexpr (BM == 128 && BN == 128) {
        if (waves == 8)
            return depth == 4 ? kernel_ptr<BM, BN, S, 8, 4, KT>() : kernel_ptr<BM, BN, S, 8, 2, KT>();
        return depth == 4 ? kernel_ptr<BM, BN, S, 4, 4, KT>() : kernel_ptr<BM, BN, S, 4, 2, KT>();
    } else if constexpr (BM == 64 && BN == 64) {
        return depth == 8   ? kernel_ptr<BM, BN, S, 4, 8, KT>()
               : depth == 4 ? kernel_ptr<BM, BN, S, 4, 4, KT>()
                            : kernel_ptr<BM, BN, S, 4, 2, KT>();
    } else if constexpr (BM != BN) {
        return depth == 3 ? kernel_ptr<BM, BN, S, 4, 3, KT>() : kernel_ptr<BM, BN, S, 4, 2, KT>();
    } else if constexpr (BM == 192) {
        // 8 waves: wave pairs splitting the K-slices (symmetric stages only)
        if (waves == 8)
            return depth == 3 ? kernel_ptr<BM, BN, S, 8, 3, KT>() : kernel_ptr<BM, BN, S, 8, 2, KT>();
        return kernel_ptr<BM, BN, S, 4, 2, KT>();
    } else {
        return kernel_ptr<BM, BN, S, 4, 2, KT>();
    }
}

template <Stage S, int KT>
const void *kernel_by_tile(int bm, int bn, int waves, int depth) {
    if (bm == 64 && bn == 64) return kernel_for<64, 64, S, KT>(waves, depth);
    if (bm == 128 && bn == 128) return kernel_for<128, 128, S, KT>(waves, depth);
    if (bm == 256 && bn == 256) return kernel_for<256, 256, S, KT>(waves, depth);
    if constexpr (S == Stage::Gram || S == Stage::Poly || S == Stage::GramT) {
        if (bm == 192 && bn == 192) return kernel_for<192, 192, S, KT>(waves, depth);
    }
    if constexpr (!StageTraits<S>::kSymmetric) {
        if (bm == 128 && bn == 256) return kernel_for<128, 256, S, KT>(waves, depth);
        if (bm == 256 && bn == 128) return kernel_for<256, 128, S, KT>(waves, depth);
    }
    return nullptr;
}

// kt: the K-masked variant (gram and apply-right only).
const void *stream_kernel(Stage s, int bm, int bn, int waves, int depth, int kt) {
    switch (s) {
        case Stage::Gram:
            return kt == 2   ? kernel_by_tile<Stage::Gram, 2>(bm, bn, waves, depth)
                   : kt == 1 ? kernel_by_tile<Stage::Gram, 1>(bm, bn, waves, depth)
                             : kernel_by_tile<Stage::Gram, 0>(bm, bn, waves, depth);
        case Stage::Poly:
            return kt ? nullptr : kernel_by_tile<Stage::Poly, 0>(bm, bn, waves, depth);
        case Stage::Apply:
            return kt ? nullptr : kernel_by_tile<Stage::Apply, 0>(bm, bn, waves, depth);
        case Stage::GramT:
            return kt ? nullptr : kernel_by_tile<Stage::GramT, 0>(bm, bn, waves, depth);
        case Stage::ApplyR:
            return kt == 1   ? kernel_by_tile<Stage::ApplyR, 1>(bm, bn, waves, depth)
                   : kt == 0 ? kernel_by_tile<Stage::ApplyR, 0>(bm, bn, waves, depth)
                             : nullptr;
    }
    return nullptr;
}

}  // namespace

int stream_waves(int bm, int bn, int requested) {
    return (bm == bn && (bm == 256 || bm == 192 || bm == 128) && requested == 8) ? 8 : 4;
}

bool stream_depth_supported(Stage s, int bm, int bn, int waves, int depth) {
    return stream_kernel(s, bm, bn, waves, depth, false) != nullptr;
}

// The halves kernel of an apply stage (polar_stream_halves_kernel) with a ring of
// `dh` slots for the halves (2 or 3), or null.
template <int DH>
const void *halves_kernel_d(Stage s, int kt) {
    switch (s) {
        case Stage::Apply:
            return kt ? nullptr : reinterpret_cast<const void *>(
                                      &polar_stream_halves_kernel<Stage::Apply, 0, DH>);
        case Stage::ApplyR:
            return kt == 2 ? nullptr
                   : kt ? reinterpret_cast<const void *>(
                            &polar_stream_halves_kernel<Stage::ApplyR, 1, DH>)
                      : reinterpret_cast<const void *>(
                            &polar_stream_halves_kernel<Stage::ApplyR, 0, DH>);
        default:
            return nullptr;
    }
}
const void *halves_kernel(Stage s, int kt, int dh) {
    return dh == 3 ? halves_kernel_d<3>(s, kt) : dh == 2 ? halves_kernel_d<2>(s, kt) : nullptr;
}

hipError_t launch_stream(Stage s, int bm, int bn, int waves, int depth, const GemmArgs &g,
                         hipStream_t stream, int k_mask) {
    if (g.halves) {
        // 256x256 whole tiles with 8 waves and two ring slots, then 256x128 halves
        const void *k = bm == 256 && bn == 256 && waves == 8 && depth == 2
                            ? halves_kernel(s, k_mask, g.halves)
                            : nullptr;
        if (k == nullptr || g.sk_units % 8 != 0) return hipErrorInvalidValue;
        const int grid = g.sk_units + 8 * g.per_xcd;
        GemmArgs copy = g;
        void *args[] = {&copy};
        return hipLaunchKernel(k, dim3(grid), dim3(512), args, 0, stream);
    }
    const void *k = stream_kernel(s, bm, bn, waves, depth, k_mask);
    if (k == nullptr) return hipErrorInvalidValue;
    const int grid = g.sk_units + 8 * g.per_xcd;
    GemmArgs copy = g;
    void *args[] = {&copy};
    return hipLaunchKernel(k, dim3(grid), dim3(64 * waves), args, 0, stream);
}

int stream_blocks_per_cu(Stage s, int bm, int bn, int waves, int depth) {
    const void *k = stream_kernel(s, bm, bn, waves, depth, false);
    if (k == nullptr) return 0;
    int n = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 64 * waves, 0) == hipSuccess ? n
                                                                                             : 0;
}

}  // namespace muon_polar
