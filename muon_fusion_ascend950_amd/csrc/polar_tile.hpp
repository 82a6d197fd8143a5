// polar_tile.hpp — gfx950 (CDNA4) bf16 MFMA tile engine shared by the three
// Polar Express stages.
//
// Building blocks:
//   * v_mfma_f32_32x32x16_bf16 on 64-wide wavefronts, fp32 accumulators;
//   * LDS tiles of kBK = 64 K-values, 16-byte chunks, XOR-swizzled so that the
//     MFMA fragment reads (ds_read_b128) and the tile writes are bank-conflict
//     free;
//   * a transposing LDS read (ds_read_b64_tr_b16) for the one operand that is
//     contracted along its row index (X in stage 3, Y = a·X + P·X).
//
// MFMA convention used throughout.  For D = A·B with A: 32x16 (m x k) and
// B: 16x32 (k x n) every lane l supplies 8 bf16 of row m = l%32 of A and of
// column n = l%32 of B, holding the same 8 K-slots (half h = l/32).  Lane l
// receives D[m][n] for n = l%32 and m = 8*(j/4) + 4*(l/32) + (j%4), j = 0..15.
// The kernels feed the operand that indexes output COLUMNS as the MFMA A side
// and the operand that indexes output ROWS as the MFMA B side, so each lane
// ends up with 4 consecutive output columns of one output row: row-major
// stores and epilogue loads are 8-byte vectors.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace muon_polar {

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using bf16x4 = __bf16 __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using u16x4 = uint16_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;    // K depth of one LDS stage
constexpr int kChunk = 8;  // bf16 values per 16-byte chunk

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  bf16 -> fp32 is exact (a 16-bit shift).  fp32 -> bf16 uses the
// language conversion, which rounds to nearest-even (gfx950 lowers it to the
// hardware v_cvt_pk_bf16_f32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// ---------------------------------------------------------------------------
// LDS swizzles.
//
// K-contiguous tile [rows][64]: 8 chunks of 16 B per 128-B row; chunk c of row r
// is stored at chunk position c ^ kc_swz(r).  Fragment reads take 32 consecutive
// rows at one chunk; any 8 consecutive rows (and rows r, r+8, ..., r+56) map to
// 8 distinct chunk positions, so both reads and row-wise writes are conflict free.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int kc_swz(int row) { return (row ^ (row >> 3)) & 7; }

__device__ __forceinline__ int kc_offset(int row, int chunk) {
    return row * kBK + ((chunk ^ kc_swz(row)) << 3);
}

// N-contiguous tile [64][BN] (stage-3 X panel, rows = K): chunk c of K-row k is
// stored at c ^ nc_swz(k).  A transposing read fetches 4 consecutive K-rows by
// 2 chunks (32 B) per 16-lane group, and a half-wave (two groups: 16 adjacent
// columns each) is served per LDS cycle.  Rows are 2*BN bytes apart, a multiple
// of the 256-byte bank window, so without the XOR all 4 rows would share banks.
// XOR by 4*(k%4) (BN = 128, 256) puts the half-wave's 16 chunks on 16 distinct
// positions of the window: no bank conflict.  BN = 64 rows have 8 chunks only;
// XOR by 2*(k%4) there (two groups then share banks).  BN = 192: rows are 384 B
// apart, so rows k and k+1 already sit half a window apart and rows k and k+2
// share banks; XOR by 4 on rows with bit 1 of k set (the half-wave's 4
// consecutive chunks start at a multiple of 4) moves rows k+2, k+3 onto the
// other half of each 8-chunk group: 16 distinct positions, and the XOR keeps
// every position inside its row of 24 chunks.
template <int BN>
__device__ __forceinline__ int nc_swz(int krow) {
    if constexpr (BN == 192) return ((krow >> 1) & 1) << 2;
    return BN >= 128 ? (krow & 3) << 2 : (krow & 3) << 1;
}
template <int BN>
__device__ __forceinline__ int nc_offset(int krow, int chunk) {
    return krow * BN + ((chunk ^ nc_swz<BN>(krow)) << 3);
}

// ---------------------------------------------------------------------------
// Global -> register tile loads (one K stage) with zero fill outside the
// extents.  VEC: 16-byte loads, valid when the leading dimension and the base
// are 16-byte aligned and the K / column extent is a multiple of 8 (so a chunk
// is entirely inside or outside).  Otherwise element loads with per-element
// masks.
// ---------------------------------------------------------------------------
template <bool VEC>
__device__ __forceinline__ u32x4 load_chunk(const uint16_t *__restrict__ p, bool row_ok, int k,
                                            int k_ext) {
    if constexpr (VEC) {
        if (row_ok && k < k_ext) return *reinterpret_cast<const u32x4 *>(p);
        return u32x4{0u, 0u, 0u, 0u};
    } else {
        uint32_t h[kChunk];
#pragma unroll
        for (int e = 0; e < kChunk; ++e) h[e] = (row_ok && k + e < k_ext) ? uint32_t(p[e]) : 0u;
        return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                     h[6] | (h[7] << 16)};
    }
}

// Tile [ROWS][kBK] of a K-contiguous matrix (row stride ld), rows row0.., K k0..
template <int ROWS, int NT, bool VEC>
struct KContigTile {
    static constexpr int kPerThread = ROWS * (kBK / kChunk) / NT;
    static_assert(kPerThread >= 1 && ROWS * (kBK / kChunk) % NT == 0, "tile/thread mismatch");
    u32x4 r[kPerThread];

    __device__ __forceinline__ void load(const uint16_t *__restrict__ base, int ld, int row0,
                                         int rows_ext, int k0, int k_ext, int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * NT;
            const int row = q >> 3, c = q & 7;
            const int gr = row0 + row, gk = k0 + c * kChunk;
            r[i] = load_chunk<VEC>(base + gr * ld + gk, gr < rows_ext, gk, k_ext);
        }
    }
    __device__ __forceinline__ void store(uint16_t *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * NT;
            *reinterpret_cast<u32x4 *>(lds + kc_offset(q >> 3, q & 7)) = r[i];
        }
    }
};

// Tile [kBK][BN] of an N-contiguous matrix (K rows k0.., columns col0..).
template <int BN, int NT, bool VEC>
struct NContigTile {
    static constexpr int kChunksPerRow = BN / kChunk;
    static constexpr int kPerThread = kBK * kChunksPerRow / NT;
    static_assert(kPerThread >= 1 && kBK * kChunksPerRow % NT == 0, "tile/thread mismatch");
    static_assert(kChunksPerRow >= 8, "nc swizzle needs BN >= 64");
    u32x4 r[kPerThread];

    __device__ __forceinline__ void load(const uint16_t *__restrict__ base, int ld, int k0,
                                         int k_ext, int col0, int col_ext, int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * NT;
            const int kr = q / kChunksPerRow, c = q % kChunksPerRow;
            const int gk = k0 + kr, gc = col0 + c * kChunk;
            r[i] = load_chunk<VEC>(base + gk * ld + gc, gk < k_ext, gc, col_ext);
        }
    }
    __device__ __forceinline__ void store(uint16_t *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = tid + i * NT;
            *reinterpret_cast<u32x4 *>(lds + nc_offset<BN>(q / kChunksPerRow, q % kChunksPerRow)) =
                r[i];
        }
    }
};

// ---------------------------------------------------------------------------
// MFMA fragment reads from LDS.
// ---------------------------------------------------------------------------
// 8 K-values (k16 step kk, half lane/32) of tile row `row` of a K-contiguous tile.
__device__ __forceinline__ bf16x8 frag_kc(const uint16_t *lds, int row, int kk, int lane) {
    const int chunk = kk * 2 + (lane >> 5);
    return *reinterpret_cast<const bf16x8 *>(lds + kc_offset(row, chunk));
}

// 8 K-values of tile column n0 + lane%16 (n0 a multiple of 16) of an N-contiguous
// tile, via two transposing reads of 4 K-rows each.  Within each group of 16
// lanes, lane i addresses K-row (kb + i/4), columns n0 + 4*(i%4) .. +3; after
// the transpose lane j holds column n0 + j for K-rows kb .. kb+3.
template <int BN>
__device__ __forceinline__ bf16x8 frag_nc_tr(const uint16_t *lds, int n0, int kk, int lane) {
    const int i = lane & 15;
    const int col = n0 + 4 * (i & 3);
    const int kb = kk * 16 + 8 * (lane >> 5) + (i >> 2);
    bf16x4 lo, hi;
    {
        const int kr = kb;
        const uint16_t *p = lds + nc_offset<BN>(kr, col >> 3) + (col & 7);
        lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4 *)(p));
    }
    {
        const int kr = kb + 4;
        const uint16_t *p = lds + nc_offset<BN>(kr, col >> 3) + (col & 7);
        hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4 *)(p));
    }
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace muon_polar

// ===========================================================================
// Direct global -> LDS loads (buffer_load_dwordx4 ... lds) for the streaming
// kernels.  One wave instruction moves 64 lanes x 16 B = 1 KiB into LDS at
// M0 + 16*lane, so the LDS image of a tile is chosen by which global chunk each
// lane fetches (the swizzles above are applied on the global side).  Lanes whose
// chunk lies outside the matrix use an offset beyond the buffer's num_records:
// the hardware returns zeros for them, which is how edge tiles are masked.
// ===========================================================================
namespace muon_polar {

using i32x4 = int32_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kOob = 0x80000000u;  // >= num_records of every buffer (< 2^31 bytes)

// Raw buffer resource (gfx9 family): base, stride 0, num_records in bytes.
// Arguments must be workgroup-uniform; readfirstlane places the descriptor in
// SGPRs even when the compiler computed a uniform value in vector registers.
__device__ __forceinline__ i32x4 make_buffer_rsrc(const void *base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(b & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>((b >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(bytes));
    r[3] = 0x00020000;
    return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// 16 B per lane from rsrc+voffset into LDS at lds_base(wave-uniform) + 16*lane.
// Issued as inline assembly so the compiler neither reorders LDS traffic around
// it nor inserts its own waits (the LDS-DMA builtin makes it wait for the transfer
// before every later LDS read); the kernels wait with vmcnt explicitly.  The LDS
// address is an M0 input operand, which the compiler loads itself, often with the
// instruction right before the asm.  On gfx9 an LDS DMA needs one wait state after
// a scalar write of M0; the compiler's hazard check cannot see inside the asm (for
// the LDS-DMA builtin it inserts that s_nop itself), so the asm carries it.  (A
// VALU write of an SGPR that a memory instruction reads needs five wait states; the
// descriptors are built well before their DMAs, none closer in the assembly of
// this build.)
__device__ __forceinline__ void dma_16B(i32x4 rsrc, uint32_t lds_base, uint32_t voffset) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory");
}

// Wait until at most N vector-memory operations of this wave are outstanding,
// finish this wave's LDS reads, then workgroup barrier.  The memory clobber keeps
// the compiler from moving LDS accesses across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// 16-byte store at device scope (sc1): written through the XCD's L2, so the line is
// not dirty there when the kernel ends, and a kernel on another XCD reads the data
// from the memory side.  For buffers the next kernel of a step reads.  `rs` covers
// 2^31 bytes from a workgroup-uniform base (store_rsrc) and `off` is the byte offset
// from it.  The store is the compiler's buffer-store builtin, not inline assembly:
// a 16-byte store reads its data registers after it issues, and only for an
// instruction it can see does the compiler insert the wait states that keep the
// next VALU write of those registers from changing the stored data.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t store_rsrc(void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void store16_sc1(__amdgpu_buffer_rsrc_t rs, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 16);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

}  // namespace muon_polar
