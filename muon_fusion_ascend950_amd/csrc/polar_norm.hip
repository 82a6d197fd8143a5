// polar_norm.hip — per-matrix normalisation X / (‖X‖_F·1.01 + 1e-6) ahead of the
// Polar Express iteration, with the rounding points of the reference recipe
// (examples/five_steps.py:18, tests/test_polar_step.py:39), evaluated there as
// bf16 torch ops:
//
//     norm = bf16(sqrt(Σ x²))            (fp32 sum of squares)
//     d    = bf16(bf16(norm · 1.01f) + 1e-6f)
//     y    = bf16(x / d)                 (fp32 division)
//
// Two bandwidth-bound passes: per-chunk fp32 partial sums of squares, then a
// scale pass in which every block re-sums its matrix's partials in the same
// fixed order (so all blocks of a matrix agree, and results are run-to-run
// identical).
#include "polar_kernels.h"
#include "polar_tile.hpp"

namespace muon_polar {

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float bf16_round(float v) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// Sum of v over the block in a fixed order: butterfly within each wave, then the
// four wave totals in index order.  `red` holds 4 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float t = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return t;
}

// Sum of squares of chunk c of matrix b into partial[b * chunks + c].
__global__ __launch_bounds__(kNormThreads) void norm_partial_kernel(const uint16_t *__restrict__ x,
                                                                    float *__restrict__ partial,
                                                                    int64_t mn, int chunks,
                                                                    int vec) {
    __shared__ float red[4];
    const int b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
    const uint16_t *base = x + int64_t(b) * mn;
    const int64_t e0 = int64_t(c) * kNormChunk;
    const int64_t e1 = e0 + kNormChunk < mn ? e0 + kNormChunk : mn;
    float acc = 0.0f;
    if (vec) {  // mn % 8 == 0 and 16-byte aligned rows of 8 elements
        for (int64_t e = e0 + threadIdx.x * 8; e < e1; e += kNormThreads * 8) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(base + e);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float lo = bf16_bits_to_f32(v[w] & 0xffffu);
                const float hi = bf16_bits_to_f32(v[w] >> 16);
                acc = fmaf(lo, lo, acc);
                acc = fmaf(hi, hi, acc);
            }
        }
    } else {
        for (int64_t e = e0 + threadIdx.x; e < e1; e += kNormThreads) {
            const float f = bf16_bits_to_f32(base[e]);
            acc = fmaf(f, f, acc);
        }
    }
    const float t = block_sum(acc, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = t;
}

// y = bf16(x / d) over chunk c of matrix b, d from the matrix's partial sums.
__global__ __launch_bounds__(kNormThreads) void norm_scale_kernel(const uint16_t *__restrict__ x,
                                                                  uint16_t *__restrict__ y,
                                                                  const float *__restrict__ partial,
                                                                  int64_t mn, int chunks, int vec) {
    __shared__ float red[4];
    const int b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
    float s = 0.0f;
    for (int i = threadIdx.x; i < chunks; i += kNormThreads) s += partial[int64_t(b) * chunks + i];
    const float total = block_sum(s, red);
    const float norm = bf16_round(sqrtf(total));
    const float d = bf16_round(bf16_round(norm * 1.01f) + 1e-6f);

    const uint16_t *xb = x + int64_t(b) * mn;
    uint16_t *yb = y + int64_t(b) * mn;
    const int64_t e0 = int64_t(c) * kNormChunk;
    const int64_t e1 = e0 + kNormChunk < mn ? e0 + kNormChunk : mn;
    if (vec) {
        for (int64_t e = e0 + threadIdx.x * 8; e < e1; e += kNormThreads * 8) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(xb + e);
            u32x4 o;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(v[w] & 0xffffu) / d);
                const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(v[w] >> 16) / d);
                o[w] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4 *>(yb + e) = o;
        }
    } else {
        for (int64_t e = e0 + threadIdx.x; e < e1; e += kNormThreads)
            yb[e] = f32_to_bf16_bits(bf16_bits_to_f32(xb[e]) / d);
    }
}

}  // namespace

int64_t norm_chunks(int64_t mn) { return (mn + kNormChunk - 1) / kNormChunk; }

hipError_t launch_normalize(const uint16_t *x, uint16_t *y, float *partial, int64_t batch,
                            int64_t mn, bool vec, hipStream_t stream) {
    const int64_t chunks = norm_chunks(mn);
    const int64_t grid = batch * chunks;
    if (grid <= 0 || grid >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    int ch = static_cast<int>(chunks), v = vec ? 1 : 0;
    void *a1[] = {&x, &partial, &mn, &ch, &v};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&norm_partial_kernel),
                                   dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), a1, 0,
                                   stream);
    if (e != hipSuccess) return e;
    void *a2[] = {&x, &y, &partial, &mn, &ch, &v};
    return hipLaunchKernel(reinterpret_cast<const void *>(&norm_scale_kernel),
                           dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), a2, 0, stream);
}

}  // namespace muon_polar
