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
//
// Also the two element-wise passes of the Muon update around the iteration:
// the momentum pass (fp32 momentum buffer and Nesterov blend, the bf16 input of
// the iteration and its sums of squares in the normalisation's own order) and
// the parameter update p = p·(1 − lr·wd) − lr·scale·O.
//
// And the row-padding copy that gives the DMA-fed stage kernels rows of a whole
// number of 64-element K-steps: X [rows, n] -> Xp [rows, np], np a multiple of 8
// (of 64 as used), the columns n .. np-1 zero, one 16-byte chunk of Xp per thread.
#include "polar_kernels.h"
#include "polar_tile.hpp"

namespace muon_polar {

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormStride = kNormThreads * 8;  // elements a block covers per iteration

// Iterations whose loads each thread issues before it uses the first of them (the
// vector loops below).  Every thread still takes its elements in increasing order,
// so the sums are those of one iteration at a time; what changes is the number of
// loads in flight per wave, which sets these bandwidth-bound passes' rate.
constexpr int kNormUnroll = 4;      // norm passes: 16 bytes per thread and iteration
constexpr int kMomentumUnroll = 2;  // momentum pass: 64 bytes per thread and iteration
constexpr int kParamUnroll = 2;     // parameter pass: 48 bytes per thread and iteration

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
                                                                    int64_t chunk, int vec) {
    __shared__ float red[4];
    const int b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
    const uint16_t *base = x + int64_t(b) * mn;
    const int64_t e0 = int64_t(c) * chunk;
    const int64_t e1 = e0 + chunk < mn ? e0 + chunk : mn;
    float acc = 0.0f;
    if (vec) {  // mn % 8 == 0 and 16-byte aligned rows of 8 elements
        for (int64_t e = e0 + threadIdx.x * 8; e < e1; e += kNormUnroll * kNormStride) {
            u32x4 v[kNormUnroll];
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u)
                if (e + u * kNormStride < e1)
                    v[u] = *reinterpret_cast<const u32x4 *>(base + e + u * kNormStride);
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u) {
                if (e + u * kNormStride >= e1) break;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float lo = bf16_bits_to_f32(v[u][w] & 0xffffu);
                    const float hi = bf16_bits_to_f32(v[u][w] >> 16);
                    acc = fmaf(lo, lo, acc);
                    acc = fmaf(hi, hi, acc);
                }
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
                                                                  int64_t mn, int chunks,
                                                                  int64_t chunk, int vec) {
    __shared__ float red[4];
    const int b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
    float s = 0.0f;
    for (int i = threadIdx.x; i < chunks; i += kNormThreads) s += partial[int64_t(b) * chunks + i];
    const float total = block_sum(s, red);
    const float norm = bf16_round(sqrtf(total));
    const float d = bf16_round(bf16_round(norm * 1.01f) + 1e-6f);

    const uint16_t *xb = x + int64_t(b) * mn;
    uint16_t *yb = y + int64_t(b) * mn;
    const int64_t e0 = int64_t(c) * chunk;
    const int64_t e1 = e0 + chunk < mn ? e0 + chunk : mn;
    if (vec) {
        const __amdgpu_buffer_rsrc_t rs_y = store_rsrc(yb + e0);
        for (int64_t e = e0 + threadIdx.x * 8; e < e1; e += kNormUnroll * kNormStride) {
            u32x4 v[kNormUnroll];
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u)
                if (e + u * kNormStride < e1)
                    v[u] = *reinterpret_cast<const u32x4 *>(xb + e + u * kNormStride);
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u) {
                if (e + u * kNormStride >= e1) break;
                u32x4 o;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t lo = f32_to_bf16_bits(bf16_bits_to_f32(v[u][w] & 0xffffu) / d);
                    const uint32_t hi = f32_to_bf16_bits(bf16_bits_to_f32(v[u][w] >> 16) / d);
                    o[w] = lo | (hi << 16);
                }
                store16_sc1(rs_y, static_cast<uint32_t>((e + u * kNormStride - e0) * 2), o);
            }
        }
    } else {
        for (int64_t e = e0 + threadIdx.x; e < e1; e += kNormThreads)
            yb[e] = f32_to_bf16_bits(bf16_bits_to_f32(xb[e]) / d);
    }
}

// torch.lerp's two-branch form (ATen Lerp.h): start + w·(end − start) for |w| < 0.5,
// else end − (end − start)·(1 − w); every operation rounded on its own.
__device__ __forceinline__ float lerp_rounded(float start, float end, float w) {
#pragma clang fp contract(off)
    return fabsf(w) < 0.5f ? start + w * (end - start) : end - (end - start) * (1.0f - w);
}

// Momentum pass of the Muon update over chunk c of matrix b (chunks as in
// norm_partial_kernel):
//     buf ← lerp(buf, g, w)                  (w = 1 − momentum)
//     g'  = lerp(g, buf, momentum) | buf     (Nesterov or plain)
//     x0  = bf16(g'),   partial[b, c] = Σ x0²  in norm_partial_kernel's order
// order8: mn % 8 == 0 (8 consecutive elements per thread and step, the vector
// path's order); vec: also 16-byte aligned g, buf and x0 (vector accesses).
template <bool kOrder8, bool kVec>
__global__ __launch_bounds__(kNormThreads) void muon_momentum_kernel(
    const float *__restrict__ g, float *__restrict__ buf, uint16_t *__restrict__ x0,
    float *__restrict__ partial, int64_t mn, int chunks, int64_t chunk, float w, float beta,
    int nesterov) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const int b = blockIdx.x / chunks, c = blockIdx.x - b * chunks;
    const int64_t base = int64_t(b) * mn;
    const int64_t e0 = int64_t(c) * chunk;
    const int64_t e1 = e0 + chunk < mn ? e0 + chunk : mn;
    float acc = 0.0f;
    auto one = [&](float gv, float bv, uint32_t &h) {
        const float nb = lerp_rounded(bv, gv, w);
        const float u = nesterov ? lerp_rounded(gv, nb, beta) : nb;
        h = f32_to_bf16_bits(u);
        const float r = bf16_bits_to_f32(h);
        acc = fmaf(r, r, acc);
        return nb;
    };
    if (kOrder8) {
        constexpr int kU = kVec ? kMomentumUnroll : 1;
        const __amdgpu_buffer_rsrc_t rs_x0 = store_rsrc(x0 + base + e0);
        for (int64_t e = e0 + threadIdx.x * 8; e < e1; e += kU * kNormStride) {
            float gv[kU][8], bv[kU][8];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t eu = e + u * kNormStride;
                if (eu >= e1) break;
                if (kVec) {
                    const f32x4 g0 = *reinterpret_cast<const f32x4 *>(g + base + eu);
                    const f32x4 g1 = *reinterpret_cast<const f32x4 *>(g + base + eu + 4);
                    const f32x4 b0 = *reinterpret_cast<const f32x4 *>(buf + base + eu);
                    const f32x4 b1 = *reinterpret_cast<const f32x4 *>(buf + base + eu + 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        gv[u][i] = g0[i]; gv[u][i + 4] = g1[i];
                        bv[u][i] = b0[i]; bv[u][i + 4] = b1[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        gv[u][i] = g[base + eu + i];
                        bv[u][i] = buf[base + eu + i];
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t eu = e + u * kNormStride;
                if (eu >= e1) break;
                float nb[8];
                uint32_t h[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) nb[i] = one(gv[u][i], bv[u][i], h[i]);
                if (kVec) {
                    *reinterpret_cast<f32x4 *>(buf + base + eu) = f32x4{nb[0], nb[1], nb[2], nb[3]};
                    *reinterpret_cast<f32x4 *>(buf + base + eu + 4) =
                        f32x4{nb[4], nb[5], nb[6], nb[7]};
                    store16_sc1(rs_x0, static_cast<uint32_t>((eu - e0) * 2),
                                u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16),
                                      h[4] | (h[5] << 16), h[6] | (h[7] << 16)});
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        buf[base + eu + i] = nb[i];
                        x0[base + eu + i] = static_cast<uint16_t>(h[i]);
                    }
                }
            }
        }
    } else {
        for (int64_t e = e0 + threadIdx.x; e < e1; e += kNormThreads) {
            uint32_t h;
            buf[base + e] = one(g[base + e], buf[base + e], h);
            x0[base + e] = static_cast<uint16_t>(h);
        }
    }
    const float t = block_sum(acc, red);
    if (threadIdx.x == 0) partial[blockIdx.x] = t;
}

// p ← p·decay + alpha·O over `total` elements (fp32 p, bf16 O; each product and
// the sum rounded on their own).
template <bool kVec>
__global__ __launch_bounds__(kNormThreads) void muon_param_update_kernel(
    float *__restrict__ p, const uint16_t *__restrict__ o, int64_t total, float decay,
    float alpha) {
#pragma clang fp contract(off)
    const int64_t stride = int64_t(gridDim.x) * kNormThreads * 8;
    if (kVec) {
        // kParamUnroll grid strides per trip, every load of the trip issued first
        for (int64_t e = (int64_t(blockIdx.x) * kNormThreads + threadIdx.x) * 8; e < total;
             e += kParamUnroll * stride) {
            u32x4 ov[kParamUnroll];
            f32x4 p0[kParamUnroll], p1[kParamUnroll];
#pragma unroll
            for (int u = 0; u < kParamUnroll; ++u) {
                const int64_t eu = e + u * stride;
                if (eu >= total) break;
                ov[u] = *reinterpret_cast<const u32x4 *>(o + eu);
                p0[u] = *reinterpret_cast<const f32x4 *>(p + eu);
                p1[u] = *reinterpret_cast<const f32x4 *>(p + eu + 4);
            }
#pragma unroll
            for (int u = 0; u < kParamUnroll; ++u) {
                const int64_t eu = e + u * stride;
                if (eu >= total) break;
                f32x4 q0 = p0[u], q1 = p1[u];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    q0[2 * i] = q0[2 * i] * decay + alpha * bf16_bits_to_f32(ov[u][i] & 0xffffu);
                    q0[2 * i + 1] = q0[2 * i + 1] * decay + alpha * bf16_bits_to_f32(ov[u][i] >> 16);
                    q1[2 * i] = q1[2 * i] * decay + alpha * bf16_bits_to_f32(ov[u][i + 2] & 0xffffu);
                    q1[2 * i + 1] =
                        q1[2 * i + 1] * decay + alpha * bf16_bits_to_f32(ov[u][i + 2] >> 16);
                }
                *reinterpret_cast<f32x4 *>(p + eu) = q0;
                *reinterpret_cast<f32x4 *>(p + eu + 4) = q1;
            }
        }
    } else {
        for (int64_t e = (int64_t(blockIdx.x) * kNormThreads + threadIdx.x) * 8; e < total;
             e += stride) {
            const int64_t end = e + 8 < total ? e + 8 : total;
            for (int64_t i = e; i < end; ++i) p[i] = p[i] * decay + alpha * bf16_bits_to_f32(o[i]);
        }
    }
}

__global__ __launch_bounds__(kNormThreads) void pad_rows_kernel(const uint16_t *__restrict__ x,
                                                                uint16_t *__restrict__ xp,
                                                                int64_t chunks, int32_t n,
                                                                int32_t row_chunks, int32_t vec) {
    // row_chunks = np / 8: chunks per padded row; vec: 16-byte loads of whole
    // chunks (n % 8 == 0 and x 16-byte aligned)
    const int64_t stride = int64_t(gridDim.x) * kNormThreads;
    for (int64_t q0 = int64_t(blockIdx.x) * kNormThreads; q0 < chunks; q0 += stride) {
        const int64_t q = q0 + threadIdx.x;
        if (q >= chunks) break;
        const __amdgpu_buffer_rsrc_t rs = store_rsrc(xp + q0 * 8);  // this block's chunks
        const int64_t r = q / row_chunks;
        const int c0 = static_cast<int>(q - r * row_chunks) * 8;
        const uint16_t *src = x + r * n + c0;
        u32x4 v;
        if (vec && c0 + 8 <= n) {
            v = *reinterpret_cast<const u32x4 *>(src);
        } else {
            uint32_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = c0 + e < n ? uint32_t(src[e]) : 0u;
            v = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                      h[6] | (h[7] << 16)};
        }
        store16_sc1(rs, static_cast<uint32_t>(threadIdx.x) * 16u, v);
    }
}

}  // namespace

hipError_t launch_pad_rows(const uint16_t *x, uint16_t *xp, int64_t rows, int64_t n, int64_t np,
                           hipStream_t stream) {
    if (rows <= 0 || n <= 0 || np < n || np % 8 != 0 || np >= (int64_t(1) << 30))
        return hipErrorInvalidValue;
    int32_t row_chunks = static_cast<int32_t>(np / 8), nn = static_cast<int32_t>(n);
    int64_t chunks = rows * row_chunks;
    int32_t vec = (n % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0) ? 1 : 0;
    const int64_t blocks = (chunks + kNormThreads - 1) / kNormThreads;
    const unsigned grid = static_cast<unsigned>(blocks < 8192 ? blocks : 8192);
    void *args[] = {&x, &xp, &chunks, &nn, &row_chunks, &vec};
    return hipLaunchKernel(reinterpret_cast<const void *>(&pad_rows_kernel), dim3(grid),
                           dim3(kNormThreads), args, 0, stream);
}

// Smaller chunks give more blocks to the passes of a small matrix; every block of
// the scale pass re-sums all of its matrix's partials, so the chunk is the smallest
// power of two from 4096 for which batch · chunks² stays within 2^24 partial loads.
// Measured (the Muon update's element-wise passes / the normalisation):
// [1,4096,14336] 330 / 61 us with 65536-element chunks, 314 / 60 with 16384, 319 / 74
// with 8192; [12,768,768] 53 / 19 us with 65536, 35 / 10 with 4096.
int64_t norm_chunk(int64_t batch, int64_t mn) {
    constexpr int64_t kMin = 4096, kMax = int64_t(1) << 20, kBudget = int64_t(1) << 24;
    int64_t chunk = kMin;
    while (chunk < kMax) {
        const int64_t c = (mn + chunk - 1) / chunk;
        if (c <= kBudget / c / (batch > 0 ? batch : 1)) break;
        chunk *= 2;
    }
    return chunk;
}

int64_t norm_chunks(int64_t batch, int64_t mn) {
    const int64_t chunk = norm_chunk(batch, mn);
    return (mn + chunk - 1) / chunk;
}

hipError_t launch_norm_scale(const uint16_t *x, uint16_t *y, const float *partial,
                             int64_t batch, int64_t mn, bool vec, hipStream_t stream) {
    int64_t chunk = norm_chunk(batch, mn);
    const int64_t chunks = norm_chunks(batch, mn);
    const int64_t grid = batch * chunks;
    if (grid <= 0 || grid >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    int ch = static_cast<int>(chunks), v = vec ? 1 : 0;
    void *a2[] = {&x, &y, &partial, &mn, &ch, &chunk, &v};
    return hipLaunchKernel(reinterpret_cast<const void *>(&norm_scale_kernel),
                           dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), a2, 0, stream);
}

hipError_t launch_muon_momentum(const float *g, float *buf, uint16_t *x0, float *partial,
                                int64_t batch, int64_t mn, float w, float beta, bool nesterov,
                                bool vec, hipStream_t stream) {
    int64_t chunk = norm_chunk(batch, mn);
    const int64_t chunks = norm_chunks(batch, mn);
    const int64_t grid = batch * chunks;
    if (grid <= 0 || grid >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    int ch = static_cast<int>(chunks), nv = nesterov ? 1 : 0;
    void *args[] = {&g, &buf, &x0, &partial, &mn, &ch, &chunk, &w, &beta, &nv};
    const bool order8 = mn % 8 == 0;
    const void *fn = order8 ? (vec ? reinterpret_cast<const void *>(&muon_momentum_kernel<true, true>)
                                   : reinterpret_cast<const void *>(&muon_momentum_kernel<true, false>))
                            : reinterpret_cast<const void *>(&muon_momentum_kernel<false, false>);
    return hipLaunchKernel(fn, dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), args, 0,
                           stream);
}

hipError_t launch_muon_param_update(float *p, const uint16_t *o, int64_t total, float decay,
                                    float alpha, bool vec, hipStream_t stream) {
    if (total <= 0) return hipErrorInvalidValue;
    // 8 elements per thread; at most 8 waves' worth of blocks per CU on 256 CUs,
    // a grid-stride loop beyond that
    const int64_t blocks = (total + kNormThreads * 8 - 1) / (kNormThreads * 8);
    const unsigned grid = static_cast<unsigned>(blocks < 4096 ? blocks : 4096);
    void *args[] = {&p, &o, &total, &decay, &alpha};
    const void *fn = vec ? reinterpret_cast<const void *>(&muon_param_update_kernel<true>)
                         : reinterpret_cast<const void *>(&muon_param_update_kernel<false>);
    return hipLaunchKernel(fn, dim3(grid), dim3(kNormThreads), args, 0, stream);
}

hipError_t launch_normalize(const uint16_t *x, uint16_t *y, float *partial, int64_t batch,
                            int64_t mn, bool vec, hipStream_t stream) {
    int64_t chunk = norm_chunk(batch, mn);
    const int64_t chunks = norm_chunks(batch, mn);
    const int64_t grid = batch * chunks;
    if (grid <= 0 || grid >= (int64_t(1) << 31)) return hipErrorInvalidValue;
    int ch = static_cast<int>(chunks), v = vec ? 1 : 0;
    void *a1[] = {&x, &partial, &mn, &ch, &chunk, &v};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&norm_partial_kernel),
                                   dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), a1, 0,
                                   stream);
    if (e != hipSuccess) return e;
    void *a2[] = {&x, &y, &partial, &mn, &ch, &chunk, &v};
    return hipLaunchKernel(reinterpret_cast<const void *>(&norm_scale_kernel),
                           dim3(static_cast<unsigned>(grid)), dim3(kNormThreads), a2, 0, stream);
}

}  // namespace muon_polar
