/*
 * muon_polar.h — C ABI of the MI355X (gfx950) Polar Express step.
 *
 * One Polar Express (Newton-Schulz) iteration of the Muon optimizer:
 *
 *     A = X·Xᵀ          (stage 1, "gram":  symmetric SYRK, upper tiles + mirror)
 *     P = b·A + c·A·A   (stage 2, "poly":  A·A with the polynomial in the epilogue)
 *     Y = a·X + P·X     (stage 3, "apply": P·X with the a·X add in the epilogue)
 *
 * X and Y are row-major contiguous bf16 tensors of shape [batch, m, n].  For
 * m > n, muon_polar_step and muon_polar_express run the right-Gram form
 *
 *     G = Xᵀ·X,   P = b·G + c·G²,   Y = a·X + X·P
 *
 * (the step of the transposed input, transposed back, without the copies; it
 * needs n % 8 == 0 and 16-byte aligned x and y, and A below is then G).  A and
 * P live in a caller-provided scratch ("workspace") of shape [batch,
 * padded_rows, padded_rows] each, where padded_rows >= min(m, n) is the larger
 * of the gram and poly stages' tile extents, reported by muon_polar_query().  The
 * padding rows and columns of A and P are written as exact zeros by the kernels,
 * so no caller memset is needed.
 *
 * Stream-K: when the last round of a stage's output tiles would leave most CUs
 * idle, the K loops of those tiles are cut into equal shares, one per
 * workgroup, and the last contributor of a tile sums the fp32 partials in a
 * fixed order (results are the same on every run of one device type, and equal
 * the unsplit ones to fp32 rounding).  The arrival counters and partial tiles
 * live in the workspace after A and P.  Each counter word carries the token of
 * the launch that wrote it, and words of other launches count as zero, so the
 * workspace needs no clearing (any content, graph replays included).  Calls that
 * share one workspace must not overlap (use one workspace per concurrent stream).
 * Stage 3 with 256x256 tiles instead runs such a last round, when it holds
 * between a quarter and a half of the resident workgroups, as 256x128 column
 * halves in the same launch (whole K each; no partials, no counters).  Results
 * of the 192x192 tiles with 8 waves and of those halves sum each output's K
 * terms in two interleaved chains (wave pairs): they equal the one-chain kernels
 * to fp32 rounding.
 *
 * Widths: the DMA-fed kernels read X in place when its rows are n % 8 == 0
 * elements from a 16-byte aligned X, or an even n from a 4-byte aligned X (16-byte
 * global->LDS transfers at 4-byte aligned addresses); the chunks of a last K-step
 * past n are masked to zeros (the same sums as a zero-padded X, bit for bit).
 * Otherwise (odd n, or X not 4-byte aligned) each step first copies X into a
 * zero-padded [batch, m, roundup(n, 64)] buffer at the end of the workspace, which
 * info.workspace_bytes includes for every n % 8 != 0.  Y is written at its own
 * width: 16-byte stores when n % 8 == 0 and y is 16-byte aligned; otherwise, with a
 * 4-byte aligned y, 16-byte stores for the 8-element chunks inside each row that starts
 * on a 4-byte boundary (every row for even n, every other row for odd n) and 2-byte
 * stores for the rest; 2-byte stores throughout when y is only 2-byte aligned.
 * Shapes whose padded copy would reach
 * 2^30 elements per matrix are rejected ("matrix too large"), like X itself.
 *
 * Buffers: x, y and the workspace must be pairwise disjoint (no in-place call:
 * every output tile of stage 3 reads X's whole K range while other tiles are
 * written to Y).
 *
 * All functions are asynchronous on the given HIP stream (launch only, no
 * synchronisation) unless MUON_POLAR_DEBUG_SYNC is set in the environment, in
 * which case every stage synchronises the stream and reports kernel faults.
 * Pointers are device pointers.  No function allocates device memory.
 *
 * Numerics: fp32 accumulation on bf16 MFMA; A and P stored as bf16 (RNE of the
 * fp32 result, P = bf16(b·A + c·(A·A)_fp32) with b, c in fp32); Y = bf16(a·X +
 * (P·X)_fp32) with one rounding and a kept in fp32.
 *
 * Return value: MUON_POLAR_OK (0) or a negative status code; the thread-local
 * message from muon_polar_last_error() gives the detail.
 */
#ifndef MUON_POLAR_H_
#define MUON_POLAR_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum muon_polar_status {
    MUON_POLAR_OK = 0,
    MUON_POLAR_ERR_INVALID_ARGUMENT = -1, /* bad shape, null pointer, m > n, ... */
    MUON_POLAR_ERR_WORKSPACE = -2,        /* workspace missing or too small */
    MUON_POLAR_ERR_HIP = -3,              /* a HIP runtime call or a launch failed */
    MUON_POLAR_ERR_CONFIG = -4            /* an MUON_POLAR_* tuning variable is out of range */
};

/* Sizes of the scratch buffers for one call.
 * Replaces the host-side tiling/launch-state builders of the reference
 * (csrc/muon_polar_step_binding.cpp:266-611): the launch configuration is
 * chosen and cached inside the library; the caller only needs the sizes. */
typedef struct muon_polar_shape_info {
    int64_t padded_rows;    /* extent and leading dimension of A and P (>= m) */
    size_t gram_bytes;      /* bytes of one [batch, padded_rows, padded_rows] bf16 buffer */
    size_t workspace_bytes; /* bytes for A and P (each 256-byte aligned) and the stream-K area */
    size_t express_workspace_bytes; /* muon_polar_express: the above, one [batch, m, n] bf16
                                       buffer and the normalisation partial sums */
    size_t muon_workspace_bytes;    /* muon_polar_muon_update: the above and one more
                                       [batch, m, n] bf16 buffer */
} muon_polar_shape_info;

int muon_polar_query(int64_t batch, int64_t m, int64_t n, muon_polar_shape_info *info);

/* Whole step: Y = a·X + (b·A + c·A²)·X with A = X·Xᵀ, three kernels in order
 * on `stream` (m > n: the right-Gram form above).  `workspace` must hold
 * info.workspace_bytes.
 * Replaces MuonPolarStepAscend950 (csrc/muon_polar_step_binding.cpp:613-673)
 * without its pad/crop copies: edges are masked in the kernels.  The reference
 * rejects m > n there (binding.cpp:622-624) and transposes in its Python
 * wrapper (muon_ascend950/ops.py:26-32). */
int muon_polar_step(const void *x, void *y, void *workspace, size_t workspace_bytes,
                    int64_t batch, int64_t m, int64_t n,
                    double a, double b, double c, hipStream_t stream);

/* muon_polar_step without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.
 * The workspace is a device array of 192 MiB (201326592 bytes) inside the
 * library, one per GPU, held from the first call on that GPU until the process
 * ends.  Where the step's plan needs a larger workspace (info.workspace_bytes)
 * only for the partial slots of its two-round stream-K split, the plan without
 * that split runs (MUON_POLAR_SK_ROUNDS=0, e.g. [2, 4096, 4096]); shapes that do
 * not fit even so are rejected with MUON_POLAR_ERR_WORKSPACE (e.g.
 * [4, 4096, 4096]; [4096, 14336] fits).  Results equal muon_polar_step's bit for
 * bit under the same plan.  No device memory is allocated
 * and no caller buffer is needed beyond x and y.  Calls that overlap on one GPU
 * (other streams, other threads) share the array and race: serialise them. */
int muon_polar_step_noalloc(const void *x, void *y, int64_t batch, int64_t m, int64_t n,
                            double a, double b, double c, hipStream_t stream);

/* The three stages one at a time.  `workspace` is NULL (workspace_bytes
 * ignored: the stage runs one output tile per workgroup) or a buffer of
 * info.workspace_bytes, the same one muon_polar_step takes (gram / poly may be
 * its A / P areas), which lets the stage use the stream-K split (and, where the
 * step takes it, the padded copy of X) exactly as inside muon_polar_step, so the
 * three calls reproduce the step bit for bit.  The reference's stage launchers
 * likewise take a device-side buffer (their tiling struct).  The stages take
 * m <= n only.  A stage's output must not overlap its inputs (every output tile
 * reads whole rows of them while other tiles are stored), and no operand may
 * overlap the workspace past its A and P areas (the arrival words, partial
 * slots and padded copy of X the stage writes); MUON_POLAR_ERR_INVALID_ARGUMENT
 * otherwise, before any launch. */

/* Stage 1: gram[bt] = X[bt]·X[bt]ᵀ into a [batch, padded_rows, padded_rows]
 * bf16 buffer (padding written as zeros).
 * Replaces launch_muon_gram_lowlevel_fused (csrc/muon_polar_step_binding.cpp:65-66,
 * csrc/muon_polar_unified_ascend950.asc:512-517). */
int muon_polar_gram(const void *x, void *gram, void *workspace, size_t workspace_bytes,
                    int64_t batch, int64_t m, int64_t n, hipStream_t stream);

/* Stage 2: poly = b·gram + c·gram·gram over [batch, padded_rows, padded_rows];
 * gram must be symmetric (as written by stage 1).
 * Replaces launch_muon_cube2_p_fused (csrc/muon_polar_step_binding.cpp:69-70,
 * csrc/muon_polar_unified_ascend950.asc:1030-1035). */
int muon_polar_poly(const void *gram, void *poly, void *workspace, size_t workspace_bytes,
                    int64_t batch, int64_t m, int64_t n, double b, double c, hipStream_t stream);

/* Stage 3: Y = a·X + poly·X; y must not overlap x or poly.
 * Replaces launch_muon_cube3_fused_lowlevel (csrc/muon_polar_step_binding.cpp:67-68,
 * csrc/muon_polar_unified_ascend950.asc:1535-1540). */
int muon_polar_apply(const void *poly, const void *x, void *y, void *workspace,
                     size_t workspace_bytes, int64_t batch, int64_t m, int64_t n, double a,
                     hipStream_t stream);

/* Several steps in one call, optionally after the per-matrix normalisation
 * X / (‖X‖_F·1.01 + 1e-6) with the rounding points of the reference recipe
 * (bf16 norm, bf16 product and sum, fp32 division rounded to bf16).
 * coefficients: `steps` triples (a, b, c), step i uses coefficients[3i..3i+2].
 * `workspace` must hold info.express_workspace_bytes; x, y and the workspace
 * must be pairwise disjoint;
 * steps >= 1, or steps == 0 with normalize (y = normalised x); m > n as for
 * muon_polar_step.
 * No reference counterpart: replaces the caller-side loop of the reference's
 * examples/five_steps.py:17-20 (normalise, then one polar_step per triple). */
int muon_polar_express(const void *x, void *y, void *workspace, size_t workspace_bytes,
                       int64_t batch, int64_t m, int64_t n, const double *coefficients,
                       int64_t steps, int normalize, hipStream_t stream);

/* Muon optimizer update of one parameter (or a batch of equally shaped ones):
 * param, grad and momentum_buffer are fp32 [batch, m, n], row-major contiguous,
 * pairwise disjoint and disjoint from the workspace.
 *
 *     buf ← lerp(buf, grad, 1 − momentum)
 *     g'  = nesterov ? lerp(grad, buf, momentum) : buf
 *     O   = muon_polar_express(bf16(g'), coefficients, steps, normalize = 1)
 *     param ← param·(1 − lr·weight_decay) − (lr·lr_scale)·O
 *
 * lerp is torch.lerp's two-branch form (start + w·(end − start) for |w| < 0.5,
 * else end − (end − start)·(1 − w)), every fp32 operation rounded on its own;
 * the scalars are rounded to fp32 as (float)(1 − momentum), (float)momentum,
 * (float)(1 − lr·weight_decay) and (float)(−lr·lr_scale).  lr_scale is the
 * caller's shape factor (nanochat's Muon: sqrt(max(1, rows / cols)) of the
 * parameter).  m > n needs n % 8 == 0 (right-Gram form).  `workspace` must hold
 * info.muon_workspace_bytes.  grad is read only; buf and param are updated in
 * place.
 * No reference counterpart: the reference provides the orthogonalisation only
 * and leaves momentum, weight decay and the parameter update to its caller
 * (README.md:130; the caller is nanochat's Muon optimizer, README.md:247). */
int muon_polar_muon_update(void *param, const void *grad, void *momentum_buffer,
                           void *workspace, size_t workspace_bytes, int64_t batch, int64_t m,
                           int64_t n, double momentum, int nesterov, const double *coefficients,
                           int64_t steps, double lr, double weight_decay, double lr_scale,
                           hipStream_t stream);

/* Host-side check of a launch plan (test support; no reference counterpart).
 * Builds the plan muon_polar_step would use for [batch, m, n] on a device of
 * `cus` compute units with blocks_per_cu[s] resident workgroups per CU for the
 * DMA-fed kernel of stage s (0 gram, 1 poly, 2 apply; the occupancy the device
 * reports), with the tuning variables of the environment, and walks every
 * workgroup of each stage with the kernels' own schedule functions.  It reports
 * the byte ranges each stage can store to, relative to the buffer each range
 * belongs to, next to those buffers' sizes.  No device is touched. */
typedef struct muon_polar_stage_extent {
    int32_t tile_m, tile_n, waves, depth;
    int32_t dma_fed;       /* 1: DMA-fed kernel; 0: register-staged */
    int32_t k_steps, total_tiles, dp_tiles, sk_units, grid;
    int32_t coverage_ok;   /* every (tile, K-step) iteration computed by exactly one workgroup
                              (a tile run as two column halves: once per half) */
    int32_t extents_ok;    /* per-matrix operand byte extents < 2^31 and passed unchanged */
    int32_t halves;        /* 1: tiles past dp_tiles run as sk_units column halves, each over
                              the whole K range (no partial slots, no arrival words) */
    int32_t diag_pairs;    /* 1 (gram, poly): the units are the off-diagonal tiles and pairs of
                              diagonal tiles (two 64x64 tiles per workgroup, never cut) */
    int64_t out_lo, out_hi, out_limit;          /* output stores, bytes: [lo, hi) vs buffer size */
    int64_t partial_lo, partial_hi, partial_limit; /* stream-K partial slots, bytes */
    int64_t counter_hi, counter_limit;          /* stream-K arrival words used vs reserved */
} muon_polar_stage_extent;

typedef struct muon_polar_plan_extents {
    int64_t workspace_bytes;  /* the step's workspace size */
    int64_t gram_bytes;       /* A at offset 0 and P at poly_offset, each this size */
    int64_t poly_offset;
    int64_t counters_offset;  /* 3 stages x counter_stride 64-bit arrival words */
    int64_t counter_stride;
    int64_t partials_offset;  /* partial slots up to pad_offset */
    int64_t pad_offset;       /* padded copy of X, written up to pad_end (0: none) */
    int64_t pad_end;
    int64_t y_bytes;          /* size of Y, the apply stage's output */
    muon_polar_stage_extent stage[3];
    /* Rows that take the padded copy: the apply of a polar_express / Muon chain's
       steps before the last, which writes its iterate padded to np columns (out_limit:
       the padded buffer); all zero for other shapes. */
    muon_polar_stage_extent chain_apply;
} muon_polar_plan_extents;

int muon_polar_check_plan(int64_t batch, int64_t m, int64_t n, int cus, const int *blocks_per_cu,
                          muon_polar_plan_extents *out);

/* Detail of the last failure on the calling thread ("" if none).
 * Replaces CheckAcl / aclGetRecentErrMsg (csrc/muon_polar_step_binding.cpp:72-75). */
const char *muon_polar_last_error(void);

/* Library version string ("0.1.1" mirrors muon_ascend950/__init__.py:10). */
const char *muon_polar_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MUON_POLAR_H_ */
