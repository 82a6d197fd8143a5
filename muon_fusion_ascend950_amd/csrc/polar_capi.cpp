// polar_capi.cpp — C ABI (include/muon_polar.h) over the gfx950 stage kernels,
// with the launch-configuration cache.
//
// Reference counterpart: csrc/muon_polar_step_binding.cpp.  The reference builds
// a CANN tiling struct per stage, copies it to device memory once per cache key
// (binding.cpp:266-611) and keys three mutex-guarded maps by (device, stream,
// shape, tuning knobs, coefficient bits).  Here a launch configuration is a small
// host struct passed to the kernels by value, so one map keyed by (device, shape,
// tuning knobs) suffices; coefficients are kernel arguments, not key material,
// and the stream is not part of the key because nothing device-side is cached.
#include "muon_polar.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <climits>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <numeric>
#include <string>
#include <unordered_map>
#include <vector>

#include "polar_kernels.h"
#include "polar_schedule.hpp"

namespace {

using muon_polar::GemmArgs;
using muon_polar::Stage;

thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

// Same parsing rule as the reference's EnvU64 (binding.cpp:77-86): unset or
// empty -> default; otherwise the leading decimal digits, or the default when
// there are none.
uint64_t env_u64(const char *name, uint64_t def, bool *present = nullptr) {
    const char *v = std::getenv(name);
    if (present) *present = (v != nullptr && v[0] != '\0');
    if (v == nullptr || v[0] == '\0') return def;
    char *end = nullptr;
    const unsigned long long parsed = std::strtoull(v, &end, 10);
    return end != v ? static_cast<uint64_t>(parsed) : def;
}

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
size_t align256(size_t v) { return (v + 255u) & ~size_t(255u); }

struct Knobs {
    uint32_t gram_tile, poly_tile, apply_bm, apply_bn;
    uint32_t stream;    // 1: DMA-fed kernels where eligible; 0: register-staged kernels only
    uint32_t stream_k;  // stream-K split of a partial last round (polar_step only), per stage:
                        // bit 0 gram, bit 1 poly, bit 2 apply (0: off everywhere)
    uint32_t waves;     // waves per workgroup of the 256x256 DMA-fed kernels (4 or 8)
    uint32_t depth[3];  // LDS ring slots of each stage's DMA-fed kernel (0: by shape)
    uint32_t pair;      // 1: 192x192 tiles run the 8-wave wave-pair kernels when waves == 8
    uint32_t halves;    // 1: apply's last round as 256x128 halves where it fits (below)
    uint32_t halves_depth;  // LDS ring slots of those halves (2 or 3)
    uint32_t diag_pairs;    // 1: triangular stages pair their diagonal tiles where it
                            // takes fewer rounds of workgroups (below)
    uint32_t sk_rounds;     // per stage (bit 0 gram, bit 1 poly, bit 2 apply): a stream-K
                            // split of 256x256 tiles with a short last round also takes
                            // the whole round before it (sk_policy)
    uint32_t sk_share;      // minimum K-steps per stream-K share (0: by tile size, sk_min_share)
    uint32_t sk_pieces;     // most stream-K pieces per cut tile (0: by tile size, sk_max_pieces)
    uint32_t y_cpol, ap_cpol;  // cache policy of the DMA-fed kernels' Y / A and P stores
                               // (GemmArgs::out_cpol)
    bool operator==(const Knobs &o) const {
        return gram_tile == o.gram_tile && poly_tile == o.poly_tile && apply_bm == o.apply_bm &&
               apply_bn == o.apply_bn && stream == o.stream && stream_k == o.stream_k &&
               waves == o.waves && depth[0] == o.depth[0] && depth[1] == o.depth[1] &&
               depth[2] == o.depth[2] && pair == o.pair && halves == o.halves &&
               halves_depth == o.halves_depth && diag_pairs == o.diag_pairs &&
               sk_rounds == o.sk_rounds && sk_share == o.sk_share && sk_pieces == o.sk_pieces && y_cpol == o.y_cpol &&
               ap_cpol == o.ap_cpol;
    }
};

struct PlanKey {
    int device;
    int64_t batch, m, n;
    Knobs knobs;
    bool operator==(const PlanKey &o) const {
        return device == o.device && batch == o.batch && m == o.m && n == o.n && knobs == o.knobs;
    }
};

struct PlanKeyHash {
    size_t operator()(const PlanKey &k) const {
        uint64_t h = 1469598103934665603ull;  // FNV-1a over the key words
        auto mix = [&h](uint64_t v) {
            h ^= v;
            h *= 1099511628211ull;
        };
        mix(static_cast<uint64_t>(k.device));
        mix(static_cast<uint64_t>(k.batch));
        mix(static_cast<uint64_t>(k.m));
        mix(static_cast<uint64_t>(k.n));
        mix(k.knobs.gram_tile);
        mix(k.knobs.poly_tile);
        mix(static_cast<uint64_t>(k.knobs.apply_bm) << 32 | k.knobs.apply_bn);
        mix(k.knobs.stream);
        mix(k.knobs.stream_k);
        mix(k.knobs.waves);
        mix(uint64_t(k.knobs.depth[0]) << 16 | uint64_t(k.knobs.depth[1]) << 8 | k.knobs.depth[2]);
        mix(k.knobs.pair);
        mix(k.knobs.halves);
        mix(k.knobs.halves_depth);
        mix(k.knobs.diag_pairs);
        mix(k.knobs.sk_rounds);
        mix(uint64_t(k.knobs.sk_pieces) << 32 | uint64_t(k.knobs.sk_share) << 16 | uint64_t(k.knobs.y_cpol) << 8 | k.knobs.ap_cpol);
        return static_cast<size_t>(h);
    }
};

// Stream-K split of one stage (see GemmArgs): tiles [0, dp_tiles) one per
// workgroup, the rest cut into sk_units equal ranges of (tile, K-step) iterations.
struct SkSplit {
    int64_t dp_tiles;
    int32_t sk_units;  // stream-K units, or (halves) the number of 256x128 halves
    int64_t sk_iters;
    int32_t halves;    // apply: the last round's tiles as 256x128 column halves with
                       // this many ring slots (0: not)
};

struct Plan {
    int64_t m, n;  // X is [m, n]
    int64_t s;     // min(m, n): extent of A and P (X·Xᵀ for m <= n, Xᵀ·X for m > n)
    bool tall;     // m > n: the right-Gram stages (GramT, ApplyR)
    int64_t mp;    // padded extent / leading dimension of A and P
    int gram_tile, poly_tile, apply_bm, apply_bn;
    int gram_nt, poly_nt;           // tiles per side of the triangular stages
    int apply_tm, apply_tn;         // tiles along rows / cols of stage 3
    int64_t gram_grid, poly_grid, apply_grid;
    size_t gram_bytes, workspace_bytes;
    bool stream;
    int y_cpol, ap_cpol;  // store cache policies (GemmArgs::out_cpol)
    int waves[3];  // waves per workgroup of the DMA-fed kernel of each stage
    int depth[3];  // LDS ring slots of the DMA-fed kernel of each stage
    // polar_step's stream-K splits (gram, poly, apply) and their workspace areas
    // after A and P: arrival words (counter_stride 64-bit words per stage), then
    // the fp32 partial slots shared by the three stages.
    SkSplit sk[3];
    // gram and poly: the DMA-fed kernel runs the off-diagonal tiles and pairs of
    // diagonal tiles as its units (GemmArgs::diag_pairs; never split)
    bool diag[2];
    bool sk_any;
    int64_t counter_stride;
    size_t counters_offset, partials_offset;
    // n % 8 != 0: the workspace holds a zero-padded [batch, m, np] buffer
    // (np = roundup(n, 64)) at pad_offset.  A step whose X the DMA-fed kernels
    // cannot read in place (odd n, or X not 4-byte aligned: their panels are
    // 16-byte chunks at 4-byte aligned addresses) first copies X into it and
    // reads the copy; Y is stored at its own width (2-byte stores).  Rows of
    // n % 8 == 0 elements, and of an even n from a 4-byte aligned X, are read in
    // place, a last K-step past n masked (dma_rows).
    bool pad;
    int64_t np;
    size_t pad_offset;
    // muon_polar_express: one [batch, m, n] bf16 buffer, then the normalisation
    // partial sums, after the step's workspace
    size_t express_x_offset, express_norm_offset, express_workspace_bytes;
    size_t muon_o_offset, muon_workspace_bytes;  // muon_polar_muon_update: + O [batch, m, n] bf16
};

std::mutex g_plan_mutex;
std::unordered_map<PlanKey, Plan, PlanKeyHash> g_plans;

// Default tile shapes (measured on MI355X).  256x256 tiles run with 8 waves
// (two per SIMD: one wave's LDS and barrier waits are covered by the other's
// MFMAs).  The symmetric stages use them for large m only — gram from m = 3072
// (its K = n is long, so stream-K shares stay long), poly from m = 4096 —
// and otherwise 128x128 tiles (two workgroups per CU) when the batch has at
// least half a tile per CU of them, else 64x64 ([1, 1024, 4096]: 64x64 gram and
// poly tiles and 128x128 apply tiles take the step from 89.8 to 54.8 us; at
// m = 2048, 128x128 is 2x faster than 256x256).  Below a whole tile per CU of
// 128x128, 64x64 tiles win while they are about one round of two per CU (at
// most 2.25 per CU): [1,2048,4096] 98.6 -> 86.7 us, [4,1024,4096] 89.1 -> 80.8 us,
// [1,2048,8192] 141.7 -> 133.9 us, [16,512,512] 30.8 -> 28.9 us; beyond, 128x128
// stays faster ([2,1536,4096] 99.4 against 102.7 us, [1,2560,4096] 132.1 against
// 156.3 us, [6,1024,2048] 68.9 against 74.8 us).  Stage 3 takes the largest of
// 256x256 and 128x128 that gives every CU a tile, else 64x64.
constexpr uint32_t kDefaultWaves = 8;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

uint32_t default_sym_tile(int64_t batch, int64_t s, int64_t large_from, int cus) {
    if (s >= large_from) return 256;
    const int64_t t = ceil_div(s, 128);
    const int64_t tiles128 = batch * (t * (t + 1) / 2);
    if (tiles128 >= cus) return 128;
    if (2 * tiles128 >= cus) {
        const int64_t t64 = ceil_div(s, 64);
        return 4 * batch * (t64 * (t64 + 1) / 2) <= 9 * int64_t(cus) ? 64 : 128;
    }
    return 64;
}
// The symmetric stages' tile where 256x256 tiles would leave most CUs idle (a
// partial round cut by stream-K) and 192x192 tiles fill one round to over 3/4:
// [4096,14336] poly 91 -> 80 us per step (136 tiles of 256 against 253 of 192 on
// 256 CUs, no split, no fix-ups); gram with the wave-pair kernels (read_knobs).
// [4,4096,4096] keeps 256x256 (poly 297 against 325 us).
bool one_round_of_192(int64_t batch, int64_t s, int cus) {
    const int64_t t192 = ceil_div(s, 192), t256 = ceil_div(s, 256);
    const int64_t tiles = batch * (t192 * (t192 + 1) / 2);
    return cus > 0 && batch * (t256 * (t256 + 1) / 2) < cus && tiles <= cus && 4 * tiles > 3 * cus;
}
uint32_t default_apply_tile(int64_t batch, int64_t m, int64_t n, int cus) {
    // 256x256 from three quarters of a round when K (min(m, n)) is 1024 or more:
    // [1,3840,3840] (225 tiles) 245.6 -> 223.5 us per step against 128x128 tiles,
    // [1,5248,2904] (252) 218.4 -> 202.5, [2,1792,3584] (196) 115.4 -> 105.6,
    // [3,1024,4608] (216) 80.8 -> 75.9; [4,768,4096] (192, 12 K-steps) 61.7
    // against 63.3 us keeps 128x128
    const int64_t t256 = batch * ceil_div(m, 256) * ceil_div(n, 256);
    if (t256 >= cus || (4 * t256 >= 3 * int64_t(cus) && std::min(m, n) >= 1024)) return 256;
    // 128x128 likewise from three quarters of a round ([4,1664,424]: 208 tiles,
    // 28.1 -> 26.6 us; [1,1224,2432]: 190 tiles, 39.0 -> 37.8 us)
    if (4 * batch * ceil_div(m, 128) * ceil_div(n, 128) >= 3 * int64_t(cus)) return 128;
    return 64;
}

// Compute units of `device` (cached; 0 when it cannot be queried).
int device_cus(int device) {
    static std::atomic<int> cache[64];
    if (device < 0 || device >= 64) return 0;
    int v = cache[device].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        v <= 0)
        return 0;
    cache[device].store(v, std::memory_order_relaxed);
    return v;
}

// LDS ring depth by shape.  Four slots where they cost no parallelism: 64x64
// tiles (two workgroups per CU still fit) and 128x128 tiles when every tile has
// a CU of its own anyway (poly at [2, 2048, 8192]: 288 -> 270 us per step).
// Otherwise two: deeper rings lower the occupancy of the MFMA-bound shapes.
int default_depth(int bm, int bn, int waves, int64_t tiles, int cus) {
    if (bm == 64 && bn == 64) return 4;
    if (bm == 128 && bn == 128 && cus > 0 && tiles <= cus) return 4;
    // 192x192 wave pairs: a third 48 KiB slot ([4096,14336] gram 225 -> 212 us,
    // poly 75 -> 72 us; the LDS holds it, one workgroup per CU either way)
    if (bm == 192 && bn == 192 && waves == 8) return 3;
    return 2;
}

// X is [batch, m, n]; s = min(m, n) is the extent of A and P.
int read_knobs(int64_t batch, int64_t m, int64_t n, int cus, Knobs &k) {
    const int64_t s = std::min(m, n);
    k.waves = static_cast<uint32_t>(env_u64("MUON_POLAR_WAVES", kDefaultWaves));
    if (k.waves != 4 && k.waves != 8)
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_WAVES must be 4 or 8");
    k.pair = static_cast<uint32_t>(env_u64("MUON_POLAR_PAIR", 1));
    if (k.pair > 1) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_PAIR must be 0 or 1");
    k.halves = static_cast<uint32_t>(env_u64("MUON_POLAR_APPLY_HALVES", 1));
    if (k.halves > 2) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_APPLY_HALVES must be 0, 1 or 2");
    // three 48 KiB slots for the halves: [4096,14336] apply 395 -> 390 us
    k.halves_depth = static_cast<uint32_t>(env_u64("MUON_POLAR_HALVES_DEPTH", 3));
    k.diag_pairs = static_cast<uint32_t>(env_u64("MUON_POLAR_DIAG_PAIRS", 1));
    if (k.diag_pairs > 1) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_DIAG_PAIRS must be 0 or 1");
    k.sk_rounds = static_cast<uint32_t>(env_u64("MUON_POLAR_SK_ROUNDS", 7));
    if (k.sk_rounds > 7)
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_SK_ROUNDS must be a stage mask (0-7)");
    // Cache policy of the output stores: device-scope (sc1) stores of A, P and Y
    // leave no dirty lines in the XCD's L2 for the end-of-kernel write-back, and
    // the next kernel (poly, apply, the next step's gram) reads them from the
    // memory-side cache.  Interleaved A/B against the previous policy (Y
    // non-temporal, A and P plain), all results bit-identical: five-step chains
    // [8,512,2048] 37.7 -> 34.6 us per step, [1,1024,4096] 42.8 -> 38.7, [8,2048,512]
    // 37.9 -> 34.3, [2,2048,8192] 249.9 -> 244.1; single steps [8,512,2048] 34.7 ->
    // 34.2, [4096,14336] 671.7 -> 664.6 and 694.0 -> 690.9 (two boxes), [14336,4096]
    // 678.6 -> 672.5; [4,4096,4096] unchanged.
    k.sk_share = static_cast<uint32_t>(env_u64("MUON_POLAR_SK_MIN_SHARE", 0));
    if (k.sk_share > 4096) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_SK_MIN_SHARE must be 0..4096");
    k.sk_pieces = static_cast<uint32_t>(env_u64("MUON_POLAR_SK_PIECES", 0));
    if (k.sk_pieces == 1 || k.sk_pieces > 16)
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_SK_PIECES must be 0 (by tile) or 2..16");
    k.y_cpol = static_cast<uint32_t>(env_u64("MUON_POLAR_Y_CPOL", 2));
    k.ap_cpol = static_cast<uint32_t>(env_u64("MUON_POLAR_AP_CPOL", 2));
    if (k.y_cpol > 4 || k.ap_cpol > 4)
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_Y_CPOL / _AP_CPOL must be 0..4");
    if (k.halves_depth != 2 && k.halves_depth != 3)
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_HALVES_DEPTH must be 2 or 3");
    // Gram takes 192x192 tiles where poly does (one round of them fills the CUs,
    // below) when they run the wave-pair kernels: [4096,14336] gram 234.4 -> 226.9
    // us (253 unsplit tiles against 136 tiles of 256x256 cut by stream-K; 4-wave
    // 192x192 tiles: 237.1 us).  Both forms (X rows or X columns as its K).
    uint32_t gram_tile = default_sym_tile(batch, s, 3072, cus);
    // A long K (80 K-steps or more) pays for 256x256 gram tiles from s = 1281 when
    // they number a quarter of the CUs or more: [6,1800,6000] 470.5 -> 450.1 us,
    // [4,5248,2176] 372.4 -> 357.6 us, [3,2560,8192] 537.0 -> 508.4 us,
    // [2,2048,8192] 245.4 -> 234.9 us, [1,3000,6000] 253.0 -> 239.4 us; with fewer
    // tiles ([1,2048,8192]: 36) 128x128 and 64x64 stay 15-25% faster, as at 64
    // K-steps ([16,1024,4096], [8,1600,4096]).
    {
        const int64_t t256 = ceil_div(s, 256);
        if (gram_tile != 256 && s > 1280 && ceil_div(std::max(m, n), 64) >= 80 &&
            4 * batch * (t256 * (t256 + 1) / 2) >= cus)
            gram_tile = 256;
        // 64x64 gram tiles that outnumber the CUs (even as diagonal pairs) leave
        // two long tiles on some CUs at 128 K-steps or more, where 128x128 tiles cut
        // by stream-K share K evenly: [1,12352,1536] 183.6 -> 154.8 us per step
        const int64_t t64 = ceil_div(s, 64);
        if (gram_tile == 64 && ceil_div(std::max(m, n), 64) >= 128 &&
            batch * (t64 * (t64 - 1) / 2 + (t64 + 1) / 2) > cus)
            gram_tile = 128;
    }
    if (gram_tile == 256 && k.waves == 8 && k.pair == 1 && one_round_of_192(batch, s, cus))
        gram_tile = 192;
    k.gram_tile = static_cast<uint32_t>(env_u64("MUON_POLAR_GRAM_TILE", gram_tile));
    // an explicit gram tile also sets the poly tile unless that is given too
    const bool gram_set = std::getenv("MUON_POLAR_GRAM_TILE") != nullptr;
    uint32_t poly_tile = default_sym_tile(batch, s, 4096, cus);
    if (poly_tile == 256 && one_round_of_192(batch, s, cus)) poly_tile = 192;
    k.poly_tile = static_cast<uint32_t>(
        env_u64("MUON_POLAR_POLY_TILE", gram_set ? k.gram_tile : poly_tile));
    k.apply_bm = static_cast<uint32_t>(
        env_u64("MUON_POLAR_APPLY_TILE_M", default_apply_tile(batch, m, n, cus)));
    k.apply_bn = static_cast<uint32_t>(env_u64("MUON_POLAR_APPLY_TILE_N", k.apply_bm));
    k.stream = static_cast<uint32_t>(env_u64("MUON_POLAR_STREAM", 1));
    if (k.stream > 1) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_STREAM must be 0 or 1");
    // MUON_POLAR_STREAM_K: 0 off, 1 on (every stage); MUON_POLAR_STREAM_K_STAGES
    // narrows it to a stage mask (bit 0 gram, bit 1 poly, bit 2 apply).
    k.stream_k = static_cast<uint32_t>(env_u64("MUON_POLAR_STREAM_K", 1));
    if (k.stream_k > 1) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_STREAM_K must be 0 or 1");
    const uint64_t sk_stages = env_u64("MUON_POLAR_STREAM_K_STAGES", 7);
    if (sk_stages > 7) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_STREAM_K_STAGES must be 0..7");
    k.stream_k *= static_cast<uint32_t>(sk_stages);
    k.depth[0] = static_cast<uint32_t>(env_u64("MUON_POLAR_GRAM_DEPTH", 0));
    k.depth[1] = static_cast<uint32_t>(env_u64("MUON_POLAR_POLY_DEPTH", 0));
    k.depth[2] = static_cast<uint32_t>(env_u64("MUON_POLAR_APPLY_DEPTH", 0));
    for (uint32_t d : k.depth)
        if (d > 8) return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_*_DEPTH must be 0 (auto) or 2..8");
    if (!muon_polar::tile_supported(Stage::Gram, k.gram_tile, k.gram_tile))
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_GRAM_TILE must be 64, 128, 192 or 256");
    if (!muon_polar::tile_supported(Stage::Poly, k.poly_tile, k.poly_tile))
        return fail(MUON_POLAR_ERR_CONFIG, "MUON_POLAR_POLY_TILE must be 64, 128, 192 or 256");
    if (!muon_polar::tile_supported(Stage::Apply, k.apply_bm, k.apply_bn))
        return fail(MUON_POLAR_ERR_CONFIG,
                    "MUON_POLAR_APPLY_TILE_M/_N must be 64x64, 128x128, 256x256, 128x256 or "
                    "256x128");
    return MUON_POLAR_OK;
}

int check_shape(int64_t batch, int64_t m, int64_t n) {
    if (batch <= 0 || m <= 0 || n <= 0)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "all dimensions must be positive");
    // 32-bit byte offsets inside one matrix (X and the padded A/P): < 2^31 bytes.
    const int64_t s = std::min(m, n);
    if (m * n >= (int64_t(1) << 30) || round_up(s, 256) * round_up(s, 256) >= (int64_t(1) << 30))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "matrix too large (2^30 elements or more)");
    if (batch > (int64_t(1) << 20))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "batch too large");
    return MUON_POLAR_OK;
}

// Stream-K for the last round of a stage when it is well under full: with
// `resident` workgroups in flight, T tiles take ceil(T / resident) rounds one
// tile per workgroup.  The rem = T % resident tiles of the last round are cut
// into about `pieces` shares of K-steps each (at most sk_max_pieces, and no more
// units than resident workgroups), which makes the last round rem * pieces / resident of a
// round plus the fixup: a tile's last contributor reads the other pieces'
// partials, so pieces stay few.  Off when the last round is over 3/4 full, when
// tiles would average under 1.5 pieces, or a share would be under min_share
// K-steps: a cut tile costs a partial store, the last contributor's partial
// reads and an epilogue, which shorter shares do not pay back.  Measured on
// MI355X: with 256x256 tiles (256 KiB partials) 16-step shares lose and 20 and
// more win or break even; 128x128 tiles (64 KiB partials) gain from 10.
// Also off when the last round already gives over 3/4 of the `cus` compute
// units a tile: with two workgroups per CU resident, a CU's second workgroup
// adds about a third to its throughput, so such a round is as good as full and
// a split only adds fixups ([8,512,2048] gram: 288 tiles of 64x64 on 256 CUs,
// unsplit 14.4 us against 18.9 us in 512 units; [3,1024,4096] 88 -> 82 us and
// [8,1024,4096] 185 -> 176 us per step).  And off when the units would outnumber
// the CUs (two on some CUs, for the same reason): gram of 64x64 tiles at
// [1,1024,4096] unsplit 37.7 against 43.2 us per step in 408 units, [2,768,3072]
// 35.9 against 44.1, [4,512,4096] 35.5 against 39.8; with one unit per CU the
// split still wins ([1,512,8192] 35.0 against 42.9, [1,700,5000] 43.2 against 49.5,
// [2,512,4096] 30.6 against 32.5).  64x64 tiles (16 KiB partials, 0.2 us K-steps):
// shares of 6 K-steps or more in up to four pieces (sk_max_pieces); three pieces of
// 12 lose ([2,150,2050] unsplit 25.6 against 27.7 us).
int64_t sk_min_share(int bm, int bn) {
    const int64_t area = int64_t(bm) * bn;
    return area >= 256 * 256 ? 20 : (area <= 64 * 64 ? 6 : 8);
}
// Most pieces a cut tile is split into.  64x64 tiles (16 KiB partials): up to four
// shares of 6 K-steps or more, which shortens the critical path of a long-K stage
// over few tiles more than the extra partial read costs (interleaved A/B against
// three shares of 16 or more, per step: [2,150,2050] 25.4 -> 24.6 us, [1,256,8192]
// 30.8 -> 27.7, [4,128,4096] 24.7 -> 23.3, [1,512,8192] 35.1 -> 33.1,
// [1,200,12000] 42.4 -> 35.5; three shares of 12: [2,150,2050] 26.5 us).  Larger
// tiles: three.
int64_t sk_max_pieces(int bm, int bn) { return int64_t(bm) * bn <= 64 * 64 ? 4 : 3; }

// Long K over few tiles: where the cut tiles would take at most a quarter of the
// CUs and a tile's K loop is longer than `pieces` shares of kLongShare K-steps,
// each tile is cut into up to kLongPieces shares of about kLongShare K-steps (at
// most one unit per CU).  A 64x64 gram tile of 2048 K-steps ([1,8,131072]) would
// otherwise run on a few workgroups, or on one (four pieces of one tile round
// down to no unit at all); the last contributor's partial reads (16 KiB each for
// 64x64 tiles) cost far less than those K-steps.
constexpr int64_t kLongShare = 64;
constexpr int64_t kLongPieces = 32;

SkSplit sk_policy(bool enabled, int64_t tiles, int64_t k_steps, int64_t resident, int64_t cus,
                  int64_t min_share, bool extra_round, int64_t pieces = 3) {
    SkSplit c{tiles, 0, 0, 0};
    if (!enabled || resident < 8) return c;
    const int64_t rem = tiles % resident;
    if (rem == 0 || rem * 4 > resident * 3 || rem * 4 > cus * 3) return c;
    if (k_steps > pieces * kLongShare && rem * pieces * 4 <= cus)
        pieces = std::max(pieces, std::min({kLongPieces, k_steps / kLongShare, cus / rem}));
    int64_t units = std::min<int64_t>(resident, rem * pieces);
    // pieces beyond three stop at one unit per CU
    if (units > cus && rem * 3 <= cus) units = cus;
    units = units / 8 * 8;
    if (units * 2 < rem * 3 || units < 8 || units > cus) return c;
    const int64_t iters = rem * k_steps;
    if (iters < min_share * units || iters >= (int64_t(1) << 31)) return c;
    c.dp_tiles = tiles - rem;
    c.sk_units = static_cast<int32_t>(units);
    c.sk_iters = iters;
    // extra_round: where the last round is short enough to be cut in three pieces
    // per tile, the split covers it and the whole round before it, one unit per
    // resident workgroup (at most one per CU), each 1 + rem / resident tiles of
    // K-steps: one round of whole tiles and a short cut round become one longer
    // round whose tiles are mostly cut in two (one partial read in a fix-up instead
    // of two), and the stage ends earlier.  Measured on MI355X with 256x256 gram
    // and poly tiles (interleaved A/B, per step): [2,4096,8192] 862 -> 836 us,
    // [8,4096,4096] 2035 -> 1993, [1,8192,16384] 3181 -> 3136, [4,4096,4096] 994
    // -> 983, [1,6144,6144] 836 -> 829; a longer last round gains nothing
    // ([3,4096,4096]: 152 of 256 tiles, 745 against 751 us), nor do 64x64 and
    // 128x128 tiles (within 0.5%).  Apply takes it only where its column halves
    // (below) do not take the cut round ([4096,14336]: the halves stay, 671 against
    // 677 us with this split instead): [1,5120,13312] 991 -> 972 us, [1,4096,17408]
    // 798 -> 790, [1,6144,6144] 806.8 against 806.0.
    if (extra_round && rem * 3 <= resident && tiles >= rem + resident && resident <= cus &&
        resident % 8 == 0 && (rem + resident) * k_steps < (int64_t(1) << 31)) {
        c.dp_tiles = tiles - rem - resident;
        c.sk_units = static_cast<int32_t>(resident);
        c.sk_iters = (rem + resident) * k_steps;
    }
    return c;
}

// Where a plan is built for: the device (its plan-cache key), its compute units
// (0: unknown, no stream-K split) and, per stage, the DMA-fed kernel's resident
// workgroups per CU (-1: ask the runtime for the device's value).
struct Target {
    int device;
    int cus;
    int blocks_per_cu[3];
};

// Byte extent of one matrix of every buffer a kernel addresses with 32-bit
// offsets must stay below 2^31: the DMA-fed kernels mark out-of-range chunks with
// the offset 2^31, which is only out of range for buffers below that size.
constexpr int64_t kMaxMatrixElems = int64_t(1) << 30;

int build_plan(int64_t batch, int64_t m, int64_t n, const Knobs &knobs, const Target &tgt,
               Plan &out) {
    const bool tall = m > n;
    const int64_t small = std::min(m, n), large = std::max(m, n);
    Plan p{};
    p.gram_tile = static_cast<int>(knobs.gram_tile);
    p.poly_tile = static_cast<int>(knobs.poly_tile);
    p.apply_bm = static_cast<int>(knobs.apply_bm);
    p.apply_bn = static_cast<int>(knobs.apply_bn);
    p.m = m;
    p.n = n;
    p.s = small;
    p.tall = tall;
    (void)large;
    // A and P are [mp, mp] with mp the larger of the two stages' tile extents.
    const int64_t ext_gram = round_up(small, p.gram_tile), ext_poly = round_up(small, p.poly_tile);
    p.mp = std::max(ext_gram, ext_poly);
    if (p.mp * p.mp >= kMaxMatrixElems)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "matrix too large (2^30 elements or more)");
    p.gram_nt = static_cast<int>(ext_gram / p.gram_tile);
    p.poly_nt = static_cast<int>(ext_poly / p.poly_tile);
    p.apply_tm = static_cast<int>((m + p.apply_bm - 1) / p.apply_bm);
    p.apply_tn = static_cast<int>((n + p.apply_bn - 1) / p.apply_bn);
    p.gram_grid = batch * (int64_t(p.gram_nt) * (p.gram_nt + 1) / 2);
    p.poly_grid = batch * (int64_t(p.poly_nt) * (p.poly_nt + 1) / 2);
    p.apply_grid = batch * int64_t(p.apply_tm) * p.apply_tn;
    p.gram_bytes = static_cast<size_t>(batch) * p.mp * p.mp * 2u;
    // The right-Gram stages exist only as DMA-fed kernels: MUON_POLAR_STREAM=0
    // selects the register-staged kernels for m <= n alone.
    p.stream = knobs.stream != 0 || tall;
    p.y_cpol = static_cast<int>(knobs.y_cpol);
    p.ap_cpol = static_cast<int>(knobs.ap_cpol);
    if (p.gram_grid >= (int64_t(1) << 31) || p.apply_grid >= (int64_t(1) << 31))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "grid too large");

    const int cus = tgt.cus;
    p.pad = p.stream && n % 8 != 0;
    p.np = p.pad ? round_up(n, 64) : n;
    // the padded copy of X is read with the same 32-bit offsets as X
    if (m * p.np >= kMaxMatrixElems)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "matrix too large (its copy padded to a multiple of 64 columns has 2^30 "
                    "elements or more)");
    // Stream-K needs the DMA-fed kernels and a device to size the split for.
    const bool sk_ok = p.stream && cus > 0;
    const int tiles_bm[3] = {p.gram_tile, p.poly_tile, p.apply_bm};
    const int tiles_bn[3] = {p.gram_tile, p.poly_tile, p.apply_bn};
    const Stage stages[3] = {tall ? Stage::GramT : Stage::Gram, Stage::Poly,
                             tall ? Stage::ApplyR : Stage::Apply};
    const int64_t grids[3] = {p.gram_grid, p.poly_grid, p.apply_grid};
    const int64_t ksteps[3] = {round_up(large, 64) / 64, round_up(small, 64) / 64,
                               round_up(small, 64) / 64};
    p.sk_any = false;
    p.counter_stride = 0;
    size_t partial_bytes = 0;
    for (int s = 0; s < 3; ++s) {
        // 192x192 tiles: 8 waves are the wave-pair kernels (MUON_POLAR_PAIR=0: 4 waves)
        const bool no_pair = tiles_bm[s] == 192 && knobs.pair == 0;
        p.waves[s] = muon_polar::stream_waves(tiles_bm[s], tiles_bn[s],
                                              no_pair ? 4 : static_cast<int>(knobs.waves));
        p.depth[s] = knobs.depth[s] != 0
                         ? static_cast<int>(knobs.depth[s])
                         : default_depth(tiles_bm[s], tiles_bn[s], p.waves[s], grids[s], cus);
        if (p.stream && !muon_polar::stream_depth_supported(stages[s], tiles_bm[s], tiles_bn[s],
                                                            p.waves[s], p.depth[s]))
            return fail(MUON_POLAR_ERR_CONFIG,
                        "no DMA-fed kernel for this tile, wave count and MUON_POLAR_*_DEPTH "
                        "(128x128: 2 or 4; 64x64: 2, 4 or 8; 128x256 / 256x128: 2 or 3; 192x192: 2, or 3 "
                        "with 8 waves; "
                        "others: 2)");
    }
    for (int s = 0; s < 3; ++s) {
        // Gram and poly on 64x64 tiles: pair the diagonal tiles when that takes
        // fewer rounds of one workgroup per CU, and then run unsplit ([8,512,2048]:
        // 288 tiles -> 256 units, one per CU, where 32 CUs ran two tiles).
        if (s < 2 && knobs.diag_pairs != 0 && p.stream && cus > 0 && tiles_bm[s] == 64 &&
            tiles_bn[s] == 64 && p.waves[s] == 4) {
            const int nt = s == 0 ? p.gram_nt : p.poly_nt;
            const int64_t units = batch * muon_polar::sym_units(nt, true);
            if (nt >= 2 && ceil_div(units, cus) < ceil_div(grids[s], cus)) {
                p.diag[s] = true;
                p.sk[s] = SkSplit{units, 0, 0, 0};
                continue;
            }
        }
        const bool sk_stage = sk_ok && (knobs.stream_k >> s & 1u) != 0;
        int occ = 0;
        if (sk_stage)
            occ = tgt.blocks_per_cu[s] >= 0
                      ? tgt.blocks_per_cu[s]
                      : muon_polar::stream_blocks_per_cu(stages[s], tiles_bm[s], tiles_bn[s],
                                                         p.waves[s], p.depth[s]);
        p.sk[s] = sk_policy(sk_ok && occ > 0, grids[s], ksteps[s], int64_t(cus) * occ, cus,
                            (knobs.sk_share ? int64_t(knobs.sk_share) : sk_min_share(tiles_bm[s], tiles_bn[s])),
                            s < 2 && (knobs.sk_rounds >> s & 1u) != 0 &&
                                tiles_bm[s] * tiles_bn[s] >= 256 * 256,
                            knobs.sk_pieces ? int64_t(knobs.sk_pieces)
                                            : sk_max_pieces(tiles_bm[s], tiles_bn[s]));
        // Apply's cut round as 256x128 column halves, one per workgroup, where the
        // halves number between a half and a whole round of resident workgroups
        // (each half is then as long as a stream-K share, or shorter): the same
        // length of the last round without partials, arrival words or fix-ups.
        // [4096,14336]: 128 tiles -> 256 halves.
        if (s == 2 && knobs.halves == 2 && sk_ok && tiles_bm[s] == 256 && tiles_bn[s] == 256 &&
            p.waves[s] == 8 && p.depth[s] == 2 && (2 * grids[s]) % 8 == 0) {
            // every tile as two halves
            p.sk[s] = SkSplit{0, static_cast<int32_t>(2 * grids[s]), 0,
                              static_cast<int32_t>(knobs.halves_depth)};
            continue;
        }
        if (s == 2 && p.sk[s].sk_units > 0 && knobs.halves == 1 && tiles_bm[s] == 256 &&
            tiles_bn[s] == 256 && p.waves[s] == 8 && p.depth[s] == 2) {
            const int64_t halves = 2 * (grids[s] - p.sk[s].dp_tiles);
            const int64_t resident = int64_t(cus) * occ;
            if (halves % 8 == 0 && 2 * halves > resident && halves <= resident) {
                p.sk[s].sk_units = static_cast<int32_t>(halves);
                p.sk[s].sk_iters = 0;
                p.sk[s].halves = static_cast<int32_t>(knobs.halves_depth);
                continue;  // no partials, no arrival words
            }
        }
        // Apply's two-round split (MUON_POLAR_SK_ROUNDS bit 2, sk_policy) where the
        // halves above do not take its cut round.
        if (s == 2 && p.sk[s].sk_units > 0 && (knobs.sk_rounds >> 2 & 1u) != 0 &&
            tiles_bm[s] * tiles_bn[s] >= 256 * 256)
            p.sk[s] = sk_policy(true, grids[s], ksteps[s], int64_t(cus) * occ, cus,
                                (knobs.sk_share ? int64_t(knobs.sk_share) : sk_min_share(tiles_bm[s], tiles_bn[s])), true);
        // A partial last round that stream-K leaves whole (its shares would be
        // too short) runs as halves too, where they fit one round.
        if (s == 2 && p.sk[s].sk_units == 0 && knobs.halves == 1 && sk_ok && occ > 0 &&
            tiles_bm[s] == 256 && tiles_bn[s] == 256 && p.waves[s] == 8 && p.depth[s] == 2) {
            const int64_t resident = int64_t(cus) * occ;
            const int64_t rem = grids[s] % resident;
            if (grids[s] > resident && rem > 0 && 4 * rem <= 3 * resident &&
                4 * rem <= 3 * int64_t(cus) && (2 * rem) % 8 == 0 && 2 * rem <= resident) {
                p.sk[s] = SkSplit{grids[s] - rem, static_cast<int32_t>(2 * rem), 0,
                                  static_cast<int32_t>(knobs.halves_depth)};
                continue;
            }
        }
        if (p.sk[s].sk_units > 0) {
            p.sk_any = true;
            const int64_t sk_tiles = grids[s] - p.sk[s].dp_tiles;
            p.counter_stride = std::max<int64_t>(p.counter_stride, sk_tiles);
            partial_bytes = std::max(partial_bytes,
                                     size_t(muon_polar::sk_slots(p.sk[s].sk_units, sk_tiles)) *
                                         tiles_bm[s] * tiles_bn[s] * sizeof(float));
        }
    }
    p.counters_offset = 2 * align256(p.gram_bytes);
    p.partials_offset =
        p.counters_offset + align256(size_t(3) * p.counter_stride * sizeof(uint64_t));
    p.pad_offset = p.partials_offset + align256(partial_bytes);
    p.workspace_bytes =
        p.pad_offset + (p.pad ? align256(static_cast<size_t>(batch) * m * p.np * 2u) : 0u);
    p.express_x_offset = p.workspace_bytes;
    // the chain's scratch iterate; with padded rows it holds a padded [batch, m, np]
    // matrix (run_steps keeps the iterates of a chain padded between its steps)
    p.express_norm_offset =
        p.express_x_offset + align256(size_t(batch) * m * (p.pad ? p.np : n) * 2u);
    p.express_workspace_bytes =
        p.express_norm_offset +
        align256(size_t(batch) * muon_polar::norm_chunks(batch, m * n) * sizeof(float));
    p.muon_o_offset = p.express_workspace_bytes;
    p.muon_workspace_bytes = p.muon_o_offset + align256(size_t(batch) * m * n * 2u);
    out = p;
    return MUON_POLAR_OK;
}

// one_round: the plan without the two-round stream-K split (MUON_POLAR_SK_ROUNDS
// = 0), whose partial area is smaller (the allocation-free step falls back to it).
int get_plan(int64_t batch, int64_t m, int64_t n, Plan &out, bool one_round = false) {
    int st = check_shape(batch, m, n);
    if (st != MUON_POLAR_OK) return st;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) device = -1;
    const int cus = device_cus(device);
    Knobs knobs{};
    st = read_knobs(batch, m, n, cus > 0 ? cus : 256, knobs);
    if (st != MUON_POLAR_OK) return st;
    if (one_round) knobs.sk_rounds = 0;
    const PlanKey key{device, batch, m, n, knobs};
    std::lock_guard<std::mutex> lock(g_plan_mutex);
    const auto found = g_plans.find(key);
    if (found != g_plans.end()) {
        out = found->second;
        return MUON_POLAR_OK;
    }
    Plan p{};
    st = build_plan(batch, m, n, knobs, Target{device, cus, {-1, -1, -1}}, p);
    if (st != MUON_POLAR_OK) return st;
    g_plans.emplace(key, p);
    out = p;
    return MUON_POLAR_OK;
}

// MUON_POLAR_DEBUG_SYNC: synchronise after each stage when the variable is
// present, whatever its value (reference binding.cpp:93-101; README.md:224).
int finish_stage(hipError_t launch, hipStream_t stream, const char *stage) {
    if (launch != hipSuccess)
        return fail(MUON_POLAR_ERR_HIP, std::string("stage ") + stage +
                                            " launch failed: " + hipGetErrorString(launch));
    if (std::getenv("MUON_POLAR_DEBUG_SYNC") != nullptr) {
        const hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess)
            return fail(MUON_POLAR_ERR_HIP,
                        std::string("stage ") + stage + " failed: " + hipGetErrorString(e));
    }
    return MUON_POLAR_OK;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// Whether the DMA-fed kernels read X rows `ldx` elements apart in place: rows of
// whole 16-byte chunks (16-byte aligned X), or rows of an even number of elements
// starting on 4-byte boundaries, whose chunks the 16-byte DMA reads at 4-byte
// aligned addresses (the chunk that straddles a row's end is masked: gram zeroes
// its positions past n in LDS, apply only feeds it to output columns >= n, which
// are not stored).
bool dma_rows(int64_t ldx, const void *x) {
    return ldx % 8 == 0 ? aligned16(x) : (ldx % 2 == 0 && aligned4(x));
}

// Whether byte ranges [a, a + a_bytes) and [b, b + b_bytes) share a byte.
bool overlaps(const void *a, size_t a_bytes, const void *b, size_t b_bytes) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + b_bytes && y < x + a_bytes;
}

// Whether [buf, buf + bytes) shares a byte with the part of a stage call's workspace
// that the call writes besides its output: the stream-K arrival words, the partial
// slots and the padded copy of X (bytes [counters_offset, workspace_bytes)).  The A and
// P areas before it may be the caller's gram and poly buffers.
bool overlaps_stage_area(const Plan &p, const void *workspace, const void *buf, size_t bytes) {
    if (workspace == nullptr) return false;
    const char *area = static_cast<const char *>(workspace) + p.counters_offset;
    return overlaps(area, p.workspace_bytes - p.counters_offset, buf, bytes);
}

// Workspace areas of polar_step's stream-K splits (null when not splitting:
// the stage entry points have no workspace and run one tile per workgroup).
struct SkArea {
    float *partials;
    uint64_t *counters;  // this stage's arrival words
};

// Launch tokens of the stream-K arrival words: a fresh one per launch, so words
// left by other launches (or never written) count as zero and need no clearing.
std::atomic<uint32_t> g_launch_token{1};

SkArea sk_area(const Plan &p, void *workspace, int stage) {
    char *ws = static_cast<char *>(workspace);
    return SkArea{reinterpret_cast<float *>(ws + p.partials_offset),
                  reinterpret_cast<uint64_t *>(ws + p.counters_offset) + stage * p.counter_stride};
}

int check_workspace(const Plan &p, const void *workspace, size_t workspace_bytes) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
        return fail(MUON_POLAR_ERR_WORKSPACE,
                    "workspace must hold " + std::to_string(p.workspace_bytes) + " bytes, got " +
                        std::to_string(workspace == nullptr ? 0 : workspace_bytes));
    if (!aligned16(workspace))
        return fail(MUON_POLAR_ERR_WORKSPACE, "workspace must be 16-byte aligned");
    return MUON_POLAR_OK;
}

// Stream-K area of one stage call: null without a workspace (no split).
int stage_area(const Plan &p, void *workspace, size_t workspace_bytes, int stage, SkArea &area,
               const SkArea *&out) {
    out = nullptr;
    if (workspace == nullptr) return MUON_POLAR_OK;
    const int st = check_workspace(p, workspace, workspace_bytes);
    if (st != MUON_POLAR_OK) return st;
    area = sk_area(p, workspace, stage);
    out = &area;
    return MUON_POLAR_OK;
}

// Super-block side of the triangular stages' tile walk (MUON_POLAR_SYM_GROUP; 1: row
// by row).  8x8 blocks of tiles measured 1.5-2.5% faster than row by row at
// [4096,14336] (771 -> 757 us) and [2,2048,8192] (297 -> 290 us), the same at
// [4,4096,4096]; with 8 or fewer tiles per side the walk is row by row anyway.
int32_t sym_group() {
    return static_cast<int32_t>(std::min<uint64_t>(64, env_u64("MUON_POLAR_SYM_GROUP", 8)));
}

// Column tiles per raster group of the apply stages: 8 for wide X (4096 x 14336:
// 56 column tiles), 4 for narrower ones (n = 4096: 16 column tiles; 476 vs 498 us).
int32_t apply_group(const Plan &p) {
    const uint64_t group_default = p.apply_tn >= 32 ? 8 : 4;
    return static_cast<int32_t>(
        std::max<uint64_t>(1, env_u64("MUON_POLAR_APPLY_GROUP_N", group_default)));
}

// One stage launch: which kernel and its by-value arguments.  The builders below
// fill it from the plan, prepare_stage adds the work split and launch_stage runs
// it; muon_polar_check_plan walks the same arguments on the host.
struct StageLaunch {
    Stage stage;
    int sk_index;     // 0 gram, 1 poly, 2 apply: the plan's split and arrival words
    int bm, bn, waves, depth;
    bool stream_ok;   // DMA-fed kernel (else register-staged)
    bool vec;         // register-staged kernel: 16-byte accesses
    int64_t grid;     // register-staged grid: one workgroup per tile
    // byte extent of one batch matrix of rowop, colop and epi, in 64 bits (the
    // GemmArgs fields are 32-bit)
    int64_t extent[3];
    // X rows read in place end inside the last K-step (ldx % 64 != 0): the
    // kernel masks that step's chunks past row_k (gram and apply-right); 2: rows
    // of ldx % 8 != 0 elements (gram), whose chunk straddling n is also masked
    int k_tail;
    GemmArgs g;
};

// x: [batch, m, n] rows `ldx` elements apart (n, or np for the padded copy).
StageLaunch gram_launch(const Plan &p, const void *x, int64_t ldx, void *gram, int64_t m,
                        int64_t n) {
    StageLaunch L{};
    GemmArgs &g = L.g;
    g.rowop = g.colop = g.epi = static_cast<const uint16_t *>(x);
    g.out = static_cast<uint16_t *>(gram);
    g.sb_row = g.sb_col = g.sb_epi = m * ldx;
    g.sb_out = p.mp * p.mp;
    g.ld_row = g.ld_col = g.ld_epi = static_cast<int32_t>(ldx);
    g.ld_out = static_cast<int32_t>(p.mp);
    g.row_rows = g.col_rows = static_cast<int32_t>(m);
    g.row_k = g.col_k = static_cast<int32_t>(n);
    g.k_loop = static_cast<int32_t>(round_up(n, 64));
    g.out_rows = g.out_cols = static_cast<int32_t>(p.mp);
    g.tiles_m = g.tiles_n = p.gram_nt;
    g.tiles_per_batch = p.gram_nt * (p.gram_nt + 1) / 2;
    g.s_epi = 0.0f;
    g.s_acc = 1.0f;
    g.out_vec = 1;
    L.extent[0] = L.extent[1] = L.extent[2] = m * ldx * 2;
    g.group_n = sym_group();
    const bool vec = (ldx % 8 == 0) && aligned16(x);
    // DMA-fed: X rows are K-contiguous panels of 16-byte chunks; a last K-step
    // past n (ldx % 64 != 0) is loaded with its chunks past n masked
    const bool dma = dma_rows(ldx, x);
    L.k_tail = ldx % 64 == 0 ? 0 : ldx % 8 == 0 ? 1 : 2;
    L.stage = Stage::Gram;
    L.sk_index = 0;
    L.bm = L.bn = p.gram_tile;
    L.waves = p.waves[0];
    L.depth = p.depth[0];
    L.stream_ok = p.stream && dma;
    L.vec = vec;
    L.grid = p.gram_grid;
    g.out_cpol = p.ap_cpol;
    return L;
}

StageLaunch poly_launch(const Plan &p, const void *gram, void *poly, double b, double c) {
    StageLaunch L{};
    GemmArgs &g = L.g;
    g.rowop = g.colop = g.epi = static_cast<const uint16_t *>(gram);
    g.out = static_cast<uint16_t *>(poly);
    g.sb_row = g.sb_col = g.sb_epi = g.sb_out = p.mp * p.mp;
    g.ld_row = g.ld_col = g.ld_epi = g.ld_out = static_cast<int32_t>(p.mp);
    g.row_rows = g.col_rows = g.row_k = g.col_k = static_cast<int32_t>(p.mp);
    // A is zero beyond row / column s: the K loop stops at s (rounded to a step).
    g.k_loop = static_cast<int32_t>(round_up(p.s, 64));
    g.out_rows = g.out_cols = static_cast<int32_t>(p.mp);
    g.tiles_m = g.tiles_n = p.poly_nt;
    g.tiles_per_batch = p.poly_nt * (p.poly_nt + 1) / 2;
    g.s_epi = static_cast<float>(b);
    g.s_acc = static_cast<float>(c);
    g.out_vec = 1;
    L.extent[0] = L.extent[1] = L.extent[2] = p.mp * p.mp * 2;
    g.group_n = sym_group();
    L.stage = Stage::Poly;
    L.sk_index = 1;
    L.bm = L.bn = p.poly_tile;
    L.waves = p.waves[1];
    L.depth = p.depth[1];
    L.stream_ok = p.stream;
    L.vec = true;
    L.grid = p.poly_grid;
    g.out_cpol = p.ap_cpol;
    return L;
}

// x: [batch, m, n] rows `ldx` elements apart (n, or np for the padded copy);
// y: [batch, m, n] dense.
// n_out (>= n, default n): columns of Y written and its row length.  A padded Y
// (n_out = np) gets the padded columns too, which come out +0 (X is zero there).
StageLaunch apply_launch(const Plan &p, const void *poly, const void *x, int64_t ldx, void *y,
                         int64_t m, int64_t n, double a, int64_t n_out = 0) {
    if (n_out <= 0) n_out = n;
    StageLaunch L{};
    GemmArgs &g = L.g;
    g.rowop = static_cast<const uint16_t *>(poly);
    g.colop = g.epi = static_cast<const uint16_t *>(x);
    g.out = static_cast<uint16_t *>(y);
    g.sb_row = p.mp * p.mp;
    g.sb_col = g.sb_epi = m * ldx;
    g.sb_out = m * n_out;
    g.ld_row = static_cast<int32_t>(p.mp);
    g.ld_col = g.ld_epi = static_cast<int32_t>(ldx);
    g.ld_out = static_cast<int32_t>(n_out);
    g.row_rows = g.row_k = static_cast<int32_t>(p.mp);
    g.col_rows = static_cast<int32_t>(n);
    g.col_k = static_cast<int32_t>(m);
    g.k_loop = static_cast<int32_t>(round_up(m, 64));  // P is zero beyond column m
    g.out_rows = static_cast<int32_t>(m);
    g.out_cols = static_cast<int32_t>(n_out);
    g.tiles_m = p.apply_tm;
    g.tiles_n = p.apply_tn;
    g.tiles_per_batch = p.apply_tm * p.apply_tn;
    g.s_epi = static_cast<float>(a);
    g.s_acc = 1.0f;
    L.extent[0] = p.mp * p.mp * 2;
    L.extent[1] = L.extent[2] = m * ldx * 2;
    g.out_vec = (n_out % 8 == 0 && aligned16(y)) ? 1 : !aligned4(y) ? 0 : n_out % 2 == 0 ? 2 : 3;
    g.group_n = apply_group(p);
    g.out_cpol = p.y_cpol;
    // DMA-fed kernel: X rows of whole 16-byte chunks (Y any alignment: 16-byte stores
    // for out_vec 1, and for 2 and 3 inside the rows they cover; 2-byte stores otherwise);
    // register-staged kernel: vectors on both or neither.
    const bool xvec = (ldx % 8 == 0) && aligned16(x);
    L.stage = Stage::Apply;
    L.sk_index = 2;
    L.bm = p.apply_bm;
    L.bn = p.apply_bn;
    L.waves = p.waves[2];
    L.depth = p.depth[2];
    L.stream_ok = p.stream && dma_rows(ldx, x);
    L.vec = xvec && g.out_vec == 1;
    L.grid = p.apply_grid;
    return L;
}

// Right-Gram stages for m > n (X is [m, n]): G = Xᵀ·X over the n x n upper
// tiles, both operands read N-contiguous from X's rows (K runs over the m rows).
StageLaunch gram_t_launch(const Plan &p, const void *x, int64_t ldx, void *gram, int64_t m,
                          int64_t n) {
    StageLaunch L{};
    GemmArgs &g = L.g;
    g.rowop = g.colop = g.epi = static_cast<const uint16_t *>(x);
    g.out = static_cast<uint16_t *>(gram);
    g.sb_row = g.sb_col = g.sb_epi = m * ldx;
    g.sb_out = p.mp * p.mp;
    g.ld_row = g.ld_col = g.ld_epi = static_cast<int32_t>(ldx);
    g.ld_out = static_cast<int32_t>(p.mp);
    g.row_rows = g.col_rows = static_cast<int32_t>(n);  // output index: columns of X
    g.row_k = g.col_k = static_cast<int32_t>(m);        // contraction: rows of X
    g.k_loop = static_cast<int32_t>(round_up(m, 64));
    g.out_rows = g.out_cols = static_cast<int32_t>(p.mp);
    g.tiles_m = g.tiles_n = p.gram_nt;
    g.tiles_per_batch = p.gram_nt * (p.gram_nt + 1) / 2;
    g.s_epi = 0.0f;
    g.s_acc = 1.0f;
    g.out_vec = 1;
    L.extent[0] = L.extent[1] = L.extent[2] = m * ldx * 2;
    g.group_n = sym_group();
    L.stage = Stage::GramT;
    L.sk_index = 0;
    L.bm = L.bn = p.gram_tile;
    L.waves = p.waves[0];
    L.depth = p.depth[0];
    L.stream_ok = true;
    L.vec = true;
    L.grid = p.gram_grid;
    g.out_cpol = p.ap_cpol;
    return L;
}

// Y = a·X + X·P for m > n: X rows and P rows (P is symmetric) are both
// K-contiguous; the output [m, n] and the a·X epilogue are stage 3's.
StageLaunch apply_r_launch(const Plan &p, const void *poly, const void *x, int64_t ldx, void *y,
                           int64_t m, int64_t n, double a) {
    StageLaunch L{};
    GemmArgs &g = L.g;
    g.rowop = g.epi = static_cast<const uint16_t *>(x);
    g.colop = static_cast<const uint16_t *>(poly);
    g.out = static_cast<uint16_t *>(y);
    g.sb_row = g.sb_epi = m * ldx;
    g.sb_out = m * n;
    g.sb_col = p.mp * p.mp;
    g.ld_row = g.ld_epi = static_cast<int32_t>(ldx);
    g.ld_out = static_cast<int32_t>(n);
    g.ld_col = static_cast<int32_t>(p.mp);
    g.row_rows = static_cast<int32_t>(m);
    g.row_k = static_cast<int32_t>(n);
    g.col_rows = g.col_k = static_cast<int32_t>(p.mp);
    g.k_loop = static_cast<int32_t>(round_up(n, 64));  // P is zero beyond column n
    g.out_rows = static_cast<int32_t>(m);
    g.out_cols = static_cast<int32_t>(n);
    g.tiles_m = p.apply_tm;
    g.tiles_n = p.apply_tn;
    g.tiles_per_batch = p.apply_tm * p.apply_tn;
    g.s_epi = static_cast<float>(a);
    g.s_acc = 1.0f;
    L.extent[0] = L.extent[2] = m * ldx * 2;
    L.extent[1] = p.mp * p.mp * 2;
    g.out_vec = (n % 8 == 0 && aligned16(y)) ? 1 : 0;
    g.group_n = apply_group(p);
    g.out_cpol = p.y_cpol;
    L.k_tail = ldx % 64 != 0 ? 1 : 0;
    L.stage = Stage::ApplyR;
    L.sk_index = 2;
    L.bm = p.apply_bm;
    L.bn = p.apply_bn;
    L.waves = p.waves[2];
    L.depth = p.depth[2];
    L.stream_ok = true;
    L.vec = true;
    L.grid = p.apply_grid;
    return L;
}

// Work split of a stage launch: whole tiles one per workgroup, plus the plan's
// stream-K split when the DMA-fed kernel runs and a stream-K area is given.
// `token` tags this launch's arrival words.
void prepare_stage(StageLaunch &L, int64_t batch, const Plan &p, const SkArea *area,
                   uint32_t token) {
    GemmArgs &g = L.g;
    g.bytes_row = static_cast<uint32_t>(L.extent[0]);
    g.bytes_col = static_cast<uint32_t>(L.extent[1]);
    g.bytes_epi = static_cast<uint32_t>(L.extent[2]);
    g.diag_pairs = 0;
    if (L.stream_ok && L.sk_index < 2 && p.diag[L.sk_index]) {
        g.diag_pairs = 1;
        g.tiles_per_batch = muon_polar::sym_units(g.tiles_m, true);
    }
    g.total_tiles = static_cast<int32_t>(batch * g.tiles_per_batch);
    g.k_steps = g.k_loop / 64;
    g.dp_tiles = g.total_tiles;
    g.sk_units = 0;
    g.sk_iters = 0;
    g.halves = 0;
    const SkSplit &sk = p.sk[L.sk_index];
    if (L.stream_ok && area != nullptr && sk.sk_units > 0) {
        g.dp_tiles = static_cast<int32_t>(sk.dp_tiles);
        g.sk_units = sk.sk_units;
        g.sk_iters = sk.sk_iters;
        if (sk.halves) {
            g.halves = sk.halves;  // whole tiles, then 256x128 halves: no partials or words
        } else {
            g.partials = area->partials;
            g.counters = area->counters;
            g.token = token;
        }
    }
    g.per_xcd = (g.dp_tiles + 7) / 8;
}

int launch_stage(StageLaunch &L, int64_t batch, const Plan &p, const SkArea *area,
                 hipStream_t stream, const char *name) {
    prepare_stage(L, batch, p, area, g_launch_token.fetch_add(1, std::memory_order_relaxed));
    const hipError_t e =
        L.stream_ok
            ? muon_polar::launch_stream(L.stage, L.bm, L.bn, L.waves, L.depth, L.g, stream,
                                        L.k_tail)
            : muon_polar::launch_gemm(L.stage, L.bm, L.bn, L.vec, L.g, static_cast<int>(L.grid),
                                      stream);
    return finish_stage(e, stream, name);
}

int run_gram(const Plan &p, const void *x, int64_t ldx, void *gram, int64_t batch, int64_t m,
             int64_t n, const SkArea *area, hipStream_t stream) {
    StageLaunch L = gram_launch(p, x, ldx, gram, m, n);
    return launch_stage(L, batch, p, area, stream, "gram");
}

int run_poly(const Plan &p, const void *gram, void *poly, int64_t batch, double b, double c,
             const SkArea *area, hipStream_t stream) {
    StageLaunch L = poly_launch(p, gram, poly, b, c);
    return launch_stage(L, batch, p, area, stream, "poly");
}

int run_apply(const Plan &p, const void *poly, const void *x, int64_t ldx, void *y, int64_t batch,
              int64_t m, int64_t n, double a, const SkArea *area, hipStream_t stream,
              int64_t n_out = 0) {
    StageLaunch L = apply_launch(p, poly, x, ldx, y, m, n, a, n_out);
    return launch_stage(L, batch, p, area, stream, "apply");
}

int run_gram_t(const Plan &p, const void *x, int64_t ldx, void *gram, int64_t batch, int64_t m,
               int64_t n, const SkArea *area, hipStream_t stream) {
    StageLaunch L = gram_t_launch(p, x, ldx, gram, m, n);
    return launch_stage(L, batch, p, area, stream, "gram");
}

int run_apply_r(const Plan &p, const void *poly, const void *x, int64_t ldx, void *y,
                int64_t batch, int64_t m, int64_t n, double a, const SkArea *area,
                hipStream_t stream) {
    StageLaunch L = apply_r_launch(p, poly, x, ldx, y, m, n, a);
    return launch_stage(L, batch, p, area, stream, "apply");
}

// m > n runs only on the DMA-fed kernels.
int check_tall(const Plan &p, const void *x, const void *y) {
    if (p.n % 8 != 0 || !aligned16(x) || !aligned16(y))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "m > n runs the right-Gram form, which needs n % 8 == 0 and 16-byte aligned "
                    "x and y; otherwise transpose outside");
    return MUON_POLAR_OK;
}

// Rows of n % 8 != 0 elements that the DMA-fed kernels cannot read in place (an
// odd n, or X not 4-byte aligned): copy X into the workspace's zero-padded buffer
// and point (xs, ldx) at it; otherwise leave them at X.
bool pad_needed(const Plan &p, const void *x) { return p.pad && !dma_rows(p.n, x); }

// force: pad rows of n % 8 != 0 elements even where they could be read in place (a
// chain's first step, which starts the chain's padded iterates).
int pad_input(const Plan &p, void *workspace, const void *x, int64_t batch, hipStream_t stream,
              const void *&xs, int64_t &ldx, bool force = false) {
    if (!(pad_needed(p, x) || (force && p.pad))) return MUON_POLAR_OK;
    uint16_t *xp = reinterpret_cast<uint16_t *>(static_cast<char *>(workspace) + p.pad_offset);
    const int st = finish_stage(
        muon_polar::launch_pad_rows(static_cast<const uint16_t *>(x), xp, batch * p.m, p.n, p.np,
                                    stream),
        stream, "pad");
    if (st != MUON_POLAR_OK) return st;
    xs = xp;
    ldx = p.np;
    return MUON_POLAR_OK;
}

// One step given the workspace: left form (m <= n) or right-Gram form; rows the
// DMA-fed kernels cannot read in place are first copied into the zero-padded
// buffer (pad_input).
// ldx_in: row length of x (p.n, or p.np for an iterate a chain keeps padded); n_out:
// row length of y (p.n, or p.np to keep the next iterate padded); force_pad: copy x
// into the padded buffer whenever its rows are not whole 16-byte chunks.
int run_step(const Plan &p, const void *x, void *y, void *workspace, int64_t batch, double a,
             double b, double c, hipStream_t stream, int64_t ldx_in = 0, int64_t n_out = 0,
             bool force_pad = false) {
    char *ws = static_cast<char *>(workspace);
    void *gram = ws;
    void *poly = ws + align256(p.gram_bytes);
    const SkArea areas[3] = {sk_area(p, workspace, 0), sk_area(p, workspace, 1),
                             sk_area(p, workspace, 2)};
    const void *xs = x;
    int64_t ldx = ldx_in > 0 ? ldx_in : p.n;
    int st =
        ldx == p.n ? pad_input(p, workspace, x, batch, stream, xs, ldx, force_pad) : MUON_POLAR_OK;
    if (st != MUON_POLAR_OK) return st;
    st = p.tall ? run_gram_t(p, xs, ldx, gram, batch, p.m, p.n, &areas[0], stream)
                : run_gram(p, xs, ldx, gram, batch, p.m, p.n, &areas[0], stream);
    if (st != MUON_POLAR_OK) return st;
    st = run_poly(p, gram, poly, batch, b, c, &areas[1], stream);
    if (st != MUON_POLAR_OK) return st;
    return p.tall ? run_apply_r(p, poly, xs, ldx, y, batch, p.m, p.n, a, &areas[2], stream)
                  : run_apply(p, poly, xs, ldx, y, batch, p.m, p.n, a, &areas[2], stream, n_out);
}

// `steps` steps from `cur` (the normalised input, in the chain's first buffer),
// alternating between `out` and `scratch` so that the last step writes `out`.
int run_steps(const Plan &p, void *workspace, const uint16_t *cur, uint16_t *out,
              uint16_t *scratch, int64_t batch, const double *coefficients, int64_t steps,
              hipStream_t stream) {
    if (steps == 0) return MUON_POLAR_OK;
    if (steps >= 2 && !p.tall && p.pad) {
        // Rows that are not whole 16-byte chunks (n % 8 != 0): the first step pads its
        // input into the workspace's padded buffer (as a single step does for odd n;
        // even n it could read in place), but writes its result padded ([m, np], the
        // padded columns +0) into the scratch iterate (sized for that), and every later
        // step reads its input in place from one padded buffer and writes the other;
        // only the last writes `out` at width n.  The same values as padding (or
        // masking) each step's input: one copy per chain, and the inner steps read
        // aligned rows and store whole chunks.
        uint16_t *pads[2] = {
            reinterpret_cast<uint16_t *>(static_cast<char *>(workspace) + p.pad_offset),
            scratch};
        for (int64_t i = 0; i < steps; ++i) {
            const bool last = i == steps - 1;
            const void *in = i == 0 ? static_cast<const void *>(cur) : pads[i % 2];
            void *dst = last ? static_cast<void *>(out) : pads[(i + 1) % 2];
            const int st = run_step(p, in, dst, workspace, batch, coefficients[3 * i],
                                    coefficients[3 * i + 1], coefficients[3 * i + 2], stream,
                                    i == 0 ? p.n : p.np, last ? p.n : p.np, true);
            if (st != MUON_POLAR_OK) return st;
        }
        return MUON_POLAR_OK;
    }
    for (int64_t i = 0; i < steps; ++i) {
        uint16_t *next = (steps - i - 1) % 2 == 0 ? out : scratch;
        const int st = run_step(p, cur, next, workspace, batch, coefficients[3 * i],
                                coefficients[3 * i + 1], coefficients[3 * i + 2], stream);
        if (st != MUON_POLAR_OK) return st;
        cur = next;
    }
    return MUON_POLAR_OK;
}

int reject_tall_stage(int64_t m, int64_t n) {
    if (m > n)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "the stage entry points expect m <= n (muon_polar_step runs m > n)");
    return MUON_POLAR_OK;
}

// ---------------------------------------------------------------- plan check
// Host walk of every workgroup of a stage launch (the kernels' own schedule
// functions, polar_schedule.hpp) that bounds the bytes each can store to: its
// output tile (and mirrored tile), its stream-K partial slots and arrival word.
// Addresses are relative to the base pointers in L.g; the caller compares them
// with the buffers' sizes.
void stage_extent(const StageLaunch &L, bool splits, muon_polar_stage_extent &e) {
    const GemmArgs &g = L.g;
    const bool sym = L.stage == Stage::Gram || L.stage == Stage::Poly || L.stage == Stage::GramT;
    e.tile_m = L.bm;
    e.tile_n = L.bn;
    e.waves = L.waves;
    e.depth = L.depth;
    e.dma_fed = L.stream_ok ? 1 : 0;
    e.k_steps = g.k_steps;
    e.total_tiles = g.total_tiles;
    e.dp_tiles = g.dp_tiles;
    e.sk_units = g.sk_units;
    e.halves = g.halves != 0 ? 1 : 0;
    e.diag_pairs = g.diag_pairs;
    e.grid = L.stream_ok ? g.sk_units + 8 * g.per_xcd : static_cast<int32_t>(L.grid);
    e.out_lo = INT64_MAX;
    e.out_hi = 0;
    e.partial_lo = INT64_MAX;
    e.partial_hi = 0;
    e.counter_hi = 0;
    e.extents_ok = 1;
    for (int i = 0; i < 3; ++i) {
        const uint32_t passed = i == 0 ? g.bytes_row : (i == 1 ? g.bytes_col : g.bytes_epi);
        if (L.extent[i] >= (int64_t(1) << 31) || int64_t(passed) != L.extent[i]) e.extents_ok = 0;
    }
    const int nk = g.k_steps;
    const int64_t slot_bytes = int64_t(L.bm) * L.bn * 4;
    // (tile, K-step) iterations covered, to show each is computed exactly once
    std::vector<uint8_t> seen(static_cast<size_t>(g.total_tiles) * nk, 0);
    bool once = true;
    auto store_tile = [&](int bt, int row0, int col0, int bn) {
        // element range [lo, hi) of one workgroup's epilogue stores (a tile of
        // L.bm x bn: bn = L.bn, or a 256x128 half of the apply stage's last round)
        int64_t lo, hi;
        if (sym) {
            // whole tile and its mirror, no bounds checks in the kernel
            const int64_t base = int64_t(bt) * g.sb_out;
            lo = base + std::min(int64_t(row0) * g.ld_out + col0, int64_t(col0) * g.ld_out + row0);
            hi = base + std::max(int64_t(row0 + L.bm - 1) * g.ld_out + col0 + L.bn,
                                 int64_t(col0 + L.bn - 1) * g.ld_out + row0 + L.bm);
            // last column tile: the zeros past the tile grid (zero_past_grid)
            const int ext = g.tiles_n * L.bn;
            if (col0 + L.bn == ext && g.ld_out > ext) {
                const int w = g.ld_out - ext;
                const int cols = row0 + L.bm == ext ? L.bm + w : L.bm;
                hi = std::max({hi, base + int64_t(row0 + L.bm - 1) * g.ld_out + g.ld_out,
                               base + int64_t(g.ld_out - 1) * g.ld_out + row0 + cols});
            }
        } else {
            const int last_row = std::min(row0 + L.bm, g.out_rows) - 1;
            if (last_row < row0 || col0 >= g.out_cols) return;
            // last 16-byte chunk that starts inside the matrix; 8-element vector
            // stores when out_vec is 1, else (2 and 3: vectors only inside the row)
            // stores up to the last column
            const int last_chunk = col0 + 8 * ((std::min(col0 + bn, g.out_cols) - 1 - col0) / 8);
            const int64_t end_col =
                g.out_vec == 1 ? last_chunk + 8 : std::min(col0 + bn, g.out_cols);
            lo = int64_t(bt) * g.sb_out + int64_t(row0) * g.ld_out + col0;
            hi = int64_t(bt) * g.sb_out + int64_t(last_row) * g.ld_out + end_col;
        }
        e.out_lo = std::min(e.out_lo, lo * 2);
        e.out_hi = std::max(e.out_hi, hi * 2);
    };
    // Triangular stages on the DMA-fed kernels: every upper tile of every batch
    // matrix started by exactly one workgroup (units may hold two diagonal tiles).
    const int64_t nbatch = g.tiles_per_batch > 0 ? g.total_tiles / g.tiles_per_batch : 0;
    const int ntm = sym ? g.tiles_m : 0;
    std::vector<uint8_t> tile_seen(static_cast<size_t>(nbatch) * ntm * ntm, 0);
    auto mark_tile = [&](int bt, int tm, int tn) {
        if (bt < 0 || bt >= nbatch || tm < 0 || tn < tm || tn >= ntm) {
            once = false;
            return;
        }
        ++tile_seen[(size_t(bt) * ntm + tm) * ntm + tn];
    };
    if (!L.stream_ok) {
        // register-staged kernels: one workgroup per tile
        for (int64_t w = 0; w < L.grid; ++w) {
            const int bt = static_cast<int>(w / g.tiles_per_batch);
            const int t = static_cast<int>(w - int64_t(bt) * g.tiles_per_batch);
            int tm, tn;
            if (sym)
                muon_polar::upper_tile_of(t, g.tiles_m, tm, tn);
            else {
                tm = t % g.tiles_m;
                tn = t / g.tiles_m;
            }
            store_tile(bt, tm * L.bm, tn * L.bn, L.bn);
            for (int k = 0; k < nk; ++k) once = once && seen[size_t(w) * nk + k]++ == 0;
        }
    } else if (g.halves) {
        // polar_stream_halves_kernel: whole tiles, then two 256x128 halves per tile
        // past dp_tiles, each over the whole K range (seen twice per K-step)
        const int dp_grid = 8 * g.per_xcd;
        for (int w = 0; w < e.grid; ++w) {
            int tlin, half = -1;
            if (w < dp_grid) {
                tlin = (w & 7) * g.per_xcd + (w >> 3);
                if (tlin >= g.dp_tiles) continue;
            } else {
                const int ws = w - dp_grid;
                const int v = (ws & 7) * (g.sk_units >> 3) + (ws >> 3);
                tlin = g.dp_tiles + (v >> 1);
                half = v & 1;
            }
            if (tlin < 0 || tlin >= g.total_tiles) {
                once = false;
                continue;
            }
            const int bt = tlin / g.tiles_per_batch;
            int tm, tn;
            muon_polar::tile_coords(g, sym, tlin - bt * g.tiles_per_batch, tm, tn);
            if (half < 0)
                store_tile(bt, tm * L.bm, tn * L.bn, L.bn);
            else
                store_tile(bt, tm * L.bm, tn * L.bn + half * (L.bn / 2), L.bn / 2);
            for (int k = 0; k < nk; ++k) ++seen[size_t(tlin) * nk + k];
        }
        // whole tiles once, halved tiles twice (one per half), nothing else
        if (sym || L.bn != 256 || g.sk_units != 2 * (g.total_tiles - g.dp_tiles)) once = false;
        for (size_t i = 0; i < seen.size(); ++i) {
            const bool halved = int64_t(i / nk) >= g.dp_tiles;
            once = once && seen[i] == (halved ? 2 : 1);
            seen[i] = 1;
        }
    } else {
        for (int w = 0; w < e.grid; ++w) {
            int unit, tile_base;
            int64_t it_lo, it_hi;
            if (!muon_polar::workgroup_range(g, w, unit, tile_base, it_lo, it_hi)) continue;
            for (int64_t hi = it_hi; hi > it_lo;) {
                const int lt = static_cast<int>((hi - 1) / nk);
                const int64_t tstart = int64_t(lt) * nk;
                const int64_t lo = tstart > it_lo ? tstart : it_lo;
                const int kbeg = static_cast<int>(lo - tstart), kend = static_cast<int>(hi - tstart);
                hi = lo;
                const int tlin = tile_base + lt;
                if (tlin < 0 || tlin >= g.total_tiles) {
                    once = false;
                    continue;
                }
                for (int k = kbeg; k < kend; ++k) once = once && seen[size_t(tlin) * nk + k]++ == 0;
                const int bt = tlin / g.tiles_per_batch;
                const int t = tlin - bt * g.tiles_per_batch;
                int tm, tn;
                muon_polar::tile_coords(g, sym, t, tm, tn);
                const bool pair = sym && muon_polar::is_diag_pair(g, t);
                if (pair) {
                    // the two diagonal tiles (tm, tm) and (tn, tn) = (tm + 1, tm + 1)
                    store_tile(bt, tm * L.bm, tm * L.bn, L.bn);
                    store_tile(bt, tn * L.bm, tn * L.bn, L.bn);
                    if (kbeg != 0 || kend != nk) once = false;  // pairs are never cut
                } else {
                    store_tile(bt, tm * L.bm, tn * L.bn, L.bn);
                }
                if (sym && kbeg == 0) {
                    mark_tile(bt, tm, pair ? tm : tn);
                    if (pair) mark_tile(bt, tn, tn);
                }
                if (kbeg != 0 || kend != nk) {
                    // cut tile: arrival word lt, partial slots of its contributors
                    if (!splits || unit < 0) {
                        once = false;
                        continue;
                    }
                    e.counter_hi = std::max<int64_t>(e.counter_hi, lt + 1);
                    const int u0 = muon_polar::sk_unit_of(g, tstart);
                    const int u1 = muon_polar::sk_unit_of(g, tstart + nk - 1);
                    if (unit < u0 || unit > u1) once = false;
                    for (int u = u0; u <= u1; ++u) {
                        const int64_t slot = muon_polar::sk_slot(u, lt);
                        e.partial_lo = std::min(e.partial_lo, slot * slot_bytes);
                        e.partial_hi = std::max(e.partial_hi, (slot + 1) * slot_bytes);
                    }
                }
            }
        }
    }
    for (uint8_t c : seen) once = once && c == 1;
    if (sym && L.stream_ok && !g.halves)
        for (int64_t bt = 0; bt < nbatch; ++bt)
            for (int tm = 0; tm < ntm; ++tm)
                for (int tn = tm; tn < ntm; ++tn)
                    once = once && tile_seen[(size_t(bt) * ntm + tm) * ntm + tn] == 1;
    e.coverage_ok = once ? 1 : 0;
    if (e.out_lo == INT64_MAX) e.out_lo = 0;
    if (e.partial_lo == INT64_MAX) e.partial_lo = 0;
}

}  // namespace

extern "C" {

int muon_polar_query(int64_t batch, int64_t m, int64_t n, muon_polar_shape_info *info) {
    if (info == nullptr) return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "info is null");
    Plan p{};
    const int st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    info->padded_rows = p.mp;
    info->gram_bytes = p.gram_bytes;
    info->workspace_bytes = p.workspace_bytes;
    info->express_workspace_bytes = p.express_workspace_bytes;
    info->muon_workspace_bytes = p.muon_workspace_bytes;
    return MUON_POLAR_OK;
}

int muon_polar_gram(const void *x, void *gram, void *workspace, size_t workspace_bytes,
                    int64_t batch, int64_t m, int64_t n, hipStream_t stream) {
    if (x == nullptr || gram == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    int st = reject_tall_stage(m, n);
    if (st != MUON_POLAR_OK) return st;
    Plan p{};
    st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    if (!aligned16(gram)) return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "gram must be 16-byte aligned");
    SkArea area{};
    const SkArea *ap = nullptr;
    st = stage_area(p, workspace, workspace_bytes, 0, area, ap);
    if (st != MUON_POLAR_OK) return st;
    // every gram tile reads X's whole K range while other tiles are stored
    const size_t x_bytes = static_cast<size_t>(batch * m * n * 2);
    if (overlaps(x, x_bytes, gram, p.gram_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "x and gram must not overlap");
    if (overlaps_stage_area(p, workspace, x, x_bytes) ||
        overlaps_stage_area(p, workspace, gram, p.gram_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "x and gram must not overlap the workspace past its A and P areas");
    // with the step's workspace, the step's route (the padded copy where pad_input
    // takes it)
    const void *xs = x;
    int64_t ldx = n;
    if (ap != nullptr) {
        st = pad_input(p, workspace, x, batch, stream, xs, ldx);
        if (st != MUON_POLAR_OK) return st;
    }
    return run_gram(p, xs, ldx, gram, batch, m, n, ap, stream);
}

int muon_polar_poly(const void *gram, void *poly, void *workspace, size_t workspace_bytes,
                    int64_t batch, int64_t m, int64_t n, double b, double c, hipStream_t stream) {
    if (gram == nullptr || poly == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    int st = reject_tall_stage(m, n);
    if (st != MUON_POLAR_OK) return st;
    Plan p{};
    st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    if (!aligned16(gram) || !aligned16(poly))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "gram and poly must be 16-byte aligned");
    SkArea area{};
    const SkArea *ap = nullptr;
    st = stage_area(p, workspace, workspace_bytes, 1, area, ap);
    if (st != MUON_POLAR_OK) return st;
    // every poly tile reads whole rows of A while other tiles are stored
    if (overlaps(gram, p.gram_bytes, poly, p.gram_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "gram and poly must not overlap");
    if (overlaps_stage_area(p, workspace, gram, p.gram_bytes) ||
        overlaps_stage_area(p, workspace, poly, p.gram_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "gram and poly must not overlap the workspace past its A and P areas");
    return run_poly(p, gram, poly, batch, b, c, ap, stream);
}

int muon_polar_apply(const void *poly, const void *x, void *y, void *workspace,
                     size_t workspace_bytes, int64_t batch, int64_t m, int64_t n, double a,
                     hipStream_t stream) {
    if (poly == nullptr || x == nullptr || y == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    int st = reject_tall_stage(m, n);
    if (st != MUON_POLAR_OK) return st;
    Plan p{};
    st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    if (!aligned16(poly)) return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "poly must be 16-byte aligned");
    SkArea area{};
    const SkArea *ap = nullptr;
    st = stage_area(p, workspace, workspace_bytes, 2, area, ap);
    if (st != MUON_POLAR_OK) return st;
    // every output tile reads X's whole K range while other tiles write Y
    const size_t xy_bytes = static_cast<size_t>(batch * m * n * 2);
    if (overlaps(x, xy_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "x and y must not overlap");
    if (overlaps(poly, p.gram_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "poly and y must not overlap");
    if (overlaps_stage_area(p, workspace, poly, p.gram_bytes) ||
        overlaps_stage_area(p, workspace, x, xy_bytes) ||
        overlaps_stage_area(p, workspace, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                    "poly, x and y must not overlap the workspace past its A and P areas");
    const void *xs = x;
    int64_t ldx = n;
    if (ap != nullptr) {
        st = pad_input(p, workspace, x, batch, stream, xs, ldx);
        if (st != MUON_POLAR_OK) return st;
    }
    return run_apply(p, poly, xs, ldx, y, batch, m, n, a, ap, stream);
}

int muon_polar_step(const void *x, void *y, void *workspace, size_t workspace_bytes, int64_t batch,
                    int64_t m, int64_t n, double a, double b, double c, hipStream_t stream) {
    if (x == nullptr || y == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    Plan p{};
    int st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    st = check_workspace(p, workspace, workspace_bytes);
    if (st != MUON_POLAR_OK) return st;
    // The apply stage reads X's whole K range for every output tile while other
    // tiles are written to Y, and the workspace holds A, P and the padded X: an
    // in-place call (y == x), or a workspace over x or y, would race.
    if (p.tall) {
        st = check_tall(p, x, y);
        if (st != MUON_POLAR_OK) return st;
    }
    const size_t xy_bytes = static_cast<size_t>(batch * m * n * 2);
    if (overlaps(x, xy_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "x and y must not overlap");
    if (overlaps(workspace, p.workspace_bytes, x, xy_bytes) ||
        overlaps(workspace, p.workspace_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "the workspace must not overlap x or y");
    return run_step(p, x, y, workspace, batch, a, b, c, stream);
}

int muon_polar_step_noalloc(const void *x, void *y, int64_t batch, int64_t m, int64_t n,
                            double a, double b, double c, hipStream_t stream) {
    if (x == nullptr || y == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    Plan p{};
    int st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    // The two-round stream-K split's partial slots can outgrow the scratch where
    // the one-round split fits ([2,4096,4096]: 259 against 143 MiB).
    if (p.workspace_bytes > muon_polar::kNoAllocScratchBytes) {
        st = get_plan(batch, m, n, p, true);
        if (st != MUON_POLAR_OK) return st;
    }
    if (p.workspace_bytes > muon_polar::kNoAllocScratchBytes)
        return fail(MUON_POLAR_ERR_WORKSPACE,
                    "this shape needs " + std::to_string(p.workspace_bytes) +
                        " bytes of scratch; muon_polar_step_noalloc holds " +
                        std::to_string(muon_polar::kNoAllocScratchBytes) +
                        " per device (call muon_polar_step with a workspace)");
    if (p.tall) {
        st = check_tall(p, x, y);
        if (st != MUON_POLAR_OK) return st;
    }
    const size_t xy_bytes = static_cast<size_t>(batch * m * n * 2);
    if (overlaps(x, xy_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "x and y must not overlap");
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        return fail(MUON_POLAR_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    void *scratch = nullptr;
    e = muon_polar::noalloc_scratch(device, &scratch);
    if (e != hipSuccess)
        return fail(MUON_POLAR_ERR_HIP,
                    std::string("scratch address (hipGetSymbolAddress): ") + hipGetErrorString(e));
    return run_step(p, x, y, scratch, batch, a, b, c, stream);
}

int muon_polar_express(const void *x, void *y, void *workspace, size_t workspace_bytes,
                       int64_t batch, int64_t m, int64_t n, const double *coefficients,
                       int64_t steps, int normalize, hipStream_t stream) {
    if (x == nullptr || y == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    if (steps < 0 || (steps == 0 && !normalize))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "steps must be >= 1 (or 0 with normalize)");
    if (steps > 0 && coefficients == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "coefficients is null");
    Plan p{};
    int st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    if (workspace == nullptr || workspace_bytes < p.express_workspace_bytes)
        return fail(MUON_POLAR_ERR_WORKSPACE,
                    "workspace must hold " + std::to_string(p.express_workspace_bytes) +
                        " bytes, got " + std::to_string(workspace == nullptr ? 0 : workspace_bytes));
    if (!aligned16(workspace))
        return fail(MUON_POLAR_ERR_WORKSPACE, "workspace must be 16-byte aligned");
    const size_t xy_bytes = static_cast<size_t>(batch * m * n * 2);
    if (overlaps(x, xy_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "x and y must not overlap");
    // the workspace holds A, P, the iterates between y's and the norm's partial sums
    if (overlaps(workspace, p.express_workspace_bytes, x, xy_bytes) ||
        overlaps(workspace, p.express_workspace_bytes, y, xy_bytes))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "the workspace must not overlap x or y");
    if (p.tall && steps > 0) {
        st = check_tall(p, x, y);
        if (st != MUON_POLAR_OK) return st;
    }

    char *ws = static_cast<char *>(workspace);
    uint16_t *scratch = reinterpret_cast<uint16_t *>(ws + p.express_x_offset);
    float *partial = reinterpret_cast<float *>(ws + p.express_norm_offset);
    uint16_t *out = static_cast<uint16_t *>(y);
    // Buffer holding the iterate after step i (i = 0: the normalised input): the
    // iterates alternate between y and the scratch buffer so that the last one is y.
    auto iterate = [&](int64_t i) { return (steps - i) % 2 == 0 ? out : scratch; };

    const uint16_t *cur = static_cast<const uint16_t *>(x);
    if (normalize) {
        uint16_t *dst = iterate(0);
        const bool vec = (m * n) % 8 == 0 && aligned16(x) && aligned16(dst);
        st = finish_stage(muon_polar::launch_normalize(cur, dst, partial, batch, m * n, vec, stream),
                          stream, "normalize");
        if (st != MUON_POLAR_OK) return st;
        cur = dst;
    }
    return run_steps(p, workspace, cur, out, scratch, batch, coefficients, steps, stream);
}

int muon_polar_muon_update(void *param, const void *grad, void *momentum_buffer,
                           void *workspace, size_t workspace_bytes, int64_t batch, int64_t m,
                           int64_t n, double momentum, int nesterov, const double *coefficients,
                           int64_t steps, double lr, double weight_decay, double lr_scale,
                           hipStream_t stream) {
    if (param == nullptr || grad == nullptr || momentum_buffer == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    if (steps < 0) return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "steps must be >= 0");
    if (steps > 0 && coefficients == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "coefficients is null");
    if (!std::isfinite(momentum) || momentum < 0.0 || momentum > 1.0)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "momentum must be in [0, 1]");
    if (!std::isfinite(lr) || !std::isfinite(weight_decay) || !std::isfinite(lr_scale))
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "lr, weight_decay and lr_scale must be finite");
    Plan p{};
    int st = get_plan(batch, m, n, p);
    if (st != MUON_POLAR_OK) return st;
    if (workspace == nullptr || workspace_bytes < p.muon_workspace_bytes)
        return fail(MUON_POLAR_ERR_WORKSPACE,
                    "workspace must hold " + std::to_string(p.muon_workspace_bytes) +
                        " bytes, got " + std::to_string(workspace == nullptr ? 0 : workspace_bytes));
    if (!aligned16(workspace))
        return fail(MUON_POLAR_ERR_WORKSPACE, "workspace must be 16-byte aligned");
    // fp32 param, grad and buffer, and the workspace: pairwise disjoint
    const uintptr_t f32_bytes = static_cast<uintptr_t>(batch * m * n * 4);
    const uintptr_t lo[4] = {reinterpret_cast<uintptr_t>(param), reinterpret_cast<uintptr_t>(grad),
                             reinterpret_cast<uintptr_t>(momentum_buffer),
                             reinterpret_cast<uintptr_t>(workspace)};
    const uintptr_t len[4] = {f32_bytes, f32_bytes, f32_bytes,
                              static_cast<uintptr_t>(p.muon_workspace_bytes)};
    for (int i = 0; i < 4; ++i)
        for (int j = i + 1; j < 4; ++j)
            if (lo[i] < lo[j] + len[j] && lo[j] < lo[i] + len[i])
                return fail(MUON_POLAR_ERR_INVALID_ARGUMENT,
                            "param, grad, momentum_buffer and workspace must not overlap");

    char *ws = static_cast<char *>(workspace);
    uint16_t *out = reinterpret_cast<uint16_t *>(ws + p.muon_o_offset);
    uint16_t *scratch = reinterpret_cast<uint16_t *>(ws + p.express_x_offset);
    if (p.tall && steps > 0) {
        st = check_tall(p, out, scratch);
        if (st != MUON_POLAR_OK) return st;
    }
    float *partial = reinterpret_cast<float *>(ws + p.express_norm_offset);
    // The normalised input goes where the iterate chain starts (out for an even
    // step count, else scratch); the momentum pass writes the other buffer, which
    // the first step overwrites only after the normalisation has read it.
    uint16_t *first = steps % 2 == 0 ? out : scratch;
    uint16_t *x0 = steps % 2 == 0 ? scratch : out;
    const int64_t mn = m * n;
    const bool vec = mn % 8 == 0 && aligned16(grad) && aligned16(momentum_buffer);
    st = finish_stage(
        muon_polar::launch_muon_momentum(static_cast<const float *>(grad),
                                         static_cast<float *>(momentum_buffer), x0, partial, batch,
                                         mn, static_cast<float>(1.0 - momentum),
                                         static_cast<float>(momentum), nesterov != 0, vec, stream),
        stream, "momentum");
    if (st != MUON_POLAR_OK) return st;
    st = finish_stage(muon_polar::launch_norm_scale(x0, first, partial, batch, mn, mn % 8 == 0,
                                                    stream),
                      stream, "normalize");
    if (st != MUON_POLAR_OK) return st;
    st = run_steps(p, workspace, first, out, scratch, batch, coefficients, steps, stream);
    if (st != MUON_POLAR_OK) return st;
    const int64_t total = batch * mn;
    return finish_stage(
        muon_polar::launch_muon_param_update(
            static_cast<float *>(param), out, total, static_cast<float>(1.0 - lr * weight_decay),
            static_cast<float>(-lr * lr_scale), total % 8 == 0 && aligned16(param), stream),
        stream, "param update");
}

int muon_polar_check_plan(int64_t batch, int64_t m, int64_t n, int cus, const int *blocks_per_cu,
                          muon_polar_plan_extents *out) {
    if (out == nullptr || blocks_per_cu == nullptr)
        return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "null pointer");
    if (cus < 0) return fail(MUON_POLAR_ERR_INVALID_ARGUMENT, "cus must be >= 0");
    int st = check_shape(batch, m, n);
    if (st != MUON_POLAR_OK) return st;
    Knobs knobs{};
    st = read_knobs(batch, m, n, cus > 0 ? cus : 256, knobs);
    if (st != MUON_POLAR_OK) return st;
    Plan p{};
    st = build_plan(batch, m, n, knobs,
                    Target{-1, cus, {blocks_per_cu[0], blocks_per_cu[1], blocks_per_cu[2]}}, p);
    if (st != MUON_POLAR_OK) return st;
    *out = muon_polar_plan_extents{};
    out->workspace_bytes = static_cast<int64_t>(p.workspace_bytes);
    out->gram_bytes = static_cast<int64_t>(p.gram_bytes);
    out->poly_offset = static_cast<int64_t>(align256(p.gram_bytes));
    out->counters_offset = static_cast<int64_t>(p.counters_offset);
    out->counter_stride = p.counter_stride;
    out->partials_offset = static_cast<int64_t>(p.partials_offset);
    out->pad_offset = static_cast<int64_t>(p.pad_offset);
    out->pad_end = p.pad ? static_cast<int64_t>(p.pad_offset) + batch * m * p.np * 2 : 0;
    out->y_bytes = batch * m * n * 2;
    // The step's route on stand-in addresses (16-byte aligned, never dereferenced):
    // the workspace, X and Y in address ranges of their own.
    char *ws = reinterpret_cast<char *>(uintptr_t(1) << 44);
    const uintptr_t kX = uintptr_t(2) << 44, kY = uintptr_t(3) << 44;
    const void *x = reinterpret_cast<const void *>(kX);
    void *y = reinterpret_cast<void *>(kY);
    const bool pad = pad_needed(p, x);
    const void *xs = pad ? static_cast<const void *>(ws + p.pad_offset) : x;
    const int64_t ldx = pad ? p.np : n;
    void *gram = ws;
    void *poly = ws + align256(p.gram_bytes);
    StageLaunch L[3] = {p.tall ? gram_t_launch(p, xs, ldx, gram, m, n) : gram_launch(p, xs, ldx, gram, m, n),
                        poly_launch(p, gram, poly, 1.0, 1.0),
                        p.tall ? apply_r_launch(p, poly, xs, ldx, y, m, n, 1.0)
                               : apply_launch(p, poly, xs, ldx, y, m, n, 1.0)};
    for (int s = 0; s < 3; ++s) {
        SkArea area{reinterpret_cast<float *>(ws + p.partials_offset),
                    reinterpret_cast<uint64_t *>(ws + p.counters_offset) + s * p.counter_stride};
        prepare_stage(L[s], batch, p, &area, 1u);
        // extents relative to the stage's output buffer, partial area and words
        stage_extent(L[s], L[s].g.sk_units > 0, out->stage[s]);
        out->stage[s].out_limit = s == 2 ? out->y_bytes : out->gram_bytes;
        out->stage[s].partial_limit = out->pad_offset - out->partials_offset;
        out->stage[s].counter_limit = p.counter_stride;
    }
    out->chain_apply = muon_polar_stage_extent{};
    if (p.pad && !p.tall) {
        // run_steps' inner steps: X and Y both padded (the padded buffer and the
        // scratch iterate); Y's extent is the padded matrix
        StageLaunch La = apply_launch(p, poly, ws + p.pad_offset, p.np, y, m, n, 1.0, p.np);
        SkArea area{reinterpret_cast<float *>(ws + p.partials_offset),
                    reinterpret_cast<uint64_t *>(ws + p.counters_offset) + 2 * p.counter_stride};
        prepare_stage(La, batch, p, &area, 1u);
        stage_extent(La, La.g.sk_units > 0, out->chain_apply);
        out->chain_apply.out_limit = batch * m * p.np * 2;
        out->chain_apply.partial_limit = out->pad_offset - out->partials_offset;
        out->chain_apply.counter_limit = p.counter_stride;
    }
    return MUON_POLAR_OK;
}

const char *muon_polar_last_error(void) { return g_last_error.c_str(); }

const char *muon_polar_version(void) { return "0.1.1"; }

}  // extern "C"
