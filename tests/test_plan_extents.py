"""Every store the stage kernels can make stays inside its buffer (CPU only).

``muon_polar_check_plan`` builds the launch plan ``muon_polar_step`` would use on a
device of 256 CUs and walks every workgroup of each stage with the kernels' own
schedule functions (``csrc/polar_schedule.hpp``): the output tiles and mirrored
tiles it stores, the stream-K partial slots it writes or reads and its arrival
word.  These tests assert that each range lies inside the buffer it belongs to, that
the (tile, K-step) iterations are computed exactly once, and that the operands'
per-matrix byte extents fit the kernels' 32-bit buffer offsets.

The occupancy (resident workgroups per CU) decides the stream-K split; it is swept
over 1-4 per stage, which covers what the device reports for every kernel.
"""

from __future__ import annotations

import pytest

from muon_fusion_ascend950_amd import capi
from tests.sweep_shapes import (FUZZ_CONFIGS, SWEEP_CONFIGS, fuzz_cases, plan_shape,
                                 sweep_config_shapes, sweep_shapes)

BASELINE_SHAPES = [(4, 4096, 4096), (1, 4096, 14336), (1, 14336, 4096), (8, 512, 2048),
                   (2, 150, 2050), (1, 129, 130)]
MORE_SHAPES = [(3, 1024, 4096), (16, 256, 1024), (1, 1000, 3000), (2, 700, 1800), (1, 3000, 1000),
               (1, 8192, 16384), (2, 6144, 8192), (4000, 16, 40), (1, 64, 100000), (1, 2048, 520),
               (1, 8, 131072), (1, 65536, 8), (2, 3, 40000), (1, 128, 65536)]
OCCUPANCIES = [(1, 1, 1), (2, 2, 2), (1, 2, 2), (2, 1, 1), (3, 3, 3), (4, 4, 4)]


def check(plan: capi.PlanExtents) -> None:
    assert plan.poly_offset >= plan.gram_bytes
    assert plan.counters_offset >= plan.poly_offset + plan.gram_bytes
    assert plan.partials_offset >= plan.counters_offset + 3 * plan.counter_stride * 8
    assert plan.pad_offset >= plan.partials_offset
    assert plan.pad_end <= plan.workspace_bytes
    # rows of n % 8 != 0 elements (a padded buffer in the workspace): a chain's inner
    # steps write their iterate padded
    chained = plan.chain_apply.total_tiles > 0
    assert plan.pad_end > 0 or not chained
    extents = [(s, plan.stage[s]) for s in range(3)] + ([(2, plan.chain_apply)] if chained else [])
    for s, e in extents:
        assert e.coverage_ok == 1, f"stage {s}: an iteration is not computed exactly once"
        assert e.extents_ok == 1, f"stage {s}: an operand extent does not fit 32-bit offsets"
        assert 0 <= e.out_lo <= e.out_hi <= e.out_limit, (
            f"stage {s}: stores [{e.out_lo}, {e.out_hi}) outside an output of {e.out_limit} bytes")
        if e.halves:
            # apply's last round as column halves: whole K per half, nothing shared
            assert s == 2 and e.dma_fed == 1 and (e.tile_m, e.tile_n, e.waves) == (256, 256, 8)
            assert e.sk_units == 2 * (e.total_tiles - e.dp_tiles) > 0
            assert e.partial_hi == 0 and e.counter_hi == 0
        elif e.sk_units > 0:
            assert e.dma_fed == 1
            assert 0 <= e.partial_lo < e.partial_hi <= e.partial_limit, (
                f"stage {s}: partial slots [{e.partial_lo}, {e.partial_hi}) outside "
                f"{e.partial_limit} bytes")
            assert 0 < e.counter_hi <= e.counter_limit
            # partial offsets are 32-bit in the kernel
            assert e.partial_hi < 2**31
        else:
            assert e.partial_hi == 0 and e.counter_hi == 0
        if e.diag_pairs:
            # off-diagonal tiles and pairs of diagonal tiles, never cut
            assert s < 2 and e.dma_fed == 1 and (e.tile_m, e.tile_n, e.waves) == (64, 64, 4)
            assert e.sk_units == 0 and e.dp_tiles == e.total_tiles


@pytest.mark.parametrize("shape", [(3, 129, 257), (2, 150, 2049), (1, 1000, 3001), (4, 64, 8191),
                                   (2, 150, 2050), (1, 129, 130), (3, 200, 1002)])
def test_padded_chain_apply_writes_the_whole_padded_iterate(shape):
    """n % 8 != 0 (odd and even): the apply of a chain's inner steps stores every column
    of the padded iterate (its padded columns come out zero, the next step's padding) and
    nothing past it, while the step's own apply stores up to column n."""
    batch, m, n = shape
    np_ = -(-n // 64) * 64
    for occ in [(1, 1, 1), (2, 2, 2)]:
        plan = capi.check_plan(*shape, cus=256, blocks_per_cu=occ)
        check(plan)
        assert plan.pad_end > 0 and plan.chain_apply.total_tiles > 0
        assert plan.chain_apply.out_limit == batch * m * np_ * 2
        assert plan.chain_apply.out_hi == batch * m * np_ * 2
        assert plan.stage[2].out_hi == plan.y_bytes


@pytest.mark.parametrize("occ", OCCUPANCIES)
@pytest.mark.parametrize("shape", BASELINE_SHAPES)
def test_baseline_plans_store_inside_their_buffers(shape, occ):
    check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


@pytest.mark.parametrize("occ", [(1, 1, 1), (2, 2, 2)])
@pytest.mark.parametrize("shape", MORE_SHAPES)
def test_other_plans_store_inside_their_buffers(shape, occ):
    check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


@pytest.mark.parametrize("occ", [(1, 1, 1), (2, 2, 2)])
@pytest.mark.parametrize("shape", sweep_shapes())
def test_sweep_plans_store_inside_their_buffers(shape, occ):
    """The shapes of the GPU sweep (tests/test_shape_sweep_gpu.py), checked here first."""
    check(capi.check_plan(*plan_shape(*shape), cus=256, blocks_per_cu=occ))


@pytest.mark.parametrize("config", sorted(SWEEP_CONFIGS))
@pytest.mark.parametrize("shape", sweep_config_shapes())
def test_sweep_configuration_plans_store_inside_their_buffers(monkeypatch, shape, config):
    """The tuned configurations of the GPU sweep, checked here first."""
    for k, v in SWEEP_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    for occ in [(1, 1, 1), (2, 2, 2)]:
        check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


def test_random_case_plans_store_inside_their_buffers(monkeypatch):
    """Every case of the GPU's random-case sweep, under its configuration, at every
    occupancy, checked here first."""
    for shape, config, _offset in fuzz_cases():
        for k in {k for v in FUZZ_CONFIGS.values() for k in v}:
            monkeypatch.delenv(k, raising=False)
        for k, v in FUZZ_CONFIGS[config].items():
            monkeypatch.setenv(k, v)
        for occ in OCCUPANCIES:
            check(capi.check_plan(*plan_shape(*shape), cus=256, blocks_per_cu=occ))


@pytest.mark.parametrize("shape,units", [((1, 8, 131072), 32), ((1, 64, 100000), 24),
                                         ((1, 65536, 8), 16), ((1, 128, 65536), 48)])
def test_long_k_over_few_tiles_is_cut_into_many_shares(shape, units):
    """A gram stage of a few 64x64 tiles with a long K loop is cut into shares of about
    64 K-steps (up to 32 per tile), where the default pieces (at most four per tile)
    would leave it to a few workgroups or, for one tile, to one."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    gram = plan.stage[0]
    assert gram.tile_m == 64 and gram.dp_tiles == 0 and gram.sk_units == units
    assert gram.k_steps * gram.total_tiles / gram.sk_units >= 60  # shares of about 64 K-steps


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 14336, 4096)])
def test_headline_plan(shape):
    """At [4096,14336] and in the right-Gram form at [14336,4096], with one
    workgroup per CU: gram and poly run one round of 192x192 tiles (253 on 256
    CUs, 8-wave wave-pair kernels, three ring slots), so A and P are padded to
    4224 rows; apply runs three rounds of whole 256x256 tiles and its last 128
    tiles as 256 column halves (no stream-K partials anywhere)."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    apply = plan.stage[2]
    assert (apply.tile_m, apply.tile_n, apply.waves) == (256, 256, 8)
    assert apply.total_tiles == 896 and apply.dp_tiles == 768
    assert apply.halves == 1 and apply.sk_units == 256
    for s in (0, 1):
        e = plan.stage[s]
        assert (e.tile_m, e.tile_n, e.waves, e.depth, e.total_tiles, e.sk_units) == (
            192, 192, 8, 3, 253, 0)
    # A reaches its last byte: gram's last tile row ends at the padded extent
    assert plan.stage[0].out_hi == plan.stage[0].out_limit == 4224 * 4224 * 2
    assert plan.partials_offset == plan.pad_offset  # no partial slots


@pytest.mark.parametrize("gram,poly", [(256, 192), (192, 256), (64, 192), (192, 128), (128, 64)])
@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 300, 1000), (3, 136, 200), (1, 1000, 3000)])
def test_unequal_symmetric_tiles_store_inside_their_buffers(monkeypatch, gram, poly, shape):
    """A and P are padded to the larger of the two stages' tile extents; the stage
    with the smaller one also writes zeros up to it, inside the buffer."""
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", str(gram))
    monkeypatch.setenv("MUON_POLAR_POLY_TILE", str(poly))
    s = min(shape[1:])
    mp = max(-(-s // gram) * gram, -(-s // poly) * poly)
    assert capi.query(*shape).padded_rows == mp
    for occ in [(1, 1, 1), (2, 2, 2)]:
        check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


@pytest.mark.parametrize("env", [{"MUON_POLAR_WAVES": "4"},
                                 {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_POLY_TILE": "128"},
                                 {"MUON_POLAR_GRAM_TILE": "192", "MUON_POLAR_POLY_TILE": "192"},
                                 {"MUON_POLAR_APPLY_TILE_M": "128", "MUON_POLAR_APPLY_TILE_N": "256"},
                                 {"MUON_POLAR_APPLY_TILE_M": "256", "MUON_POLAR_APPLY_TILE_N": "128"},
                                 {"MUON_POLAR_SYM_GROUP": "1"}, {"MUON_POLAR_APPLY_GROUP_N": "3"},
                                 {"MUON_POLAR_STREAM": "0"}])
@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 700, 1800), (8, 512, 2048)])
def test_tuned_plans_store_inside_their_buffers(monkeypatch, env, shape):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for occ in [(1, 1, 1), (2, 2, 2)]:
        check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


def test_without_a_device_count_nothing_splits():
    plan = capi.check_plan(1, 4096, 14336, cus=0, blocks_per_cu=(1, 1, 1))
    check(plan)
    assert all(plan.stage[s].sk_units == 0 for s in range(3))


@pytest.mark.parametrize("shape", [(1, 32512, 33025), (1, 16_000_000, 66), (1, 4_000_000, 260)])
def test_padded_copy_beyond_32_bit_offsets_is_rejected(shape):
    """Rows of n % 8 != 0 elements go through a copy padded to a multiple of 64
    columns.  X fits 32-bit offsets here but that copy would not (2.15-2.56 GB): the
    out-of-range marker of the DMA (offset 2^31) would then address real rows.  Such
    shapes are rejected."""
    with pytest.raises(capi.CapiError, match="too large") as err:
        capi.query(*shape)
    assert err.value.status == capi.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("shape", [(1, 10_000_000, 72), (1, 20_000_000, 8), (2, 300, 1000),
                                   (1, 1000, 3000), (3, 523, 200)])
def test_rows_of_whole_chunks_are_read_in_place(shape):
    """n % 8 == 0: X is read in place (a last K-step past n is masked in the
    kernels), so the plan holds no padded copy and such tall shapes, whose copy
    padded to 64 columns would pass 2^30 elements, are accepted."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    assert plan.pad_end == 0
    check(plan)


def _random_shapes(count: int, seed: int):
    import numpy as np

    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        b = int(rng.integers(1, 17))
        short = int(rng.integers(1, 4097))
        long = int(rng.integers(short, 16385))
        out.append((b, short, long) if rng.random() < 0.6 else (b, long, short))
    return out


@pytest.mark.parametrize("shape", _random_shapes(200, seed=7), ids=lambda s: "x".join(map(str, s)))
def test_random_plans_store_inside_their_buffers(shape):
    """Seeded random shapes (batch 1-16, sides up to 16384, wide and tall): every
    stage's walk stays inside its buffers and computes each iteration once, at the
    occupancies the kernels can report."""
    for occ in [(1, 1, 1), (2, 2, 2), (1, 2, 2)]:
        check(capi.check_plan(*shape, cus=256, blocks_per_cu=occ))


def _units(nt: int) -> int:
    return nt * (nt - 1) // 2 + (nt + 1) // 2


@pytest.mark.parametrize("shape", [(8, 512, 2048), (8, 2048, 512), (10, 440, 1024),
                                   (10, 1024, 440), (10, 448, 1024)])
@pytest.mark.parametrize("occ", [(1, 1, 1), (2, 2, 2)])
def test_diagonal_pairs_cover_every_upper_tile_once(shape, occ):
    """Where pairing the diagonal 64x64 tiles takes fewer rounds of one workgroup per
    CU (288 tiles -> 256 units at [8,512,2048]; 7 tiles a side leave a last diagonal
    tile alone), gram and poly run off-diagonal tiles and diagonal pairs, unsplit.
    The walk checks that every upper tile of every matrix is started by exactly one
    workgroup and that the stores of both tiles of a pair stay inside A and P."""
    batch, m, n = shape
    nt = -(-min(m, n) // 64)
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=occ)
    check(plan)
    for s in (0, 1):
        e = plan.stage[s]
        assert e.diag_pairs == 1
        assert e.total_tiles == batch * _units(nt) <= 256
        assert e.grid == 8 * -(-e.total_tiles // 8)


@pytest.mark.parametrize("shape", [(8, 512, 2048), (10, 440, 1024)])
def test_diagonal_pairs_switch(monkeypatch, shape):
    """MUON_POLAR_DIAG_PAIRS=0: every upper tile a unit of its own again."""
    monkeypatch.setenv("MUON_POLAR_DIAG_PAIRS", "0")
    batch, m, n = shape
    nt = -(-min(m, n) // 64)
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(2, 2, 2))
    check(plan)
    for s in (0, 1):
        assert plan.stage[s].diag_pairs == 0
        assert plan.stage[s].total_tiles == batch * nt * (nt + 1) // 2


@pytest.mark.parametrize("shape", [(4, 512, 4096), (16, 256, 1024), (3, 1024, 4096)])
def test_no_diagonal_pairs_where_rounds_stay_the_same(shape):
    """Shapes whose units would take as many rounds as their tiles keep every tile."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(2, 2, 2))
    check(plan)
    assert plan.stage[0].diag_pairs == 0 and plan.stage[1].diag_pairs == 0


@pytest.mark.parametrize("shape", [(2, 2048, 4352), (1, 3000, 6000), (2, 4352, 2048),
                                   (1, 6000, 3000), (1, 2560, 7000)])
def test_short_last_round_runs_as_halves(shape):
    """Apply's 256x256 tiles with a last round stream-K leaves whole (shares under 20
    K-steps): that round runs as 256x128 halves, no partials, every tile covered."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(2, 2, 1))
    check(plan)
    e = plan.stage[2]
    assert e.halves == 1 and (e.tile_m, e.tile_n, e.waves) == (256, 256, 8)
    assert e.dp_tiles == e.total_tiles - e.total_tiles % 256
    assert e.sk_units == 2 * (e.total_tiles % 256) > 0


@pytest.mark.parametrize("shape", [(4, 1344, 6000), (4, 1496, 34240), (4, 1344, 20000)])
def test_long_k_gram_takes_256_tiles_from_1281(shape):
    """A gram of 80+ K-steps on A sides above 1280 takes 256x256 tiles cut by stream-K
    when those tiles number a quarter of the CUs (4 x 21 = 84 here): every iteration
    covered once, partial slots and arrival words inside the workspace."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    e = plan.stage[0]
    assert (e.tile_m, e.tile_n, e.waves) == (256, 256, 8)
    assert e.k_steps >= 80 and e.total_tiles == 4 * 21 and e.sk_units > 0


@pytest.mark.parametrize("shape", [(1, 1504, 10000), (1, 12352, 1536), (1, 10000, 1504)])
def test_long_k_gram_takes_128_tiles_where_64_units_outnumber_the_cus(shape):
    """A gram of 128+ K-steps whose 64x64 units (diagonal pairs counted) outnumber the
    CUs (300 > 256 at A side 1504-1536) takes 128x128 tiles cut by stream-K, in the
    wide form and in the right-Gram form (X columns as K)."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    e = plan.stage[0]
    assert (e.tile_m, e.tile_n) == (128, 128)
    assert e.k_steps >= 128 and e.dp_tiles == 0 and e.sk_units > e.total_tiles


@pytest.mark.parametrize("shape,rem", [((4, 4096, 4096), 32), ((2, 4096, 8192), 16),
                                       ((1, 8192, 16384), 16), ((8, 4096, 4096), 64)])
def test_short_last_round_splits_with_the_round_before(shape, rem):
    """256x256 gram and poly tiles whose last round is at most a third of the CUs: the
    split covers that round and the whole round before it, one unit per CU (most cut
    tiles then have two contributors); MUON_POLAR_SK_ROUNDS=0 keeps the one-round split
    of three pieces per tile."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    for s in (0, 1):
        e = plan.stage[s]
        assert (e.tile_m, e.tile_n) == (256, 256)
        assert e.total_tiles % 256 == rem
        assert e.dp_tiles == e.total_tiles - rem - 256 and e.sk_units == 256


def test_one_round_split_without_the_extra_round(monkeypatch):
    monkeypatch.setenv("MUON_POLAR_SK_ROUNDS", "0")
    plan = capi.check_plan(4, 4096, 4096, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    for s in (0, 1):
        e = plan.stage[s]
        assert e.dp_tiles == 512 and e.sk_units == 96


def test_long_last_round_keeps_the_one_round_split():
    """[3,4096,4096]: 152 tiles in the last round (over a third of the CUs)."""
    plan = capi.check_plan(3, 4096, 4096, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    for s in (0, 1):
        assert plan.stage[s].dp_tiles == 256 and plan.stage[s].sk_units == 256


def test_sk_rounds_rejects_a_bad_mask(monkeypatch):
    monkeypatch.setenv("MUON_POLAR_SK_ROUNDS", "8")
    with pytest.raises(capi.CapiError):
        capi.check_plan(4, 4096, 4096, cus=256)


@pytest.mark.parametrize("shape,rem", [((1, 5120, 13312), 16), ((1, 4096, 17408), 64)])
def test_apply_short_last_round_splits_with_the_round_before(shape, rem):
    """Apply's 256x256 tiles with a short last round that the column halves do not
    take (at most a quarter of the CUs as halves): the two-round split."""
    plan = capi.check_plan(*shape, cus=256, blocks_per_cu=(1, 1, 1))
    check(plan)
    e = plan.stage[2]
    assert e.halves == 0 and (e.tile_m, e.tile_n) == (256, 256)
    assert e.total_tiles % 256 == rem
    assert e.dp_tiles == e.total_tiles - rem - 256 and e.sk_units == 256
