"""Shapes of the seeded polar_step sweep (tests/test_shape_sweep_gpu.py), shared with the
CPU plan check (tests/test_plan_extents.py), which walks each shape's launch plan before
any GPU run of it."""

from __future__ import annotations

import numpy as np


def sweep_shapes(count: int = 32, seed: int = 2026):
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(count):
        width_class = i % 4  # odd, even (not 8), multiple of 8 (not 64), multiple of 64
        short = int(rng.integers(1, 1100))
        long_ = short + int(rng.integers(0, 2400))
        if width_class == 0:
            long_ |= 1
        elif width_class == 1:
            long_ = long_ - long_ % 8 + int(rng.choice([2, 4, 6]))
        elif width_class == 2:
            long_ = max(8, long_ - long_ % 8)
            if long_ % 64 == 0:
                long_ += 8
        else:
            long_ = max(64, long_ - long_ % 64)
        long_ = max(long_, short)
        batch = int(rng.choice([1, 1, 2, 3]))
        tall = rng.random() < 0.3 and short < long_
        if tall:
            # M > N: the width class describes N (the short side, the rows' length)
            n = short if width_class != 3 else max(64, short - short % 64)
            if width_class == 0:
                n |= 1
            elif width_class == 1:
                n = max(2, n - n % 8 + 2)
            elif width_class == 2:
                n = max(8, n - n % 8)
                if n % 64 == 0:
                    n += 8
            m = max(long_, n + 1)
            shapes.append((batch, m, n))
        else:
            shapes.append((batch, short, long_))
    return shapes



def plan_shape(batch: int, m: int, n: int):
    """The (batch, m, n) the C ABI plans for: M > N with N % 8 != 0 reaches it transposed
    (the reference's wrapper route), every other shape as given."""
    return (batch, n, m) if m > n and n % 8 != 0 else (batch, m, n)


# Tuned configurations the sweep also runs (on its first ten M <= N shapes): every tile
# size, both wave counts, other ring depths, stream-K off and the register-staged family.
SWEEP_CONFIGS = {
    "tiles64_depths": {"MUON_POLAR_GRAM_TILE": "64", "MUON_POLAR_POLY_TILE": "64",
                       "MUON_POLAR_APPLY_TILE_M": "64", "MUON_POLAR_APPLY_TILE_N": "64",
                       "MUON_POLAR_GRAM_DEPTH": "8", "MUON_POLAR_POLY_DEPTH": "2",
                       "MUON_POLAR_APPLY_DEPTH": "4", "MUON_POLAR_DIAG_PAIRS": "0"},
    "tiles128": {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_POLY_TILE": "128",
                 "MUON_POLAR_APPLY_TILE_M": "128", "MUON_POLAR_APPLY_TILE_N": "128"},
    "tiles256_4waves": {"MUON_POLAR_GRAM_TILE": "256", "MUON_POLAR_POLY_TILE": "256",
                        "MUON_POLAR_APPLY_TILE_M": "256", "MUON_POLAR_APPLY_TILE_N": "256",
                        "MUON_POLAR_WAVES": "4"},
    "pairs192_unsplit": {"MUON_POLAR_GRAM_TILE": "192", "MUON_POLAR_POLY_TILE": "192",
                         "MUON_POLAR_STREAM_K": "0"},
    "register_staged": {"MUON_POLAR_STREAM": "0"},
}


def sweep_config_shapes():
    """The M <= N shapes the configurations run on."""
    return [s for s in sweep_shapes() if s[1] <= s[2]][:10]


# Configurations of the random-case sweep: the tuned ones above, the defaults, and the
# default with one of its plan features off (the two-round stream-K split, diagonal
# pairs, apply's column halves).
FUZZ_CONFIGS = dict(SWEEP_CONFIGS)
FUZZ_CONFIGS.update({
    "default": {},
    "one_round": {"MUON_POLAR_SK_ROUNDS": "0"},
    "no_pairs": {"MUON_POLAR_DIAG_PAIRS": "0"},
    "no_halves": {"MUON_POLAR_APPLY_HALVES": "0"},
})


def fuzz_cases(count: int = 160, seed: int = 777):
    """Seeded random (shape, configuration, Y offset in elements) cases: batch 1-4,
    sides up to about 4500 (at most 6M elements), all four width classes, 30% tall;
    Y at 0, 1 or 2 elements past a 16-byte boundary (only 0 for the right-Gram form,
    which needs a 16-byte aligned Y)."""
    rng = np.random.default_rng(seed)
    names = sorted(FUZZ_CONFIGS)
    cases = []
    while len(cases) < count:
        batch = int(rng.choice([1, 1, 2, 3, 4]))
        short = int(rng.integers(1, 1500))
        long_ = short + int(rng.integers(0, 3000))
        kind = int(rng.integers(0, 4))
        if kind == 0:
            long_ |= 1
        elif kind == 1:
            long_ = max(2, long_ - long_ % 8 + int(rng.choice([2, 4, 6])))
        elif kind == 2:
            long_ = max(8, long_ - long_ % 8)
        else:
            long_ = max(64, long_ - long_ % 64)
        long_ = max(long_, short)
        tall = rng.random() < 0.3 and short < long_
        m, n = (long_, short) if tall else (short, long_)
        config = names[int(rng.integers(0, len(names)))]
        offset = int(rng.choice([0, 0, 1, 2]))
        if batch * m * n > 6_000_000:
            continue
        if m > n:
            offset = 0
        cases.append(((batch, m, n), config, offset))
    return cases
