"""bench.py's host-side contract (CPU): the credited-FLOP count the metric divides by, the
configuration list, the input recipe, the committed traffic figure it reports, and the
refusal of more than one GPU.

* credited FLOPs: the BASELINE.json north star counts M²N + 2M³ + 2M²N per matrix with
  M ≤ N after the wrapper transpose; checked against hand-computed values at the headline
  and batched shapes, and for the transposed shape.
* CONFIGS: every BASELINE.json configuration, one and five steps where it asks for both.
* make_input: seeded N(0,1) bf16, each matrix scaled to Frobenius norm just under 1
  (x / (‖x‖_F·1.01 + 1e-6), reference tests/test_polar_step.py:38-39).
* read_traffic: the bytes per apply launch that profiles/apply_4096x14336_hbm_traffic.txt
  states.
* --gpus 2 (or WORLD_SIZE 2) exits with status 2 and says why, before touching a GPU.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_credited_flops_hand_values():
    # [4096,14336]: 4096²·14336 + 2·4096³ + 2·4096²·14336 = 858 993 459 200
    assert bench.credited_flops(1, 4096, 14336) == 858_993_459_200
    # M > N counts the transposed problem
    assert bench.credited_flops(1, 14336, 4096) == 858_993_459_200
    # [8,512,2048]: 8 · (512²·2048 + 2·512³ + 2·512²·2048) = 15 032 385 536
    assert bench.credited_flops(8, 512, 2048) == 15_032_385_536
    # [4,4096,4096]: 4 · 5·4096³
    assert bench.credited_flops(4, 4096, 4096) == 4 * 5 * 4096**3
    # the formula term by term at a small odd shape
    m, n = 3, 7
    assert bench.credited_flops(2, m, n) == 2 * (m * m * n + 2 * m**3 + 2 * m * m * n)


def test_configs_cover_baseline():
    got = {(name, tuple(shape), steps) for name, shape, steps in bench.CONFIGS}
    want = {
        ("cfg0", (129, 130), 1),
        ("cfg1", (2, 150, 2050), 1),
        ("cfg2", (8, 512, 2048), 1),
        ("cfg3", (8, 512, 2048), 5),
        ("cfg4", (4096, 14336), 1), ("cfg4", (4096, 14336), 5),
        ("cfg4", (14336, 4096), 1), ("cfg4", (14336, 4096), 5),
        ("cfg4", (4, 4096, 4096), 1), ("cfg4", (4, 4096, 4096), 5),
    }
    assert got == want
    assert bench.HEADLINE == (1, 4096, 14336) and bench.SECONDARY == (8, 512, 2048)


def test_make_input_recipe():
    x = bench.make_input((3, 40, 70), seed=7)
    assert x.dtype == torch.bfloat16 and x.shape == (3, 40, 70)
    norms = x.float().norm(dim=(-2, -1))
    # bf16 rounding of each entry moves the norm by at most ~2^-8 relative
    assert torch.all((norms - 1 / 1.01).abs() < 1e-2)
    assert torch.equal(x, bench.make_input((3, 40, 70), seed=7))
    assert not torch.equal(x, bench.make_input((3, 40, 70), seed=8))


def test_read_traffic_matches_profile():
    text = (ROOT / "profiles" / "apply_4096x14336_hbm_traffic.txt").read_text()
    line = [ln for ln in text.splitlines() if ln.startswith("traffic_bytes_per_launch:")]
    assert len(line) == 1
    assert bench.read_traffic() == pytest.approx(float(line[0].split(":")[1]))
    # at least the algorithmic bytes of the launch (P, X and Y once each)
    assert bench.read_traffic() >= 4096 * 4096 * 2 + 2 * 4096 * 14336 * 2


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args],
                       env={**os.environ, **env}, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "single-GPU" in r.stderr


def test_bench_formula_is_the_reference_formula():
    """bench.py's own restatement of tests/test_polar_step.py:22-28 (used for its accuracy
    gates and the PyTorch-eager comparison point) equals the oracle's, step by step."""
    from oracle import polar_oracle as O

    x = bench.make_input((2, 24, 40), seed=3).float()
    coeffs = O.COEFFICIENTS[:3]
    assert torch.allclose(bench.torch_formula(x, coeffs), O.reference_formula_torch(x, coeffs),
                          rtol=0, atol=1e-6)


def test_accuracy_gate_reports_relf():
    x = bench.make_input((1, 32, 64), seed=4)
    y = bench.torch_formula(x.float(), [bench.COEFFS]).bfloat16()
    good = bench.accuracy(y, x, [bench.COEFFS])
    assert good["gate_6e-2"] == "pass" and good["relF_vs_fp32_formula"] < 1e-2
    # the all-zero output passes the 6e-2 gate at these magnitudes; relF exposes it
    zero = bench.accuracy(torch.zeros_like(y), x, [bench.COEFFS])
    assert zero["relF_vs_fp32_formula"] == pytest.approx(1.0)


def test_cpu_info_fields():
    info = bench.cpu_info()
    assert set(info) == {"cpu_model", "isa_flags"} and isinstance(info["isa_flags"], list)
