"""muon_polar_step_noalloc (the step on the library's own per-GPU scratch) against
muon_polar_step with a caller workspace, through the C ABI, bit for bit.

Calls in a row on one GPU share the scratch: the second and third calls take
smaller inputs, so stale A, P, partials and arrival words of a larger call are in
the scratch when they run.
"""

from __future__ import annotations

import pytest
import torch

from oracle import polar_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def capi():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    from muon_fusion_ascend950_amd import capi as c

    return c


def with_workspace(capi, x, coeffs):
    ws, _ = capi.alloc_workspace(*x.shape)
    y = torch.empty_like(x)
    capi.step(x, y, ws, *coeffs)
    return y


def test_noalloc_equals_workspace_entry(capi):
    # [4096,14336] first (the largest A and P in the scratch), then smaller shapes over
    # what that call left behind: [2,150,2050] cuts its gram tiles by stream-K
    # (partials and arrival words in the scratch), [3,129,257] takes the padded copy of
    # X (also in the scratch), [2,1000,136] the right-Gram form
    for shape, seed in (((1, 4096, 14336), 0), ((8, 512, 2048), 1), ((2, 150, 2050), 2),
                        ((1, 129, 130), 3), ((2, 300, 1000), 4), ((3, 129, 257), 5),
                        ((2, 1000, 136), 6)):
        print(f"noalloc {shape}", flush=True)
        x = O.make_input(shape, seed=seed).to(DEV)
        coeffs = O.COEFFICIENTS[seed % 5]
        y = torch.empty_like(x)
        capi.step_noalloc(x, y, *coeffs)
        want = with_workspace(capi, x, coeffs)
        torch.cuda.synchronize()
        assert torch.equal(y, want), shape
    # the same small call again: the scratch now holds its own previous contents
    y2 = torch.empty_like(x)
    capi.step_noalloc(x, y2, *coeffs)
    torch.cuda.synchronize()
    assert torch.equal(y2, want)


def test_noalloc_random_cases_equal_workspace_entry(capi, monkeypatch):
    """Forty of the seeded random cases (tests/sweep_shapes.py fuzz_cases) in a row on
    the one scratch, each under its configuration: every call finds the previous call's
    A, P, partials and arrival words there, of another shape and plan."""
    from tests.sweep_shapes import FUZZ_CONFIGS, fuzz_cases

    knobs = sorted({k for v in FUZZ_CONFIGS.values() for k in v})
    # the cases the C ABI takes as given (the reference wrapper transposes M > N with
    # N % 8 != 0 outside it)
    cases = [c for c in fuzz_cases() if not (c[0][1] > c[0][2] and c[0][2] % 8 != 0)][:40]
    ran = 0
    for i, ((batch, m, n), config, _offset) in enumerate(cases):
        for k in knobs:
            monkeypatch.delenv(k, raising=False)
        for k, v in FUZZ_CONFIGS[config].items():
            monkeypatch.setenv(k, v)
        print(f"noalloc random case {i}: {(batch, m, n)} {config}", flush=True)
        x = O.make_input((batch, m, n), seed=3000 + i).to(DEV)
        coeffs = O.COEFFICIENTS[i % 5]
        y = torch.empty_like(x)
        capi.step_noalloc(x, y, *coeffs)
        want = with_workspace(capi, x, coeffs)
        torch.cuda.synchronize()
        assert torch.equal(y, want), (i, (batch, m, n), config)
        ran += 1
    assert ran == 40


def test_noalloc_right_gram_form(capi):
    x = O.make_input((1, 2048, 512), seed=4).to(DEV)
    y = torch.empty_like(x)
    capi.step_noalloc(x, y, *O.COEFFICIENTS[0])
    torch.cuda.synchronize()
    assert torch.equal(y, with_workspace(capi, x, O.COEFFICIENTS[0]))


def test_noalloc_falls_back_to_the_one_round_split(capi, monkeypatch):
    """[2,4096,4096]: the default plan's two-round stream-K split needs more than the
    192 MiB scratch (its partial slots), the one-round split fits: the allocation-free
    step runs that plan, bit for bit the workspace entry with MUON_POLAR_SK_ROUNDS=0,
    and to bf16 precision the default plan."""
    from tests.test_polar_step_gpu import assert_close_kernels

    shape = (2, 4096, 4096)
    assert capi.query(*shape).workspace_bytes > 192 << 20
    print(f"noalloc fallback {shape}", flush=True)
    x = O.make_input(shape, seed=5).to(DEV)
    coeffs = O.COEFFICIENTS[0]
    y = torch.empty_like(x)
    capi.step_noalloc(x, y, *coeffs)
    default = with_workspace(capi, x, coeffs)
    monkeypatch.setenv("MUON_POLAR_SK_ROUNDS", "0")
    assert capi.query(*shape).workspace_bytes <= 192 << 20
    one_round = with_workspace(capi, x, coeffs)
    torch.cuda.synchronize()
    assert torch.equal(y, one_round)
    assert_close_kernels(y, default)


def test_noalloc_rejects_shapes_beyond_its_scratch(capi):
    """Real device tensors of a shape whose workspace exceeds the scratch: refused
    with MUON_POLAR_ERR_WORKSPACE, Y left untouched."""
    shape = (4, 4096, 4096)
    assert 2 * capi.query(*shape).gram_bytes > 192 << 20
    x = torch.zeros(shape, dtype=torch.bfloat16, device=DEV)
    y = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(capi.CapiError) as err:
        capi.step_noalloc(x, y, *O.COEFFICIENTS[0])
    assert err.value.status == capi.ERR_WORKSPACE
    assert "muon_polar_step_noalloc holds" in capi.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(y).all()


# Run in a child process (started from here as an ordinary subprocess) so that the
# library has never resolved its scratch when the captured call is made: the first
# muon_polar_step_noalloc call of that process happens under HIP graph capture.
_CAPTURE_CHILD = r"""
import json, sys
import torch
from muon_fusion_ascend950_amd import capi
from oracle import polar_oracle as O

DEV = "cuda"
MIB = 1 << 20
out = {}
cases = [((1, 4096, 14336), 0), ((8, 512, 2048), 1), ((2, 150, 2050), 2), ((1, 2048, 512), 3)]
xs, wants = [], []
for shape, seed in cases:
    x = O.make_input(shape, seed=seed).to(DEV)
    ws, _ = capi.alloc_workspace(*shape)
    want = torch.empty_like(x)
    capi.step(x, want, ws, *O.COEFFICIENTS[seed])
    xs.append(x)
    wants.append(want)
    del ws
ys = [torch.empty_like(x) for x in xs]
torch.cuda.synchronize()
torch.cuda.empty_cache()
out["free_before_first_noalloc_mib"] = torch.cuda.mem_get_info()[0] / MIB
print("child: workspace results ready; capturing the first noalloc call", flush=True)

g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    capi.step_noalloc(xs[0], ys[0], *O.COEFFICIENTS[0])
torch.cuda.synchronize()
out["free_after_capture_mib"] = torch.cuda.mem_get_info()[0] / MIB

replays = []
for r in range(3):
    ys[0].fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    replays.append(bool(torch.equal(ys[0], wants[0])))
    # eager calls of other shapes over the same scratch between replays
    for i in (1, 2, 3):
        ys[i].fill_(float("nan"))
        capi.step_noalloc(xs[i], ys[i], *O.COEFFICIENTS[cases[i][1]])
    torch.cuda.synchronize()
    replays.append(all(bool(torch.equal(ys[i], wants[i])) for i in (1, 2, 3)))
out["replays_equal"] = replays
print("child: replays checked", flush=True)

torch.cuda.synchronize()
free_a = torch.cuda.mem_get_info()[0]
for i in range(len(cases)):
    capi.step_noalloc(xs[i], ys[i], *O.COEFFICIENTS[cases[i][1]])
torch.cuda.synchronize()
free_b = torch.cuda.mem_get_info()[0]
out["free_change_over_warm_calls_bytes"] = free_a - free_b
out["warm_equal"] = all(bool(torch.equal(ys[i], wants[i])) for i in range(len(cases)))
print(json.dumps(out), flush=True)
"""


def test_noalloc_first_call_under_graph_capture_in_a_fresh_process(capi):
    """The first call a process makes is captured into a HIP graph (the scratch
    address is resolved during capture); every replay equals the workspace entry bit
    for bit, with eager calls of other shapes over the same scratch in between; warm
    calls leave the device's free memory unchanged.  Also reports when the 192 MiB
    array is committed: the free memory before the first call and after it."""
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    env = dict(os.environ)
    env["PYTHONPATH"] = str(root) + os.pathsep + env.get("PYTHONPATH", "")
    print("noalloc capture child: start", flush=True)
    proc = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_CHILD], cwd=root, env=env,
                          capture_output=True, text=True, timeout=240)
    print(proc.stdout[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    out = json.loads(proc.stdout.strip().splitlines()[-1])
    assert all(out["replays_equal"]), out
    assert out["warm_equal"], out
    assert out["free_change_over_warm_calls_bytes"] == 0, out
    committed = out["free_before_first_noalloc_mib"] - out["free_after_capture_mib"]
    print(f"noalloc scratch: {committed:.1f} MiB of free device memory taken by the first "
          f"(captured) call", flush=True)
    # the array is committed either at that call (about 192 MiB taken there) or
    # before it, with the library's other code (nothing taken there)
    assert committed < 192 + 64, out
