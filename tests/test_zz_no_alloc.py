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
    # [4096,14336]: every stage cuts its last round (partials and arrival words in
    # the scratch); then smaller shapes over the scratch that call left behind
    for shape, seed in (((1, 4096, 14336), 0), ((8, 512, 2048), 1), ((2, 150, 2050), 2),
                        ((1, 129, 130), 3), ((2, 300, 1000), 4)):
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
    info = capi.query(4, 4096, 4096)
    assert info.workspace_bytes > 192 << 20
    lib = capi.load()
    # never dereferenced: the size check fails before any launch
    st = lib.muon_polar_step_noalloc(1 << 20, 1 << 40, 4, 4096, 4096, 1.0, 1.0, 1.0, None)
    assert st == capi.ERR_WORKSPACE
    assert "muon_polar_step_noalloc holds" in capi.last_error()
