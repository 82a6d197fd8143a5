"""HIP-graph capture of polar_step, the op's registration checks, and gram invariants
(GPU; marked ``gpu``).

* A captured step (three stage kernels, workspace from the graph's pool) replays
  bit-identically to eager calls, replay after replay, with eager work on the same buffers
  in between (the reference never tested capture).  The stream-K arrival
  words carry a launch token: a replay reuses its captured token and finds the zero counts
  its last run left, eager launches on the same workspace in between use other tokens.
* A workspace full of garbage gives the same bits as a fresh one (no clearing needed).
* ``torch.library.opcheck``: schema and FakeTensor registration of the ops
  (reference ``_loader.py:41-48``, ``binding.cpp:679``).
* ``torch.compile`` (``aot_eager`` backend, full graph) traces the Python wrapper and the op
  through its FakeTensor registration and runs the same kernels: compiled results equal
  eager ones bit for bit, for the direct, transposing and right-Gram routes.
* Gram invariants that pin stage 1 without a reference run: ``trace(A) = ‖X‖_F²`` and
  ``diag(A) ≥ 0`` (sums of squares).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def polar_step(x, a, b, c):
    from muon_fusion_ascend950_amd import polar_step as ps

    return ps(x, a, b, c)


@pytest.mark.parametrize("shape", [(8, 512, 2048), (2, 768, 4096), (2, 150, 2050),
                                   (2, 4096, 4096)])
def test_graph_replays_match_eager(shape):
    """(2, 768, 4096) splits its gram stage (stream-K arrival words in the graph's
    workspace); (2, 150, 2050) runs the register-staged kernels; (2, 4096, 4096) splits
    gram and poly over two rounds (units over two or three tiles each)."""
    x_static = O.make_input(shape, seed=30).to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            polar_step(x_static, *C0)  # plans and allocator state before capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = polar_step(x_static, *C0)
    for r in range(4):
        x_new = O.make_input(shape, seed=31 + r).to(DEV)
        x_static.copy_(x_new)
        graph.replay()
        want = polar_step(x_new, *C0)  # eager, between replays
        torch.cuda.synchronize()
        assert torch.equal(y_static, want), f"replay {r} differs from eager"


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 1024, 4096), (8, 512, 2048),
                                   (2, 4096, 4096)])
def test_garbage_workspace_and_shared_workspace_replays(shape):
    """The C ABI step on a workspace filled with random bytes equals the step on a zeroed
    one, bit for bit; a graph that captured a step on one workspace still replays
    correctly after eager steps of other inputs ran on that same workspace."""
    from muon_fusion_ascend950_amd import capi

    batch, m, n = shape
    print(f"garbage workspace {shape}", flush=True)
    x = O.make_input(shape, seed=34).to(DEV)
    ws, info = capi.alloc_workspace(batch, m, n)
    gen = torch.Generator(device=DEV).manual_seed(35)
    ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=DEV, generator=gen))
    y_garbage = torch.empty_like(x)
    capi.step(x, y_garbage, ws, *C0)
    ws_zero = torch.zeros_like(ws)
    y_zero = torch.empty_like(x)
    capi.step(x, y_zero, ws_zero, *C0)
    torch.cuda.synchronize()
    assert torch.equal(y_garbage, y_zero)

    y_graph = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        capi.step(x, y_graph, ws, *C0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.step(x, y_graph, ws, *C0)
    other = O.make_input(shape, seed=36).to(DEV)
    y_other = torch.empty_like(x)
    for r in range(3):
        y_graph.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_zero), f"replay {r}"
        capi.step(other, y_other, ws, *C0)  # eager, same workspace, another token
        torch.cuda.synchronize()


def test_opcheck_schema_and_fake():
    x = O.make_input((2, 64, 256), seed=32).to(DEV)
    torch.library.opcheck(torch.ops.muon_ascend950.polar_step.default, (x, *C0),
                          test_utils=("test_schema", "test_faketensor"))
    xt = O.make_input((2, 256, 64), seed=33).to(DEV)
    torch.library.opcheck(torch.ops.muon_ascend950.polar_step_tall.default, (xt, *C0),
                          test_utils=("test_schema", "test_faketensor"))
    flat = [float(v) for triple in O.COEFFICIENTS[:2] for v in triple]
    torch.library.opcheck(torch.ops.muon_ascend950.polar_express.default, (x, flat, True),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("shape", [(129, 130), (130, 129), (2, 300, 1000), (1000, 64)])
def test_torch_compile_matches_eager(shape):
    """Dynamo traces polar_step (checks, the M > N policy, the op through its fake
    implementation) into one graph; the compiled call launches the same kernels."""
    import muon_ascend950
    import muon_fusion_ascend950_amd as mf

    torch._dynamo.reset()

    @torch.compile(backend="aot_eager", fullgraph=True)
    def step(x):
        return muon_ascend950.polar_step(x, *C0)

    @torch.compile(backend="aot_eager", fullgraph=True)
    def express(x):
        return mf.polar_express(x, O.COEFFICIENTS[:2])

    x = O.make_input(shape, seed=34).to(DEV)
    y = step(x)
    z = express(x)
    torch.cuda.synchronize()
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    assert torch.equal(y, muon_ascend950.polar_step(x, *C0))
    assert torch.equal(z, mf.polar_express(x, O.COEFFICIENTS[:2]))


@pytest.mark.parametrize("shape", [(2, 300, 1000), (1, 4096, 14336), (3, 1024, 8192)])
def test_gram_trace_and_diagonal(shape):
    from muon_fusion_ascend950_amd import capi

    x = O.make_input(shape, seed=33).to(DEV)
    batch, m, n = shape
    ws, info = capi.alloc_workspace(batch, m, n)
    mp = info.padded_rows
    gram = ws[:info.gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    capi.gram(x, gram, workspace=ws)
    torch.cuda.synchronize()
    diag = torch.diagonal(gram[:, :m, :m], dim1=-2, dim2=-1).float().cpu().numpy()
    assert (diag >= 0).all()
    sumsq = (x.double() ** 2).sum(dim=(-2, -1)).cpu().numpy()
    trace = diag.astype(np.float64).sum(axis=-1)
    # each diagonal entry is one bf16 rounding of an fp32 sum of squares: relative
    # error ≤ 2^-8 per entry, so the trace is within 2^-8 of ‖X‖_F² (all terms ≥ 0)
    assert np.all(np.abs(trace - sumsq) <= 2.0**-8 * sumsq)
