"""Muon update on the GPU (marked ``gpu``): ``muon_update`` / ``Muon`` against the oracle.

The update is element-wise fp32 work around the Polar Express iteration, so it is
checked bit for bit where the arithmetic is fixed:

* the momentum buffer equals the oracle's ``muon_momentum`` (torch.lerp's two-branch
  form, every operation rounded on its own);
* the orthogonalised direction O equals ``polar_express`` (normalise + steps) of the
  oracle's bf16 iteration input, run on the GPU: the momentum pass sums the squares for
  the normalisation in the normalisation pass's own order;
* the parameter equals the oracle's ``muon_param_update`` of that O;

and O itself matches the oracle's rounding-point emulation to the iteration's precision.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
# wide, batch, tall with N % 8 == 0 (right-Gram), ragged (scalar element paths), tall
# with N % 8 != 0 (transposed route), headline parameter shape
# partial sums of squares over chunks of 4096 elements (the small shapes), 8192 with a
# 16-element last chunk ([4100,4100]) and 16384 ([4096,14336]); m·n not a multiple of 8
# ([3,150,2050], [2,129,257]: the momentum pass's element-wise path); odd width
# ([2,129,257]: the padded copy of X in every step)
SHAPES = [(1, 512, 2048), (2, 300, 1000), (1, 2048, 512), (3, 150, 2050), (1, 520, 130),
          (2, 129, 257), (1, 4100, 4100), (1, 4096, 14336)]


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def f32_bits(a) -> np.ndarray:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_f32_equal(got, want, what):
    # both sides of a comparison can come from the GPU (O from polar_express): equal
    # NaNs would pass a bit comparison, so the values must be finite too
    assert np.isfinite(f32_bits(want).view(np.float32)).all(), f"{what}: non-finite values"
    gb, wb = f32_bits(got).ravel(), f32_bits(want).ravel()
    bad = np.flatnonzero(gb != wb)
    assert bad.size == 0, f"{what}: {bad.size} of {gb.size} differ, first at {bad[0]}"


def state(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    p = torch.randn(shape, generator=gen) * 0.02
    g = torch.randn(shape, generator=gen) * 1e-3
    buf = torch.randn(shape, generator=gen) * 1e-3
    return p, g, buf


@pytest.mark.parametrize("nesterov,wd", [(True, 0.0), (False, 0.1)])
@pytest.mark.parametrize("shape", SHAPES)
def test_update_chain_is_bitwise(shape, nesterov, wd):
    from muon_fusion_ascend950_amd import muon_update, polar_express
    from muon_fusion_ascend950_amd.optim import default_lr_scale

    print(f"muon update {shape} nesterov={nesterov} wd={wd}", flush=True)
    p, g, buf = state(shape, seed=51)
    lr, beta = 0.05, 0.95
    p_d, g_d, buf_d = p.to(DEV), g.to(DEV), buf.to(DEV)
    muon_update(p_d, g_d, buf_d, lr=lr, momentum=beta, nesterov=nesterov, weight_decay=wd)
    torch.cuda.synchronize()

    new_buf, u = O.muon_momentum(g.numpy(), buf.numpy(), beta, nesterov)
    assert_f32_equal(buf_d, new_buf, "momentum buffer")
    assert torch.equal(g_d.cpu(), g)  # grad is read only
    x0 = torch.from_numpy(u).to(torch.bfloat16).to(DEV)
    o = polar_express(x0)
    torch.cuda.synchronize()
    scale = default_lr_scale(shape[-2], shape[-1])
    want_p = O.muon_param_update(p.numpy(), o.float().cpu().numpy(), lr, wd, scale)
    assert_f32_equal(p_d, want_p, "param")


def _random_muon_cases():
    from tests.sweep_shapes import fuzz_cases

    return [c for c in fuzz_cases()[40:70]]


@pytest.mark.parametrize("case", _random_muon_cases(),
                         ids=[f"{b}x{m}x{n}-{c}" for (b, m, n), c, _ in _random_muon_cases()])
def test_random_case_update_chain_is_bitwise(monkeypatch, case):
    """Thirty of the seeded random cases (tests/sweep_shapes.py fuzz_cases), each under
    its configuration: the momentum buffer bit-exact against the oracle, the parameter
    bit-exact against the oracle's parameter pass over polar_express of the oracle's bf16
    input."""
    from muon_fusion_ascend950_amd import muon_update, polar_express
    from muon_fusion_ascend950_amd.optim import default_lr_scale
    from tests.sweep_shapes import FUZZ_CONFIGS

    shape, config, _offset = case
    for k in {k for v in FUZZ_CONFIGS.values() for k in v}:
        monkeypatch.delenv(k, raising=False)
    for k, v in FUZZ_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    print(f"muon random case {shape} {config}", flush=True)
    p, g, buf = state(shape, seed=53)
    lr, beta = 0.05, 0.9
    p_d, g_d, buf_d = p.to(DEV), g.to(DEV), buf.to(DEV)
    muon_update(p_d, g_d, buf_d, lr=lr, momentum=beta, nesterov=True, weight_decay=0.01)
    torch.cuda.synchronize()
    new_buf, u = O.muon_momentum(g.numpy(), buf.numpy(), beta, True)
    assert_f32_equal(buf_d, new_buf, "momentum buffer")
    o = polar_express(torch.from_numpy(u).to(torch.bfloat16).to(DEV))
    torch.cuda.synchronize()
    scale = default_lr_scale(shape[-2], shape[-1])
    want_p = O.muon_param_update(p.numpy(), o.float().cpu().numpy(), lr, 0.01, scale)
    assert_f32_equal(p_d, want_p, "param")


@pytest.mark.parametrize("shape", [(2, 300, 1000), (1, 2048, 512), (1, 520, 130)])
def test_direction_matches_oracle(shape):
    """O from the parameter change against the oracle's whole update (float64 sums,
    the kernels' rounding points): normwise to the five-step precision."""
    from muon_fusion_ascend950_amd import muon_update
    from muon_fusion_ascend950_amd.optim import default_lr_scale

    _, g, buf = state(shape, seed=52)
    lr = 0.05
    p_d = torch.zeros(shape, device=DEV)
    muon_update(p_d, g.to(DEV), buf.to(DEV), lr=lr)
    torch.cuda.synchronize()
    scale = default_lr_scale(shape[-2], shape[-1])
    _, _, o_ref = O.muon_update_fused(np.zeros(shape, np.float32), g.numpy(), buf.numpy(), 0.95,
                                      True, O.COEFFICIENTS, lr, 0.0, scale)
    o_got = -p_d.cpu().numpy().astype(np.float64) / np.float64(np.float32(lr * scale))
    assert O.rel_frobenius(o_got, o_ref) <= 2e-2
    # Polar Express drives every singular value of O towards 1
    s = np.linalg.svd(o_got[0], compute_uv=False)
    assert np.all(np.abs(s - 1.0) < 0.35)


def test_optimizer_steps_match_the_oracle_loop():
    """Muon over several steps on a 2-D, a 3-D (stacked) and a tall unaligned matrix
    parameter: buffers bit for bit, parameters to the iteration's precision."""
    from muon_fusion_ascend950_amd import Muon
    from muon_fusion_ascend950_amd.optim import default_lr_scale

    shapes = [(256, 512), (3, 64, 128), (200, 36)]
    gen = torch.Generator().manual_seed(53)
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(DEV)) for s in shapes]
    grads = [[torch.randn(s, generator=gen) * 1e-3 for s in shapes] for _ in range(3)]
    start = [p.detach().cpu().numpy().astype(np.float64) for p in params]
    ref_p = [p.detach().cpu().numpy().copy() for p in params]
    ref_b = [np.zeros(s, np.float32) for s in shapes]
    opt = Muon(params, lr=0.03, momentum=0.9, weight_decay=0.05)
    for step_grads in grads:
        for p, gr in zip(params, step_grads):
            p.grad = gr.to(DEV)
        opt.step()
        for i, (s, gr) in enumerate(zip(shapes, step_grads)):
            ref_p[i], ref_b[i], _ = O.muon_update_fused(
                ref_p[i], gr.numpy(), ref_b[i], 0.9, True, O.COEFFICIENTS, 0.03, 0.05,
                default_lr_scale(s[-2], s[-1]))
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        assert_f32_equal(opt.state[p]["momentum_buffer"], ref_b[i], f"buffer {shapes[i]}")
        moved = p.detach().cpu().numpy().astype(np.float64) - start[i]
        assert O.rel_frobenius(moved, ref_p[i].astype(np.float64) - start[i]) <= 3e-2


def test_non_contiguous_and_bf16_grad():
    from muon_fusion_ascend950_amd import muon_update

    p, g, buf = state((1, 300, 1000), seed=54)
    p1, b1 = p[0].to(DEV), buf[0].to(DEV)
    muon_update(p1, g[0].to(DEV).bfloat16().float(), b1, lr=0.05)
    # the same values in column-major storage
    p2 = p[0].T.contiguous().to(DEV).T
    b2 = buf[0].T.contiguous().to(DEV).T
    assert not p2.is_contiguous()
    muon_update(p2, g[0].to(DEV).bfloat16(), b2, lr=0.05)
    torch.cuda.synchronize()
    assert torch.equal(p1, p2) and torch.equal(b1, b2)


def test_rejects_wrong_dtypes_on_gpu():
    from muon_fusion_ascend950_amd import muon_update

    p = torch.zeros(16, 32, device=DEV)
    with pytest.raises(TypeError, match="float32"):
        muon_update(p.bfloat16(), p, p.clone(), lr=0.1)
    with pytest.raises(RuntimeError, match="float32"):
        torch.ops.muon_ascend950.muon_update(p[None], p[None].bfloat16(), p[None].clone(), 0.9,
                                             True, [1.0, 0.0, 0.0], 0.1, 0.0, 1.0)


def test_same_shape_parameters_update_in_one_batched_call(monkeypatch):
    """Muon (group_shapes, the default) stacks small parameters of one shape into one
    native call per step: the momentum buffers equal those of one call per parameter
    bit for bit, the parameters agree to the iteration's precision; a parameter above
    4M elements and a lone shape stay single calls."""
    import muon_fusion_ascend950_amd.optim as optim
    from muon_fusion_ascend950_amd import Muon

    shapes = [(256, 512)] * 3 + [(3, 64, 128)] * 2 + [(200, 36)] * 2 + [(96, 80)] + [(2048, 2049)] * 2
    gen = torch.Generator().manual_seed(61)
    base = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    grads = [[torch.randn(s, generator=gen) * 1e-3 for s in shapes] for _ in range(2)]
    real = optim.muon_update
    calls = []

    def counting(param, *args, **kwargs):
        calls.append(tuple(param.shape))
        return real(param, *args, **kwargs)

    monkeypatch.setattr(optim, "muon_update", counting)
    results = {}
    for grouped in (True, False):
        params = [torch.nn.Parameter(b.clone().to(DEV)) for b in base]
        opt = Muon(params, lr=0.03, momentum=0.9, weight_decay=0.05, group_shapes=grouped)
        calls.clear()
        for step_grads in grads:
            for p, g in zip(params, step_grads):
                p.grad = g.to(DEV)
            opt.step()
        torch.cuda.synchronize()
        results[grouped] = ([p.detach().cpu() for p in params],
                            [opt.state[p]["momentum_buffer"].cpu() for p in params], list(calls))
    (p_g, b_g, c_g), (p_u, b_u, c_u) = results[True], results[False]
    assert len(c_u) == 2 * len(shapes)
    per_step = sorted([(3, 256, 512), (2, 3, 64, 128), (2, 200, 36), (96, 80), (2048, 2049),
                       (2048, 2049)])
    assert sorted(c_g) == sorted(per_step * 2)
    for i, s in enumerate(shapes):
        assert torch.equal(b_g[i], b_u[i]), f"buffer {s}"
        moved_g = (p_g[i] - base[i]).double().numpy()
        moved_u = (p_u[i] - base[i]).double().numpy()
        assert O.rel_frobenius(moved_g, moved_u) <= 1e-2, s
