"""Host-side boundary: Python surface, torch op registration, FakeTensor path and the
C ABI library — everything that runs without a GPU.

Reference behaviour being mirrored: muon_ascend950/ops.py:6-33 (checks, 2-D/3-D,
M > N transpose), _loader.py:10-49 (library discovery, fake kernel), and the op schema
of csrc/muon_polar_step_binding.cpp:677-685.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import muon_fusion_ascend950_amd as mf
from oracle import polar_oracle as O
from muon_fusion_ascend950_amd import _loader, capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "muon_polar.h"
C0 = (8.156554524902461, -22.48329292557795, 15.878769915207462)


# ----------------------------------------------------------------------------- python surface
def test_public_surface():
    import muon_ascend950

    assert muon_ascend950.polar_step is mf.polar_step
    assert muon_ascend950.polar_express is mf.polar_express
    assert mf.__version__ == "0.1.1" == muon_ascend950.__version__
    assert mf.__all__ == ["COEFFICIENTS", "Muon", "muon_update", "polar_express", "polar_step"]
    # the reference's five triples (tests/test_polar_step.py:13-19)
    assert mf.COEFFICIENTS == tuple(tuple(t) for t in O.COEFFICIENTS)


def test_rejects_non_tensor():
    with pytest.raises(TypeError, match="torch.Tensor"):
        mf.polar_step([[1.0]], *C0)


def test_rejects_cpu_tensor():
    with pytest.raises(ValueError, match="ROCm GPU"):
        mf.polar_step(torch.zeros(4, 8, dtype=torch.bfloat16), *C0)


@pytest.mark.parametrize(
    "shape,dtype,exc,msg",
    [
        ((4, 8), torch.float32, TypeError, "bfloat16"),
        ((4, 8), torch.float16, TypeError, "bfloat16"),
        ((8,), torch.bfloat16, ValueError, "shape"),
        ((1, 2, 4, 8), torch.bfloat16, ValueError, "shape"),
        ((0, 8), torch.bfloat16, ValueError, "positive"),
        ((2, 0, 8), torch.bfloat16, ValueError, "positive"),
    ],
)
def test_argument_checks_on_device_tensors(shape, dtype, exc, msg):
    with FakeTensorMode():
        x = torch.empty(shape, dtype=dtype, device="cuda")
        with pytest.raises(exc, match=msg):
            mf.polar_step(x, *C0)


@pytest.mark.parametrize("shape", [(129, 130), (130, 129), (2, 150, 2050), (3, 70, 20), (1, 1)])
def test_fake_path_preserves_shape_and_dtype(shape):
    # FakeTensor kernel registered by the loader (reference _loader.py:41-48)
    with FakeTensorMode():
        x = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        y = mf.polar_step(x, *C0)
        assert y.shape == x.shape and y.dtype == torch.bfloat16 and y.device == x.device
        assert y.is_contiguous()


def test_fake_kernel_on_op_directly():
    with FakeTensorMode():
        x = torch.empty(2, 5, 9, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
        y = torch.ops.muon_ascend950.polar_step(x, 1.0, 2.0, 3.0)
        assert y.shape == x.shape and y.is_contiguous()


def test_op_schema_matches_reference():
    schema = str(torch.ops.muon_ascend950.polar_step.default._schema)
    assert schema == "muon_ascend950::polar_step(Tensor x, float a, float b, float c) -> Tensor"


def test_express_fake_and_schema():
    schema = str(torch.ops.muon_ascend950.polar_express.default._schema)
    assert schema == ("muon_ascend950::polar_express(Tensor x, float[] coefficients, bool normalize)"
                      " -> Tensor")
    with FakeTensorMode():
        for shape in [(2, 5, 9), (9, 5), (3, 40, 7)]:
            x = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
            y = mf.polar_express(x)
            assert y.shape == x.shape and y.dtype == torch.bfloat16


def test_express_rejects_bad_arguments():
    with FakeTensorMode():
        x = torch.empty(2, 5, 9, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(ValueError, match="triples"):
            mf.polar_express(x, [(1.0, 2.0)])
        with pytest.raises(ValueError, match="nothing to do"):
            mf.polar_express(x, [], normalize=False)
        with pytest.raises(TypeError, match="bfloat16"):
            mf.polar_express(x.float())


def test_express_entry_validates_before_launch():
    lib = capi.load()
    coeffs = (ctypes.c_double * 3)(1.0, 2.0, 3.0)
    info = capi.query(1, 4, 8)
    assert info.express_workspace_bytes >= info.workspace_bytes + 4 * 8 * 2
    big = info.express_workspace_bytes
    assert lib.muon_polar_express(None, 16, 16, big, 1, 4, 8, coeffs, 1, 1, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_express(16, 4096, 16, big, 1, 4, 8, coeffs, 0, 0, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_express(16, 4096, 16, big, 1, 4, 8, None, 2, 1, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_express(16, 4096, 16, big - 1, 1, 4, 8, coeffs, 1, 1, None) == capi.ERR_WORKSPACE
    # x and y overlap: rejected before anything launches (pointers never dereferenced)
    assert lib.muon_polar_express(16, 32, 16, big, 1, 4, 8, coeffs, 1, 1, None) == capi.ERR_INVALID_ARGUMENT
    assert "overlap" in capi.last_error()


def test_muon_update_fake_and_schema():
    schema = str(torch.ops.muon_ascend950.muon_update.default._schema)
    assert schema == ("muon_ascend950::muon_update(Tensor(a!) param, Tensor grad, "
                      "Tensor(b!) momentum_buffer, float momentum, bool nesterov, "
                      "float[] coefficients, float lr, float weight_decay, float lr_scale) -> ()")
    with FakeTensorMode():
        # wide, batched, tall with N % 8 == 0, tall otherwise (transposed route),
        # several leading dimensions, non-contiguous
        for shape in [(5, 9), (2, 5, 9), (40, 16), (40, 7), (4, 3, 16, 8)]:
            p = torch.empty(shape, dtype=torch.float32, device="cuda")
            mf.muon_update(p, torch.empty_like(p), torch.zeros_like(p), lr=0.02)
        # non-contiguous param and buffer, bf16 grad
        p = torch.empty(9, 5, dtype=torch.float32, device="cuda").mT
        b = torch.zeros(9, 5, dtype=torch.float32, device="cuda").mT
        mf.muon_update(p, torch.empty(5, 9, dtype=torch.bfloat16, device="cuda"), b, lr=0.02)


def test_muon_update_rejects_bad_arguments():
    with FakeTensorMode():
        p = torch.empty(8, 16, dtype=torch.float32, device="cuda")
        g, b = torch.empty_like(p), torch.zeros_like(p)
        with pytest.raises(TypeError, match="float32"):
            mf.muon_update(p.bfloat16(), g, b, lr=0.1)
        with pytest.raises(TypeError, match="grad"):
            mf.muon_update(p, g.half(), b, lr=0.1)
        with pytest.raises(ValueError, match="ndim"):
            mf.muon_update(p[0], g[0], b[0], lr=0.1)
        with pytest.raises(ValueError, match="one shape"):
            mf.muon_update(p, g[:4], b, lr=0.1)
        with pytest.raises(ValueError, match="coefficient triples"):
            mf.muon_update(p, g, b, lr=0.1, ns_steps=6)
    with pytest.raises(ValueError, match="ROCm GPU"):
        cpu = torch.zeros(8, 16)
        mf.muon_update(cpu, cpu.clone(), cpu.clone(), lr=0.1)
    w = torch.nn.Parameter(torch.zeros(8, 16))
    for kwargs in ({"lr": -1.0}, {"momentum": 1.5}, {"weight_decay": -0.1}, {"ns_steps": 0},
                   {"ns_steps": 6}):
        with pytest.raises(ValueError):
            mf.Muon([w], **kwargs)


def test_muon_default_lr_scale():
    from muon_fusion_ascend950_amd.optim import default_lr_scale

    assert default_lr_scale(512, 2048) == 1.0
    assert default_lr_scale(2048, 512) == 2.0
    assert default_lr_scale(300, 300) == 1.0


def test_muon_entry_validates_before_launch():
    lib = capi.load()
    coeffs = (ctypes.c_double * 3)(1.0, 2.0, 3.0)
    info = capi.query(1, 4, 8)
    assert info.muon_workspace_bytes >= info.express_workspace_bytes + 4 * 8 * 2
    big = info.muon_workspace_bytes
    # distinct, non-overlapping fake addresses; nothing is dereferenced before the checks
    p, g, b, ws = 1 << 20, 2 << 20, 3 << 20, 4 << 20

    def call(*, p=p, g=g, b=b, ws=ws, size=big, m=4, n=8, momentum=0.95, steps=1, cf=coeffs,
             lr=0.1, wd=0.0, scale=1.0):
        return lib.muon_polar_muon_update(p, g, b, ws, size, 1, m, n, momentum, 1, cf, steps, lr,
                                          wd, scale, None)

    assert call(p=None) == capi.ERR_INVALID_ARGUMENT
    assert call(steps=-1) == capi.ERR_INVALID_ARGUMENT
    assert call(cf=None) == capi.ERR_INVALID_ARGUMENT
    assert call(momentum=1.5) == capi.ERR_INVALID_ARGUMENT
    assert call(lr=float("nan")) == capi.ERR_INVALID_ARGUMENT
    assert call(size=big - 1) == capi.ERR_WORKSPACE
    assert call(g=p + 64) == capi.ERR_INVALID_ARGUMENT and "overlap" in capi.last_error()
    assert call(ws=b + 16) == capi.ERR_INVALID_ARGUMENT and "overlap" in capi.last_error()
    tall = capi.query(1, 20, 12).muon_workspace_bytes
    assert call(m=20, n=12, size=tall) == capi.ERR_INVALID_ARGUMENT
    assert "n % 8 == 0" in capi.last_error()


def test_loader_is_idempotent():
    _loader.load_library()
    _loader.load_library()
    assert _loader._LOADED


def test_loader_env_override(monkeypatch, tmp_path):
    monkeypatch.setenv("MUON_ASCEND950_LIBRARY", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="does not exist"):
        _loader._library_path()
    real = next((ROOT / "muon_fusion_ascend950_amd").glob("_C*.so"))
    monkeypatch.setenv("MUON_ASCEND950_LIBRARY", str(real))
    assert _loader._library_path() == real.resolve()


def test_import_fails_loudly_without_native_library(tmp_path):
    """A missing native library is a hard error at import: there is no CPU fallback."""
    pkg = tmp_path / "muon_fusion_ascend950_amd"
    pkg.mkdir()
    for f in ("__init__.py", "_loader.py", "ops.py"):
        (pkg / f).write_text((ROOT / "muon_fusion_ascend950_amd" / f).read_text())
    env = dict(os.environ, PYTHONPATH=str(tmp_path))
    env.pop("MUON_ASCEND950_LIBRARY", None)
    proc = subprocess.run([sys.executable, "-c", "import muon_fusion_ascend950_amd"],
                          cwd=tmp_path, env=env, capture_output=True, text=True, timeout=300)
    assert proc.returncode != 0
    assert "native library is missing" in proc.stderr


# ----------------------------------------------------------------------------- C ABI library
def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(muon_polar_\w+)\s*\(", text, re.M)))


def test_header_declares_the_exported_set():
    assert declared_functions() == sorted(capi.EXPORTED_FUNCTIONS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(capi.library_path()))
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (muon_polar_\w+)$", out, re.M))
    assert exported == set(declared_functions())


def test_capi_version():
    assert capi.load().muon_polar_version().decode() == "0.1.1"


@pytest.mark.parametrize("batch,m,n", [(1, 129, 130), (2, 150, 2050), (8, 512, 2048),
                                       (1, 4096, 14336), (4, 4096, 4096), (3, 1, 1)])
def test_query_sizes(batch, m, n):
    info = capi.query(batch, m, n)
    mp = info.padded_rows
    assert mp >= m and mp % 64 == 0 and mp - m < 256
    assert info.gram_bytes == batch * mp * mp * 2
    assert info.workspace_bytes >= 2 * info.gram_bytes
    assert info.workspace_bytes % 256 == 0


@pytest.mark.parametrize("batch,m,n", [(0, 4, 4), (1, 0, 4), (1, 4, 0), (-1, 4, 4)])
def test_query_rejects_bad_shapes(batch, m, n):
    with pytest.raises(capi.CapiError) as err:
        capi.query(batch, m, n)
    assert err.value.status == capi.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("m,n", [(5, 4), (700, 256), (14336, 4096)])
def test_query_tall_sizes_the_right_gram(m, n):
    """m > n: the Gram matrix is XᵀX, n x n, so the padding follows n and the
    sizes equal those of the transposed shape."""
    tall = capi.query(2, m, n)
    wide = capi.query(2, n, m)
    assert tall.padded_rows == wide.padded_rows and tall.padded_rows >= n
    assert tall.gram_bytes == wide.gram_bytes
    assert tall.express_workspace_bytes >= 2 * tall.gram_bytes + 2 * 2 * m * n


def test_tall_step_needs_n_multiple_of_8():
    lib = capi.load()
    # non-null pointers are never dereferenced: the shape check fails first
    st = lib.muon_polar_step(16, 16, 16, 1 << 30, 1, 20, 12, 1.0, 1.0, 1.0, None)
    assert st == capi.ERR_INVALID_ARGUMENT
    assert "n % 8 == 0" in lib.muon_polar_last_error().decode()


def test_tall_stage_entries_are_rejected():
    lib = capi.load()
    for call in (lambda: lib.muon_polar_gram(16, 16, None, 0, 1, 24, 16, None),
                 lambda: lib.muon_polar_poly(16, 16, None, 0, 1, 24, 16, 1.0, 1.0, None),
                 lambda: lib.muon_polar_apply(16, 16, 16, None, 0, 1, 24, 16, 1.0, None)):
        assert call() == capi.ERR_INVALID_ARGUMENT
        assert "m <= n" in lib.muon_polar_last_error().decode()


def test_query_rejects_oversized_matrix():
    with pytest.raises(capi.CapiError, match="too large"):
        capi.query(1, 46341, 46341)


def test_entry_points_validate_before_launch():
    lib = capi.load()
    assert lib.muon_polar_step(None, None, None, 0, 1, 4, 8, 1.0, 1.0, 1.0, None) == capi.ERR_INVALID_ARGUMENT
    # non-null but never dereferenced: the workspace check fails first, nothing launches
    assert lib.muon_polar_step(16, 16, None, 0, 1, 4, 8, 1.0, 1.0, 1.0, None) == capi.ERR_WORKSPACE
    assert "workspace must hold" in capi.last_error()
    assert lib.muon_polar_step(16, 16, 16, 1, 1, 4, 8, 1.0, 1.0, 1.0, None) == capi.ERR_WORKSPACE
    assert lib.muon_polar_step(16, 16, 16, 1 << 20, 1, 8, 4, 1.0, 1.0, 1.0, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_gram(None, 16, None, 0, 1, 4, 8, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_poly(16, None, None, 0, 1, 4, 8, 1.0, 1.0, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_apply(16, 16, None, None, 0, 1, 4, 8, 1.0, None) == capi.ERR_INVALID_ARGUMENT
    assert lib.muon_polar_gram(16, 17, None, 0, 1, 4, 8, None) == capi.ERR_INVALID_ARGUMENT  # misaligned
    # an optional stage workspace, when given, is checked like polar_step's
    assert lib.muon_polar_gram(16, 16, 16, 1, 1, 4, 8, None) == capi.ERR_WORKSPACE
    assert lib.muon_polar_poly(16, 16, 16, 1, 1, 4, 8, 1.0, 1.0, None) == capi.ERR_WORKSPACE
    assert lib.muon_polar_apply(16, 16, 16, 16, 1, 1, 4, 8, 1.0, None) == capi.ERR_WORKSPACE
    assert lib.muon_polar_apply(16, 16, 16, 17, 1 << 20, 1, 4, 8, 1.0, None) == capi.ERR_WORKSPACE


@pytest.mark.parametrize("var,value", [("MUON_POLAR_GRAM_TILE", "96"), ("MUON_POLAR_POLY_TILE", "512"),
                                       ("MUON_POLAR_APPLY_TILE_M", "32"),
                                       ("MUON_POLAR_APPLY_TILE_N", "100"),
                                       ("MUON_POLAR_WAVES", "6"), ("MUON_POLAR_STREAM_K", "2")])
def test_bad_tuning_variable_is_a_config_error(monkeypatch, var, value):
    monkeypatch.setenv(var, value)
    with pytest.raises(capi.CapiError) as err:
        capi.query(1, 512, 2048)
    assert err.value.status == capi.ERR_CONFIG


def test_tuning_variables_enter_the_plan(monkeypatch):
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", "256")
    assert capi.query(1, 300, 700).padded_rows == 512
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", "64")
    monkeypatch.setenv("MUON_POLAR_POLY_TILE", "64")
    assert capi.query(1, 300, 700).padded_rows == 320
    # A and P are padded to the larger of the two stages' tile extents
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", "192")
    assert capi.query(1, 300, 700).padded_rows == 384
    monkeypatch.setenv("MUON_POLAR_POLY_TILE", "256")
    assert capi.query(1, 300, 700).padded_rows == 512


def test_build_entry_does_not_import_the_package():
    """build() must work before a native library exists (or when the one in place is
    stale): it loads the build script by path, never the package."""
    import subprocess
    import sys

    code = ("import sys, __graft_entry__ as g; m = g._load_builder(); "
            "assert callable(m.build); "
            "assert 'muon_fusion_ascend950_amd' not in sys.modules, 'package imported'")
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_in_place_step_and_apply_are_rejected():
    """y over x would race (every apply tile reads X's whole K range while other
    tiles write Y): the step and the apply stage refuse it before any launch."""
    lib = capi.load()
    info = capi.query(1, 64, 128)
    x = 1 << 20  # never dereferenced: the checks fail first
    ws = 1 << 32
    st = lib.muon_polar_step(x, x, ws, info.workspace_bytes, 1, 64, 128, 1.0, 1.0, 1.0, None)
    assert st == capi.ERR_INVALID_ARGUMENT and "must not overlap" in capi.last_error()
    st = lib.muon_polar_step(x, x + 64 * 128, ws, info.workspace_bytes, 1, 64, 128, 1.0, 1.0,
                             1.0, None)  # half-overlapping rows
    assert st == capi.ERR_INVALID_ARGUMENT and "must not overlap" in capi.last_error()
    st = lib.muon_polar_step(x, ws + 4096, ws, info.workspace_bytes, 1, 64, 128, 1.0, 1.0, 1.0,
                             None)  # y inside the workspace
    assert st == capi.ERR_INVALID_ARGUMENT and "workspace must not overlap" in capi.last_error()
    st = lib.muon_polar_apply(ws, x, x, None, 0, 1, 64, 128, 1.0, None)
    assert st == capi.ERR_INVALID_ARGUMENT and "must not overlap" in capi.last_error()
    st = lib.muon_polar_apply(ws, x, ws + 256, None, 0, 1, 64, 128, 1.0, None)
    assert st == capi.ERR_INVALID_ARGUMENT and "poly and y must not overlap" in capi.last_error()


def test_noalloc_rejects_shapes_beyond_its_scratch_before_any_launch():
    """muon_polar_step_noalloc's size check runs on the host before any device call:
    [4,4096,4096] needs more than its 192 MiB scratch even with the one-round split
    (A and P alone are 256 MiB), so it is rejected.  The non-null pointers are never
    dereferenced."""
    lib = capi.load()
    info = capi.query(4, 4096, 4096)
    assert 2 * info.gram_bytes > 192 << 20
    st = lib.muon_polar_step_noalloc(16, 1 << 40, 4, 4096, 4096, 1.0, 1.0, 1.0, None)
    assert st == capi.ERR_WORKSPACE
    assert "muon_polar_step_noalloc holds" in capi.last_error()
    # a null x or y is refused first
    assert lib.muon_polar_step_noalloc(None, 16, 1, 8, 8, 1.0, 1.0, 1.0, None) == capi.ERR_INVALID_ARGUMENT


def test_stage_calls_reject_overlapping_buffers_before_any_launch():
    """The stage entry points and muon_polar_express refuse an output over one of
    their inputs, and operands over the part of the workspace the call writes besides
    its output (arrival words, partial slots, padded copy of X), before any device
    call: the stand-in addresses below are never dereferenced."""
    lib = capi.load()
    batch, m, n = 2, 150, 2050
    info = capi.query(batch, m, n)
    wsb = info.workspace_bytes
    stage_area = 2 * (-(-info.gram_bytes // 256) * 256)  # past the A and P areas
    W, X, Y, G, P = (k << 40 for k in (1, 2, 3, 4, 5))
    bad = capi.ERR_INVALID_ARGUMENT
    # gram over x; x or gram in the workspace's stage area
    assert lib.muon_polar_gram(X, X + 4096, None, 0, batch, m, n, None) == bad
    assert "x and gram" in capi.last_error()
    assert lib.muon_polar_gram(W + stage_area, G, W, wsb, batch, m, n, None) == bad
    assert lib.muon_polar_gram(X, W + stage_area, W, wsb, batch, m, n, None) == bad
    # poly in place; poly in the stage area
    assert lib.muon_polar_poly(G, G, None, 0, batch, m, n, 1.0, 1.0, None) == bad
    assert "gram and poly" in capi.last_error()
    assert lib.muon_polar_poly(G, W + stage_area, W, wsb, batch, m, n, 1.0, 1.0, None) == bad
    # apply with y in the stage area, or x there (the padded copy is written there)
    assert lib.muon_polar_apply(P, X, W + stage_area, W, wsb, batch, m, n, 1.0, None) == bad
    assert lib.muon_polar_apply(P, W + stage_area, Y, W, wsb, batch, m, n, 1.0, None) == bad
    # express: the workspace over y
    coeffs = (ctypes.c_double * 3)(1.0, 1.0, 1.0)
    ews = info.express_workspace_bytes
    assert lib.muon_polar_express(X, W + 4096, W, ews, batch, m, n, coeffs, 1, 1, None) == bad
    assert "workspace must not overlap" in capi.last_error()
