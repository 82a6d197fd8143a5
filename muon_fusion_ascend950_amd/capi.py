"""ctypes binding of the C ABI declared in ``include/muon_polar.h``.

The torch operator (``_C.so``) links the same ``libmuon_polar.so``, so calls made
here and through ``torch.ops.muon_ascend950.polar_step`` share one launch-config
cache.  The tensor helpers take torch device tensors only for their pointers and
launch on torch's current HIP stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

EXPORTED_FUNCTIONS = (
    "muon_polar_query",
    "muon_polar_step",
    "muon_polar_step_noalloc",
    "muon_polar_gram",
    "muon_polar_poly",
    "muon_polar_apply",
    "muon_polar_express",
    "muon_polar_muon_update",
    "muon_polar_check_plan",
    "muon_polar_last_error",
    "muon_polar_version",
)

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_WORKSPACE = -2
ERR_HIP = -3
ERR_CONFIG = -4


class ShapeInfo(ctypes.Structure):
    _fields_ = [
        ("padded_rows", ctypes.c_int64),
        ("gram_bytes", ctypes.c_size_t),
        ("workspace_bytes", ctypes.c_size_t),
        ("express_workspace_bytes", ctypes.c_size_t),
        ("muon_workspace_bytes", ctypes.c_size_t),
    ]


class StageExtent(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "tile_m", "tile_n", "waves", "depth", "dma_fed", "k_steps", "total_tiles", "dp_tiles",
        "sk_units", "grid", "coverage_ok", "extents_ok", "halves", "diag_pairs")] + [
        (name, ctypes.c_int64) for name in (
            "out_lo", "out_hi", "out_limit", "partial_lo", "partial_hi", "partial_limit",
            "counter_hi", "counter_limit")]


class PlanExtents(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in (
        "workspace_bytes", "gram_bytes", "poly_offset", "counters_offset", "counter_stride",
        "partials_offset", "pad_offset", "pad_end", "y_bytes")] + [
        ("stage", StageExtent * 3), ("chain_apply", StageExtent)]


class CapiError(RuntimeError):
    def __init__(self, func: str, status: int, detail: str):
        super().__init__(f"{func} failed with status {status}: {detail}")
        self.status = status
        self.detail = detail


_LIB = None


def library_path() -> Path:
    configured = os.environ.get("MUON_POLAR_CAPI_LIBRARY")
    if configured:
        return Path(configured).expanduser().resolve()
    return Path(__file__).resolve().parent / "libmuon_polar.so"


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.is_file():
        raise RuntimeError(
            f"libmuon_polar.so is missing at {path}; build it with "
            "`python setup.py build_ext --inplace`"
        )
    lib = ctypes.CDLL(str(path))
    i64, vp, sz, dbl = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_double
    lib.muon_polar_query.argtypes = [i64, i64, i64, ctypes.POINTER(ShapeInfo)]
    lib.muon_polar_step.argtypes = [vp, vp, vp, sz, i64, i64, i64, dbl, dbl, dbl, vp]
    lib.muon_polar_step_noalloc.argtypes = [vp, vp, i64, i64, i64, dbl, dbl, dbl, vp]
    lib.muon_polar_gram.argtypes = [vp, vp, vp, sz, i64, i64, i64, vp]
    lib.muon_polar_poly.argtypes = [vp, vp, vp, sz, i64, i64, i64, dbl, dbl, vp]
    lib.muon_polar_apply.argtypes = [vp, vp, vp, vp, sz, i64, i64, i64, dbl, vp]
    lib.muon_polar_express.argtypes = [vp, vp, vp, sz, i64, i64, i64,
                                       ctypes.POINTER(ctypes.c_double), i64, ctypes.c_int, vp]
    lib.muon_polar_muon_update.argtypes = [vp, vp, vp, vp, sz, i64, i64, i64, dbl, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_double), i64, dbl, dbl, dbl,
                                           vp]
    lib.muon_polar_check_plan.argtypes = [i64, i64, i64, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(PlanExtents)]
    for name in ("muon_polar_query", "muon_polar_step", "muon_polar_step_noalloc",
                 "muon_polar_gram", "muon_polar_poly",
                 "muon_polar_apply", "muon_polar_express", "muon_polar_muon_update",
                 "muon_polar_check_plan"):
        getattr(lib, name).restype = ctypes.c_int
    lib.muon_polar_last_error.argtypes = []
    lib.muon_polar_last_error.restype = ctypes.c_char_p
    lib.muon_polar_version.argtypes = []
    lib.muon_polar_version.restype = ctypes.c_char_p
    _LIB = lib
    return lib


def last_error() -> str:
    return load().muon_polar_last_error().decode()


def check(func: str, status: int) -> None:
    if status != OK:
        raise CapiError(func, status, last_error())


def query(batch: int, m: int, n: int) -> ShapeInfo:
    info = ShapeInfo()
    check("muon_polar_query", load().muon_polar_query(batch, m, n, ctypes.byref(info)))
    return info


def check_plan(batch: int, m: int, n: int, cus: int = 256, blocks_per_cu=(1, 1, 1)) -> PlanExtents:
    """muon_polar_check_plan: store extents of the step's plan for a device of `cus`
    compute units and the given resident workgroups per CU of each stage's kernel."""
    out = PlanExtents()
    occ = (ctypes.c_int * 3)(*blocks_per_cu)
    check("muon_polar_check_plan", load().muon_polar_check_plan(batch, m, n, cus, occ,
                                                                ctypes.byref(out)))
    return out


# --------------------------------------------------------------- torch tensor helpers
def _stream(stream):
    if stream is not None:
        return stream
    import torch

    return torch.cuda.current_stream().cuda_stream


def _bmn(x):
    if x.ndim == 2:
        return 1, x.shape[0], x.shape[1]
    return x.shape[0], x.shape[1], x.shape[2]


def alloc_workspace(batch: int, m: int, n: int, device="cuda"):
    import torch

    info = query(batch, m, n)
    return torch.empty(info.workspace_bytes, dtype=torch.uint8, device=device), info


def step(x, y, workspace, a: float, b: float, c: float, stream=None) -> None:
    batch, m, n = _bmn(x)
    check("muon_polar_step", load().muon_polar_step(
        x.data_ptr(), y.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        batch, m, n, float(a), float(b), float(c), _stream(stream)))


def step_noalloc(x, y, a: float, b: float, c: float, stream=None) -> None:
    """muon_polar_step_noalloc: the step with the library's own per-GPU scratch."""
    batch, m, n = _bmn(x)
    check("muon_polar_step_noalloc", load().muon_polar_step_noalloc(
        x.data_ptr(), y.data_ptr(), batch, m, n, float(a), float(b), float(c), _stream(stream)))


def _ws(workspace):
    """(pointer, bytes) of an optional workspace tensor (None: no stream-K split)."""
    if workspace is None:
        return None, 0
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def alloc_express_workspace(batch: int, m: int, n: int, device="cuda"):
    import torch

    info = query(batch, m, n)
    return torch.empty(info.express_workspace_bytes, dtype=torch.uint8, device=device), info


def express(x, y, workspace, coefficients, normalize: bool = True, stream=None) -> None:
    """muon_polar_express: coefficients is a sequence of (a, b, c) triples."""
    batch, m, n = _bmn(x)
    flat = [float(v) for triple in coefficients for v in triple]
    arr = (ctypes.c_double * max(1, len(flat)))(*flat)
    check("muon_polar_express", load().muon_polar_express(
        x.data_ptr(), y.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        batch, m, n, arr, len(flat) // 3, int(bool(normalize)), _stream(stream)))


def gram(x, gram_buf, stream=None, workspace=None) -> None:
    batch, m, n = _bmn(x)
    check("muon_polar_gram", load().muon_polar_gram(
        x.data_ptr(), gram_buf.data_ptr(), *_ws(workspace), batch, m, n, _stream(stream)))


def poly(gram_buf, poly_buf, batch: int, m: int, n: int, b: float, c: float, stream=None,
         workspace=None) -> None:
    check("muon_polar_poly", load().muon_polar_poly(
        gram_buf.data_ptr(), poly_buf.data_ptr(), *_ws(workspace), batch, m, n, float(b),
        float(c), _stream(stream)))


def apply(poly_buf, x, y, a: float, stream=None, workspace=None) -> None:
    batch, m, n = _bmn(x)
    check("muon_polar_apply", load().muon_polar_apply(
        poly_buf.data_ptr(), x.data_ptr(), y.data_ptr(), *_ws(workspace), batch, m, n,
        float(a), _stream(stream)))


def alloc_muon_workspace(batch: int, m: int, n: int, device="cuda"):
    import torch

    info = query(batch, m, n)
    return torch.empty(info.muon_workspace_bytes, dtype=torch.uint8, device=device), info


def muon_update(param, grad, momentum_buffer, workspace, coefficients, *, momentum: float,
                nesterov: bool, lr: float, weight_decay: float, lr_scale: float,
                stream=None) -> None:
    """muon_polar_muon_update on fp32 [batch, m, n] tensors (param and buffer in place)."""
    batch, m, n = _bmn(param)
    flat = [float(v) for triple in coefficients for v in triple]
    arr = (ctypes.c_double * max(1, len(flat)))(*flat)
    check("muon_polar_muon_update", load().muon_polar_muon_update(
        param.data_ptr(), grad.data_ptr(), momentum_buffer.data_ptr(), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), batch, m, n, float(momentum),
        int(bool(nesterov)), arr, len(flat) // 3, float(lr), float(weight_decay), float(lr_scale),
        _stream(stream)))
