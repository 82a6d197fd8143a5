"""Locate and load the native operator library.

Mirrors the reference loader (``muon_ascend950/_loader.py:1-50``):

* ``MUON_ASCEND950_LIBRARY`` names the operator library explicitly
  (``_loader.py:11-16``); otherwise the first ``_C*.so`` next to this package is
  used (``_loader.py:18-25``);
* ``torch.ops.load_library`` registers ``muon_ascend950::polar_step``
  (``_loader.py:39``), and a FakeTensor kernel is registered for tracing, tolerating
  an earlier registration (``_loader.py:41-48``);
* loading is idempotent (``_loader.py:7``, ``:30-31``, ``:49``).

Differences: the accelerator check asks for a ROCm build of torch instead of
``torch_npu``, and a missing library is a hard error (there is no CPU fallback).
"""

from __future__ import annotations

import os
from pathlib import Path

_LOADED = False


def _library_path() -> Path:
    configured = os.environ.get("MUON_ASCEND950_LIBRARY")
    if configured:
        path = Path(configured).expanduser().resolve()
        if not path.is_file():
            raise RuntimeError(f"MUON_ASCEND950_LIBRARY does not exist: {path}")
        return path

    package_dir = Path(__file__).resolve().parent
    candidates = sorted(package_dir.glob("_C*.so"))
    if not candidates:
        raise RuntimeError(
            "muon_ascend950 native library is missing. Build it in place with "
            "`python setup.py build_ext --inplace` for the current torch/ROCm environment."
        )
    return candidates[0]


def load_library() -> None:
    global _LOADED
    if _LOADED:
        return

    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("muon_ascend950 requires torch built for ROCm") from exc
    if not getattr(torch.version, "hip", None):
        raise RuntimeError("muon_ascend950 requires torch built for ROCm (torch.version.hip is unset)")

    torch.ops.load_library(str(_library_path()))

    def fake_polar_step(x, a: float, b: float, c: float):
        return torch.empty_like(x, memory_format=torch.contiguous_format)

    def fake_polar_express(x, coefficients, normalize: bool):
        return torch.empty_like(x, memory_format=torch.contiguous_format)

    def fake_muon_update(param, grad, momentum_buffer, momentum, nesterov, coefficients, lr,
                         weight_decay, lr_scale):
        return None

    for name, fake in (("muon_ascend950::polar_step", fake_polar_step),
                       ("muon_ascend950::polar_step_tall", fake_polar_step),
                       ("muon_ascend950::polar_express", fake_polar_express),
                       ("muon_ascend950::muon_update", fake_muon_update)):
        try:
            torch.library.register_fake(name)(fake)
        except RuntimeError as exc:
            if "already has" not in str(exc):
                raise
    _LOADED = True
