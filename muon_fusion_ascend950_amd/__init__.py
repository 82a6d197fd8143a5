"""MI355X (gfx950) Polar Express step: ``polar_step(x, a, b, c)``.

Drop-in for the reference package surface (``muon_ascend950/__init__.py:1-10``):
importing loads the native library and registers ``muon_ascend950::polar_step``.
"""

from ._loader import load_library

load_library()

from .ops import polar_step  # noqa: E402

__all__ = ["polar_step"]
__version__ = "0.1.1"
