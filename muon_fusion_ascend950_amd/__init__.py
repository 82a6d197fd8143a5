"""MI355X (gfx950) Polar Express step: ``polar_step(x, a, b, c)``.

Drop-in for the reference package surface (``muon_ascend950/__init__.py:1-10``):
importing loads the native library and registers ``muon_ascend950::polar_step``.
``polar_express`` (normalise + several steps in one call) has no reference
counterpart; it replaces the loop of the reference's ``examples/five_steps.py``.
"""

from ._loader import load_library

load_library()

from .ops import COEFFICIENTS, polar_express, polar_step  # noqa: E402

__all__ = ["COEFFICIENTS", "polar_express", "polar_step"]
__version__ = "0.1.1"
