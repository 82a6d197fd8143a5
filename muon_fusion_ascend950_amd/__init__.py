"""MI355X (gfx950) Polar Express step: ``polar_step(x, a, b, c)``.

Drop-in for the reference package surface (``muon_ascend950/__init__.py:1-10``):
importing loads the native library and registers ``muon_ascend950::polar_step``.
``polar_express`` (normalise + several steps in one call) has no reference
counterpart; it replaces the loop of the reference's ``examples/five_steps.py``.
``Muon`` / ``muon_update`` run the optimizer update around the iteration (momentum,
orthogonalisation, shape-scaled step, weight decay) that the reference leaves to its
caller.
"""

from ._loader import load_library

load_library()

from .ops import COEFFICIENTS, polar_express, polar_step  # noqa: E402
from .optim import Muon, muon_update  # noqa: E402

__all__ = ["COEFFICIENTS", "Muon", "muon_update", "polar_express", "polar_step"]
__version__ = "0.1.1"
