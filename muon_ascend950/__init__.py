"""Drop-in import name of the reference package (``muon_ascend950``).

``from muon_ascend950 import polar_step`` resolves to the MI355X implementation in
``muon_fusion_ascend950_amd``.
"""

from muon_fusion_ascend950_amd import COEFFICIENTS, __version__, polar_express, polar_step

__all__ = ["polar_step", "polar_express", "COEFFICIENTS"]
