"""libzmoe_hip: the MI355X (gfx950) MoE-layer hot path behind a C ABI.

``zmoe.ops`` holds the torch-facing wrappers, ``zmoe.functional`` the autograd
functions of the dense layers around the experts; ``zmoe._lib`` the ctypes binding
of include/zmoe.h. The reference-shaped modules (``scattermoe``, ``modeling``)
sit next to this package and call into it.
"""

from . import _lib, functional, muon, ops, profiling  # noqa: F401
from ._lib import LIB_PATH, ZmoeError, load  # noqa: F401

__all__ = ["ops", "functional", "profiling", "load", "LIB_PATH", "ZmoeError"]
