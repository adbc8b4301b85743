"""Faster-GS's rasterizer backend surface (`FasterGSCudaBackend`) over the MI355X path: the
`_C` extension functions and `torch_bindings` (RasterizerSettings, diff_rasterize, _Rasterize,
FusedAdam), so that code importing `f"{BACKEND}._C"` and `f"{BACKEND}.torch_bindings.rasterization"`
(phase1/tests/test_parity.py:31, cluster/tests/test_lean_adam.py:17-18,107-108) runs with
BACKEND = "amdsplat.fastergs"."""
from . import _C
from .torch_bindings import FusedAdam, RasterizerSettings, _Rasterize, diff_rasterize

__all__ = ["_C", "RasterizerSettings", "diff_rasterize", "_Rasterize", "FusedAdam"]
