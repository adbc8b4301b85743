"""Faster-GS's `torch_bindings` package surface (rasterization and the fused Adam)."""
from ...adam import FusedAdam
from .rasterization import RasterizerSettings, _Rasterize, diff_rasterize

__all__ = ["RasterizerSettings", "diff_rasterize", "_Rasterize", "FusedAdam"]
