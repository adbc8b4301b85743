"""Drop-in for the phase0 `splat2d` package (phase0/splat2d/__init__.py): the Cholesky-
parametrised 2D splat renderer with two custom backward passes, on the MI355X.

Mode "pixel" is the per-pixel atomic backward (A); mode "splat" is the bucketed backward (B)
that replays from forward checkpoints. float32 and float64 are supported, on CUDA (ROCm)
tensors only; there is no CPU build. ref_render (and ref_state in splat2d.ops) is the dense
PyTorch reference model, for checking and small scenes only.
"""
from splat2d.ops import MODES, Mode, TileBins, bin_tiles, load_extension, ref_render, render

__all__ = ["MODES", "Mode", "TileBins", "bin_tiles", "load_extension", "ref_render", "render"]
