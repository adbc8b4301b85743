"""amdsplat: MI355X-native (gfx950) differentiable Gaussian-splat rasterizer.

`rasterize(means, scales, quats, opacities, sh, viewmat, K, W, H) -> (image, alpha, aux)` runs
the 3D path through hand-written HIP kernels behind a C ABI (include/amdsplat.h). The 2D
drop-in surfaces live in the sibling packages `gs2d` and `splat2d`.
"""
from .adam import FusedAdam, adam_step, adam_step_sparse
from .loss import fused_ssim, l1_ssim_loss
from .raster3d import (Camera, backward_pass, densification_stats, forward_pass, pruning_scores, rasterize,
                       rasterize_inference)

__all__ = ["Camera", "rasterize", "rasterize_inference", "pruning_scores", "forward_pass", "backward_pass", "densification_stats", "FusedAdam", "adam_step", "adam_step_sparse",
           "l1_ssim_loss", "fused_ssim"]
