"""Fused Adam for the Gaussian parameters (mirrors Faster-GS's FusedAdam and its lean variant,
cluster/patches/fastergs_lean_adam.patch:221-312).

`FusedAdam(params, lr, eps, sparse=False, lowp_moment_groups=())` is a torch.optim.Adam whose
step() runs every parameter group in one HIP launch (gs_adam_step). sparse: only primitives
visible in the view (tiles_touched > 0) are updated; the others keep parameters and moments. The
mask is step(visibility=aux["visibility"]) of the forward, or, when step() is not handed one,
the one the last differentiable forward left in the class-attribute hand-off of the reference's
patch (_Rasterize.last_visibility, cluster/patches/fastergs_lean_adam.patch:329-343).
lowp_moment_groups: names of groups whose exp_avg / exp_avg_sq are kept in bfloat16 with
stochastic rounding. With both off this is the dense float32 update.

`adam_step` / `adam_step_sparse` mirror the extension functions `_C.adam_step` and
`_C.adam_step_sparse` (same argument order) for callers that keep their own optimizer state.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import call, ptr


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.GS_FLOAT32
    if t.dtype == torch.bfloat16:
        return _lib.GS_BFLOAT16
    raise TypeError(f"moments must be float32 or bfloat16, got {t.dtype}")


def _check(param, grad, exp_avg, exp_avg_sq):
    if not (param.is_cuda and param.is_contiguous() and param.dtype == torch.float32):
        raise ValueError("param must be a contiguous float32 CUDA tensor")
    if not (grad.is_contiguous() and grad.dtype == torch.float32 and grad.numel() == param.numel()):
        raise ValueError("bad grad: contiguous float32 with the shape of param")
    if exp_avg.dtype != exp_avg_sq.dtype:
        raise ValueError("exp_avg and exp_avg_sq must share a dtype")
    if not (exp_avg.is_contiguous() and exp_avg_sq.is_contiguous() and exp_avg.numel() == param.numel()
            and exp_avg_sq.numel() == param.numel()):
        raise ValueError("bad moments: contiguous, with the shape of param")


def _group(grad, param, exp_avg, exp_avg_sq, step, lr, beta1, beta2, eps) -> _lib.GsAdamGroup:
    return _lib.GsAdamGroup(ptr(grad), ptr(param), ptr(exp_avg), ptr(exp_avg_sq), param.numel(),
                            _dtype_code(exp_avg), int(step), float(lr), float(beta1), float(beta2), float(eps))


def _launch(groups, n_primitives: int, visibility, device) -> None:
    for i in range(0, len(groups), _lib.GS_ADAM_MAX_GROUPS):
        chunk = groups[i:i + _lib.GS_ADAM_MAX_GROUPS]
        arr = (_lib.GsAdamGroup * len(chunk))(*chunk)
        call("gs_adam_step", arr, len(chunk), int(n_primitives), ptr(visibility), _lib.stream_handle(device))


def _visibility(visibility, n_primitives: int):
    if visibility is None or visibility.numel() == 0:
        return None
    if not (visibility.is_cuda and visibility.is_contiguous() and visibility.dtype == torch.int32
            and visibility.numel() == n_primitives):
        raise ValueError("visibility must be int32 [n_primitives] on the GPU")
    return visibility


@torch.no_grad()
def adam_step(param_grad, param, exp_avg, exp_avg_sq, step_count, learning_rate, beta1, beta2, epsilon):
    """Dense Adam step of one tensor (float32 moments)."""
    adam_step_sparse(param_grad, param, exp_avg, exp_avg_sq, None, step_count, learning_rate, beta1, beta2,
                     epsilon)


@torch.no_grad()
def adam_step_sparse(param_grad, param, exp_avg, exp_avg_sq, visibility, step_count, learning_rate, beta1, beta2,
                     epsilon):
    """Adam step of one [n_primitives, ...] tensor; visibility int32 [n_primitives] (> 0 = update)
    or None / an empty tensor (dense); moments float32 or bfloat16."""
    _check(param, param_grad, exp_avg, exp_avg_sq)
    if param.numel() == 0:
        return
    n_prim = param.shape[0] if param.dim() else 1
    vis = _visibility(visibility, n_prim)
    _launch([_group(param_grad, param, exp_avg, exp_avg_sq, step_count, learning_rate, beta1, beta2, epsilon)],
            n_prim, vis, param.device)


class FusedAdam(torch.optim.Adam):
    """Fused Adam over single-tensor parameter groups (each group: params=[tensor], lr, name)."""

    def __init__(self, params, lr, eps, sparse: bool = False, lowp_moment_groups: tuple = ()) -> None:
        super().__init__(params=params, lr=lr, eps=eps)
        self.sparse = sparse
        self.lowp_moment_groups = set(lowp_moment_groups)
        self.n_dense_fallbacks = 0
        from .fastergs import _Rasterize
        from .raster3d import _Rasterize3D

        _Rasterize3D.track_visibility = sparse
        _Rasterize.track_visibility = sparse

    @torch.no_grad()
    def step(self, visibility: torch.Tensor | None = None) -> None:
        """visibility: int32 [n_primitives] (> 0 = update), e.g. aux["visibility"] of the view's
        forward; None takes the last differentiable forward's (sparse only)."""
        from .raster3d import _Rasterize3D

        if not self.sparse:
            visibility = None
        elif visibility is None:
            visibility = _Rasterize3D.last_visibility
        batches: dict = {}
        for group in self.param_groups:
            assert len(group["params"]) == 1, "more than one tensor in group"
            param = group["params"][0]
            if param.grad is None or param.numel() == 0:
                continue
            lowp = group.get("name") in self.lowp_moment_groups
            moment_dtype = torch.bfloat16 if lowp else param.dtype
            state = self.state[param]
            if len(state) == 0:
                state["step"] = 0
                state["exp_avg"] = torch.zeros_like(param, dtype=moment_dtype)
                state["exp_avg_sq"] = torch.zeros_like(param, dtype=moment_dtype)
            elif state["exp_avg"].dtype != moment_dtype:
                state["exp_avg"] = state["exp_avg"].to(moment_dtype)
                state["exp_avg_sq"] = state["exp_avg_sq"].to(moment_dtype)
            state["step"] += 1
            grad = param.grad.contiguous()
            _check(param, grad, state["exp_avg"], state["exp_avg_sq"])
            n_prim = param.shape[0]
            vis = visibility
            if vis is not None and vis.numel() != n_prim:
                vis = None  # a mask of another model size: update this group densely
                self.n_dense_fallbacks += 1
            key = (n_prim, None if vis is None else vis.data_ptr(), param.device)
            b1, b2 = group["betas"]
            batches.setdefault(key, (vis, []))[1].append(
                _group(grad, param, state["exp_avg"], state["exp_avg_sq"], state["step"], group["lr"], b1, b2,
                       group["eps"]))
        for (n_prim, _, device), (vis, groups) in batches.items():
            _launch(groups, n_prim, _visibility(vis, n_prim), device)
