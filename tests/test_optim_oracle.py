"""CPU checks of the fused-Adam restatement (oracle/optim.c), mirroring the properties
cluster/tests/test_lean_adam.py:37-105 checks on the GPU: the dense update against
torch.optim.Adam (the library routine), the masked update, and the bfloat16 stochastic rounding.
"""
import numpy as np
import pytest
import torch

import optim as P


def torch_adam(p0, grads, lr, eps, betas=(0.9, 0.999)):
    p = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Adam([p], lr=lr, eps=eps, betas=betas)
    for g in grads:
        p.grad = torch.from_numpy(g)
        opt.step()
    st = opt.state[p]
    return p.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()


# The reference's update forms v' = fma(beta2, v - g*g, g*g): when g*g >> v (first steps, gradient
# spikes) the rounding of v - g*g costs up to ~2^-24 / (1 - beta2) relative in v' (~6e-5 for
# beta2 = 0.999), which torch.optim.Adam's beta2 v + (1 - beta2) g*g does not; beta is also
# rounded to float32 first (1 - 0.999 moves by 1.3e-5 relative). Hence 1e-4 on v and on the
# update, 1e-6 on m. eps = 1e-4 (> sqrt(v)) fails if eps were added inside the square root.
@pytest.mark.parametrize("betas,eps", [((0.875, 1.0 - 2.0 ** -10), 1e-8), ((0.9, 0.999), 1e-8), ((0.9, 0.999), 1e-4)])
@pytest.mark.parametrize("shape", [(1000, 3), (777, 1), (500, 15, 3)])
def test_dense_matches_torch_adam(shape, betas, eps):
    rng = np.random.default_rng(0)
    p0 = rng.standard_normal(shape).astype(np.float32)
    grads = [(rng.standard_normal(shape) * 1e-2).astype(np.float32) for _ in range(20)]
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for k, g in enumerate(grads, 1):
        P.adam_step(g, p, m, v, k, 1e-3, beta1=betas[0], beta2=betas[1], eps=eps)
    pr, mr, vr = torch_adam(p0, grads, 1e-3, eps, betas)
    assert np.abs(m - mr).max() <= 1e-6 * np.abs(mr).max()
    assert np.abs(v - vr).max() <= 1e-4 * np.abs(vr).max()
    assert np.abs((p - p0) - (pr - p0)).max() <= 1e-4 * np.abs(pr - p0).max()


def test_masked_rows():
    rng = np.random.default_rng(1)
    shape = (2000, 4)
    p0 = rng.standard_normal(shape).astype(np.float32)
    m0 = np.abs(rng.standard_normal(shape)).astype(np.float32)
    v0 = rng.random(shape).astype(np.float32)
    g = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    vis = (rng.random(shape[0]) < 0.4).astype(np.int32) * rng.integers(1, 50, shape[0]).astype(np.int32)
    pd, md, vd = p0.copy(), m0.copy(), v0.copy()
    P.adam_step(g, pd, md, vd, 7, 1e-3)
    pm, mm, vm = p0.copy(), m0.copy(), v0.copy()
    P.adam_step(g, pm, mm, vm, 7, 1e-3, visibility=vis)
    sel = vis > 0
    assert np.array_equal(pm[sel], pd[sel]) and np.array_equal(mm[sel], md[sel]) and np.array_equal(vm[sel], vd[sel])
    assert np.array_equal(pm[~sel], p0[~sel]) and np.array_equal(mm[~sel], m0[~sel])
    assert np.array_equal(vm[~sel], v0[~sel])


def test_stochastic_rounding_is_unbiased_and_uniform():
    # the noise of element i at a step is the hash of (i ^ seed): its low 16 bits must be uniform
    seed = (0x9E3779B9 * 3 + 0x85EBCA6B) & 0xFFFFFFFF
    r = np.array([P.sr_hash(i ^ seed) & 0xFFFF for i in range(20000)], np.int64)
    counts = np.bincount(r >> 12, minlength=16)  # 16 equal bins
    chi2 = float(((counts - 1250.0) ** 2 / 1250.0).sum())
    assert chi2 < 45.0  # 15 degrees of freedom, p ~ 1e-4
    # rounding a value between two bfloat16 neighbours lands on each with the right frequency
    x = np.float32(1.0 + 0.3 * 2.0 ** -7)  # 30% of the way from 1.0 to the next bfloat16
    bits = P.bf16_sr(np.full(20000, x, np.float32), np.array([P.sr_hash(i) for i in range(20000)], np.uint32))
    up = float((bits == 0x3F81).mean())
    assert set(np.unique(bits)) <= {0x3F80, 0x3F81}
    assert abs(up - 0.3) < 0.02


def test_bf16_moments_track_float32():
    rng = np.random.default_rng(2)
    shape = (4000, 3)
    p = rng.standard_normal(shape).astype(np.float32)
    pl = p.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    ml, vl = np.zeros(shape, np.uint16), np.zeros(shape, np.uint16)
    scale = (rng.random((shape[0], 1)) * 1e-3 + 1e-6).astype(np.float32)
    bias = (rng.standard_normal(shape) * scale).astype(np.float32)
    p0 = p.copy()
    for k in range(1, 301):
        g = (bias + rng.standard_normal(shape) * scale).astype(np.float32)
        P.adam_step(g, p, m, v, k, 1.25e-4)
        P.adam_step(g, pl, ml, vl, k, 1.25e-4)
    vlf = (vl.astype(np.uint32) << 16).view(np.float32)
    assert np.median(np.abs(vlf - v) / (np.abs(v) + 1e-30)) < 0.05
    dr, dl = p - p0, pl - p0
    assert np.linalg.norm(dr - dl) / np.linalg.norm(dr) < 0.02
