"""CPU check of the blends' strip culling (strip_mask_band in 3dgs-project_amd/csrc/blend.hip): a
float32 restatement of the device formula, run over every (tile, splat) pair of the oracle's
lists, never drops a strip (4 pixel rows of a tile) in which some pixel has alpha >= 1/255
under the blends' own float32 evaluation (power = a0 + dy (s2 dy + b1), clamped, 2^power). The
restatement uses exact square roots and reciprocals where the kernel uses the hardware's
approximate ones (within 1 ulp): the 0.05 px + 1e-3 relative margin covers both. The GPU
parity tests compare the culled blends with the oracle, which does not cull."""
import numpy as np
import pytest

import oracle as O
from amdsplat import scenes

f32 = np.float32
K_NH = f32(-0.5 * np.log2(np.e))
K_N = f32(-np.log2(np.e))
ALPHA_MIN = f32(1.0 / 255.0)


def fma32(a, b, c):
    return (np.asarray(a, np.float64) * b + c).astype(f32)


def band_mask(rec, tx0, ty0, ymask):
    mx, my, A, B, C, thr = (rec[:, k] for k in (0, 1, 2, 3, 4, 7))
    det = fma32(A, C, -(B * B))
    t = A + C
    cond = (det > 0) & (A > 0) & (C > 0) & (thr > 0) & (t * t < f32(4096) * det)
    m = np.zeros(len(rec), np.uint32)
    with np.errstate(all="ignore"):
        q = (thr + thr) * A
        idet = f32(1) / det
        umax = fma32(np.sqrt(q * idet), f32(1.001), f32(0.05))
        us = -B * np.sqrt((thr + thr) * (f32(1) / C) * idet)
        iA = f32(1) / A
        c0 = (tx0.astype(f32) + f32(0.5)) - mx
        c1 = c0 + f32(15)
        for s in range(4):
            ya = ((ty0 + 4 * s).astype(f32) + f32(0.5)) - my
            ua, ub = np.maximum(ya, -umax), np.minimum(ya + f32(3), umax)
            ur, ul = np.minimum(np.maximum(us, ua), ub), np.minimum(np.maximum(-us, ua), ub)
            sr = np.sqrt(np.maximum(fma32(-det * ur, ur, q), f32(0)))
            sl = np.sqrt(np.maximum(fma32(-det * ul, ul, q), f32(0)))
            fr, fl = fma32(-B, ur, sr) * iA, fma32(-B, ul, -sl) * iA
            mg = fma32(f32(1e-3), np.maximum(np.abs(fr), np.abs(fl)), f32(0.05))
            keep = (ua <= ub) & (fr + mg >= c0) & (fl - mg <= c1)
            m |= keep.astype(np.uint32) << np.uint32(s)
    return np.where(cond, m & ymask, ymask)


def dropped_hits(sc, pose):
    cam = sc.cameras[pose]
    rec, touched = O.preprocess_fwd(*[t.numpy() for t in sc.params()], cam, 3)
    keys, pl, _, _ = O.bin_instances(rec, touched, cam)
    tiles_x = (cam.width + 15) // 16
    tile = (keys >> np.uint64(32)).astype(np.int64)
    tx0, ty0 = (tile % tiles_x) * 16, (tile // tiles_x) * 16
    r = rec[pl.astype(np.int64)]
    bnd = r[:, 12:16].view(np.int32)
    ymask = np.zeros(len(r), np.uint32)
    for s in range(4):
        row0 = ty0 + 4 * s
        ymask |= ((bnd[:, 2] <= row0 + 3) & (bnd[:, 3] >= row0)).astype(np.uint32) << np.uint32(s)
    bm = band_mask(r, tx0, ty0, ymask)
    cols = np.arange(16, dtype=f32) + f32(0.5)
    bad = 0
    for s in range(4):
        idx = np.nonzero(((ymask >> s) & 1) & ~((bm >> s) & 1))[0]
        if len(idx) == 0:
            continue
        rr = r[idx]
        s0, s1, s2, o = rr[:, 2] * K_NH, rr[:, 3] * K_N, rr[:, 4] * K_NH, rr[:, 5]
        dx = rr[:, :1] - (tx0[idx, None].astype(f32) + cols[None, :])
        a0, b1 = (s0[:, None] * dx) * dx, s1[:, None] * dx
        for row in range(4):
            dy = (rr[:, 1] - ((ty0[idx] + 4 * s + row).astype(f32) + f32(0.5)))[:, None]
            pw = np.clip(fma32(dy, fma32(s2[:, None], dy, b1), a0), f32(-64), f32(0))
            bad += int(((o[:, None] * np.exp2(pw)) >= ALPHA_MIN).any(1).sum())
    kept = int(sum(((bm >> s) & 1).sum() for s in range(4)))
    before = int(sum(((ymask >> s) & 1).sum() for s in range(4)))
    return bad, kept, before


@pytest.mark.parametrize("n,W,H,scale,opacity,seed", [
    (20_000, 333, 250, (0.005, 0.08), (0.05, 0.95), 2),   # partial tiles
    (8_000, 200, 152, (0.05, 0.4), (0.3, 0.99), 3),      # large, overlapping splats
    (30_000, 321, 217, (0.0005, 0.006), (0.02, 0.99), 4),  # splats smaller than a pixel
])
def test_strip_culling_keeps_every_hit_strip_small_scenes(n, W, H, scale, opacity, seed):
    sc = scenes.small_scene(n, W, H, seed=seed, scale=scale, opacity=opacity, depth=(2.0, 8.0))
    bad, kept, before = dropped_hits(sc, 0)
    assert bad == 0 and kept <= before


def test_strip_culling_keeps_every_hit_strip_1m():
    bad, kept, before = dropped_hits(scenes.sh3_1m(), 0)
    assert bad == 0
    assert kept < 0.9 * before  # the culling removes about 13% of the strips at this size
