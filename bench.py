"""Benchmark: 3D Gaussian-splat rasterizer fwd+bwd ms/iter on one MI355X.

Workload (default, sh3_1m): 1M Gaussians, SH degree 3, 1297x840, fx=fy=1160, 8 seeded orbit
poses (radius U(3,5)); one step = forward + backward of one view (poses cycled) with a seeded
N(0,1) upstream image gradient, through the autograd operator rasterize(...) -> image.backward.
Inputs are resident in HBM before the timed region.

    python bench.py [--steps K] [--warmup W]
                    [--workload sh3_1m|sh3_3m|sh_rgb_100k|toy2d_fit|toy2d_bench|phase0_bench|l1_ssim]
                    [--no-cpu-baseline] [--no-train-step] [--no-variants] [--no-probes]
    python bench.py --probes          # only the achievable-ceiling probes (copy, read, FMA)

Prints ONE JSON line. `value` is the wall time of K autograd steps / K. A second pass over the
same K steps with HIP events between the stages gives the per-stage times and the per-pose
medians (K/8 steps per pose). `roofline` is for the kernel with the largest share of the step,
the bucketed blend backward: it is bound by the FP32 VALU issue rate, so `achieved` is its
algorithmic VALU work (a per-pair operation model over the pairs it evaluated, counted in a
separate pass) over its event-timed duration, against the published FP32 vector peak; beside it
the counter-measured issue rate (committed SQ summary), its HBM rate (algorithmic bytes) and the
achievable ceilings measured here by plain copy, read-only and FMA kernels. `train_step`
(secondary) times the full training step on the same scene: forward, L1 + D-SSIM loss,
backward and fused Adam (dense and visibility-masked), with the optimizer's HBM rate; `variants`
the inference forward, the pruning-score blend and fwd+bwd under proper antialiasing.
`cpu_baseline` is the oracle (the C restatement of the same rules) on the host cores, one view's
fwd+bwd, all cores (median of 5 after a warm-up) and one thread (median of 3).

toy2d_fit is the 2D image fit (4096 Gaussians, 256x256, L1, Adam): the GPU step through the HIP
kernels, beside the dense PyTorch reference path (render_reference) on the host cores.
toy2d_bench and phase0_bench time the 2D extensions' kernels alone on the reference's own bench
scenes (toy2d/bench.py, bench/phase0/backward_bench.py), beside the reference's published figures.
l1_ssim times the fused L1 + D-SSIM loss kernels alone on the 1M workload's frame size.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "3dgs-project_amd"))

HBM_PEAK_GBS = 8000.0
# FP32 VALU lane operations per second: the published 157.3 TFLOP/s FP32 vector peak with an
# FMA counted as 2 FLOP (one lane operation)
VALU_PEAK_TOPS = 157.3 / 2
# The issue rate this build can reach: the published peak counts packed FP32 (two lanes' worth per
# v_pk_* instruction), which the build does not use, so plain VALU instructions issue at half of
# it: one wave64 instruction per 4 cycles per SIMD, 4 SIMDs x 256 CUs at 2.4 GHz
VALU_ISSUE_PEAK_INSTR = 256 * 4 * 2.4e9 / 4
METRIC = "fwd+bwd ms/iter @1M Gaussians SH3 1297x840; per-stage HBM GB/s vs roofline"
# stages that are one kernel each (the others group several kernels)
SINGLE_KERNEL = {"preprocess": "preprocess_fwd_kernel", "blend_fwd": "blend_fwd_strip_kernel",
                 "blend_bwd": "blend_bwd_bucket_kernel", "preprocess_bwd": "preprocess_bwd_kernel"}
# VALU work model of the 3D bucketed blend backward (lane operations, an FMA counted once):
# per evaluated (pixel, splat) pair, the falloff (dy, power 2 FMA, exp2, times opacity, alpha
# test and select), T alpha, the colour dot (3), the three colour sums, rho, 1 - alpha, the
# clamp and reciprocal, dL/dalpha (2), dL/dpower and its dy factor, the three power sums and the
# T update: 27; per splat and lane of a walked bucket, the column terms (dx, a0 (2), b1, and the
# two mean-gradient column factors): 6; per splat a bucket reduces, 9 values summed over 64
# lanes: 9 * 63.
OPS_PER_PAIR, OPS_PER_STEP_LANE, OPS_PER_REDUCTION = 27, 6, 9 * 63


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=160)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", default="sh3_1m",
                    choices=["sh3_1m", "sh3_3m", "sh_rgb_100k", "toy2d_fit", "toy2d_bench", "phase0_bench", "l1_ssim"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=5, help="all-core CPU baseline runs (median)")
    ap.add_argument("--cpu-single-runs", type=int, default=3, help="single-thread CPU baseline runs (0 = skip)")
    ap.add_argument("--probes", action="store_true", help="only run the copy / read / FMA probes and exit")
    ap.add_argument("--no-probes", action="store_true")
    ap.add_argument("--no-train-step", action="store_true", help="skip the training-step measurement")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the inference / pruning-score / antialiasing variants (profiling runs)")
    ap.add_argument("--binning", default="auto", choices=["auto", "radix", "spans"],
                    help="the tile binning of the 3D workloads (auto: the library's choice for the size)")
    ap.add_argument("--json-out", default=None)
    return ap.parse_args()


# ---------------------------------------------------------------------------------------
# Achievable ceilings
# ---------------------------------------------------------------------------------------
def _event_ms(fn, reps: int, warmup: int = 3) -> float:
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def probes() -> dict:
    """Plain copy and read-only sweeps of 1 GiB (well beyond the last-level cache) and
    independent FP32 FMA chains on every SIMD, launched by the library on the current stream."""
    import torch

    from amdsplat import _lib
    from amdsplat._lib import call, ptr

    st = _lib.stream_handle()
    n = 1 << 28  # floats: 1 GiB
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    sums = torch.empty(_lib.size_call("gs_probe_read_sums", n), device="cuda")
    copy_ms = _event_ms(lambda: call("gs_probe_copy", ptr(a), ptr(b), n, st), 10)
    read_ms = _event_ms(lambda: call("gs_probe_read", ptr(a), n, ptr(sums), st), 10)
    del a, b, sums
    threads, iters = 256 * 4 * 8 * 64, 2048  # 8 wavefronts per SIMD
    out = torch.empty(threads, device="cuda")
    fma_ms = _event_ms(lambda: call("gs_probe_fma", ptr(out), threads, iters, st), 5)
    fma_ops = threads * iters * 64  # 16 chains x 4 per iteration
    return {"copy_gbs": round(8 * n / (copy_ms * 1e6), 1), "read_gbs": round(4 * n / (read_ms * 1e6), 1),
            "fma_tops": round(fma_ops / (fma_ms * 1e-3) / 1e12, 2),
            "note": "copy: 1 GiB read + 1 GiB written; read: 1 GiB read; fma: 16 independent v_fma_f32 chains per "
                    "lane, 8 wavefronts per SIMD, T lane-op/s (the 157.3 TFLOP/s peak counts packed FP32, two "
                    "lanes per instruction, which this build does not use)"}


# ---------------------------------------------------------------------------------------
# 3D workloads
# ---------------------------------------------------------------------------------------
def span_count(fs) -> int:
    """Row spans of a forward (distinct (Gaussian, tile row) pairs of its instances): the unit
    of the span binning's traffic."""
    import torch

    rg = fs.ranges.long()
    T, tx, ty = fs.cam.n_tiles, fs.cam.tiles_x, fs.cam.tiles_y
    tile = torch.repeat_interleave(torch.arange(T, device=rg.device), rg[:, 1] - rg[:, 0])
    key = fs.point_list.long() * ty + tile // tx
    return int(torch.unique(key).numel())


def stage_bytes(fs, n_visible, active_buckets, splat_steps, used_pairs, staged, ckpt_written,
                atomics_per_pair=9, spans=None):
    """Algorithmic (compulsory) HBM bytes per stage for the measured counts: each datum read or
    written once (fp32). spans: the row-span count when the forward took the span binning (its
    instance offsets are None), else None. The path is the forward's: no offsets for the span
    binning."""
    n, m, K = fs.n, fs.m, fs.sh_coeffs
    T = fs.cam.n_tiles
    P = fs.cam.width * fs.cam.height
    B = int(fs.bucket_offsets[-1].item())
    # the depth sort: 3 radix passes over N (histogram read 4 B, key+value read and write 16 B),
    # the last one also gathering the counts into depth order (read + write 8 B)
    sub = {"depth_sort": 3 * 20 * n + (8 * n if spans is None else 0)}
    if spans is None:
        # the scan of the counts in depth order (read, offsets written)
        sub["instance_offsets"] = 8 * n
        # tile keys of 16 bits below 65536 tiles, else 32
        kb = 2 if T <= 65536 else 4
        # emission: order and offset per Gaussian, 48 B of the record of the visible, key + value
        # per instance; tile sort pass 1 (histogram read kb, key+value read and written) and
        # pass 2 (histogram kb, key+value read, value written); ranges and bucket offsets
        sub["key_duplication"] = 8 * n + 48 * n_visible + (kb + 4) * m
        sub["tile_sort"] = (kb + 2 * (kb + 4)) * m + (kb + (kb + 4) + 4) * m
        sub["ranges_buckets"] = 20 * T + 4 * B
        depth = sub["depth_sort"] + sub["instance_offsets"]
    else:
        # rows: order 4 B and 48 B of the record of the visible per Gaussian, each span gathered
        # (8 B written, read) and placed by row (8 B written); columns: each span read by the
        # column count (8 B), tile counts; the write: each span read (8 B), the point list 4 B per
        # instance, ranges and bucket offsets
        sub["span_rows"] = 4 * n + 48 * n_visible + 24 * spans
        sub["span_columns"] = 8 * spans + 4 * T
        sub["span_write"] = 8 * spans + 4 * m + 16 * T + 4 * B
        depth = sub["depth_sort"]
    binning = sum(v for k, v in sub.items() if k not in ("depth_sort", "instance_offsets"))
    return {
        # params 44 B/Gaussian + tiles_touched and depth key 8 B; SH 12 K B and the 64 B record
        # per visible one; the empty bounds (16 B) of each culled one's record
        "preprocess": 44 * n + 8 * n + n_visible * (12 * K + 64) + 16 * (n - n_visible),
        "depth_order": depth,
        "binning": binning,
        # per staged list entry: id + 64 B record; per pixel: image 12 + final T 4 + n_contrib 4;
        # the checkpoints written (4 KiB per bucket reached); tile max, bucket_to_tile, and the
        # backward's screen-space gradient buffer the forward zeroes (48 B of float32 sums and
        # 32 B of float64 conic sums per Gaussian)
        "blend_fwd": staged * (4 + 64) + P * 20 + ckpt_written * 4096 + 4 * T + 4 * B + 80 * n,
        # per active bucket: checkpoints 4 KiB + grad image 12, image 12, n_contrib 4 per pixel;
        # per bucket-splat step: id + record; per reduced bucket-splat: 9 fp32 atomics (11 with
        # the |dL/dmean2d| sums)
        "blend_bwd": active_buckets * (4096 + 256 * 28) + splat_steps * (4 + 64) + used_pairs * 4 * atomics_per_pair,
        # tiles_touched of every Gaussian; params, SH and grad2d of the visible (the colour clamp
        # is recomputed from the SH rows, the record is not read); every output row written
        "preprocess_bwd": 4 * n + n_visible * (44 + 12 * K + 48) + n * (44 + 12 * K),
        "substages": sub,
    }


def substage_times(step, k_steps: int) -> dict:
    """Mean ms of each stage the library marks inside its calls (gs_stage_marks), over k_steps
    steps; each step is waited for before the next."""
    import torch

    from amdsplat import _lib

    L = _lib.lib()
    cap = 64
    ms = (ctypes.c_float * cap)()
    names = (ctypes.c_char_p * cap)()
    acc = {}
    torch.cuda.synchronize()
    for k in range(k_steps):
        L.gs_stage_marks(1)
        step(k)
        n = L.gs_stage_marks_read(ms, names, cap)
        L.gs_stage_marks(0)
        if n < 0:
            raise RuntimeError(L.gs_last_error().decode())
        for i in range(n):
            name = names[i].decode()
            if name != "start":
                acc.setdefault(name, []).append(ms[i])
    return {k2: statistics.mean(v) for k2, v in acc.items()}


def bucket_stats(fs):
    """(active buckets, sum of tile_max, staged list entries, checkpoints written) of a forward:
    the forward blend stages 256 list entries at a time and stops after the batch in which every
    pixel of the tile has stopped (at or after its tile_max)."""
    import numpy as np

    boff = fs.bucket_offsets.cpu().numpy().astype(np.int64)
    tmax = fs.tile_max.cpu().numpy().astype(np.int64)
    rg = fs.ranges.cpu().numpy().astype(np.int64)
    length = rg[:, 1] - rg[:, 0]
    nbk = np.diff(boff)
    active = np.minimum(nbk, (tmax + 31) // 32)
    staged = np.minimum(length, (tmax + 255) // 256 * 256)
    return int(active.sum()), int(tmax.sum()), int(staged.sum()), int(((staged + 31) // 32).sum())


def _profile_value(name: str, key: str, workload: str):
    """A figure from a committed profile summary, if that summary was measured on `workload`
    (its heading ends with the workload's name); None otherwise."""
    f = ROOT / "profiles" / name
    if not f.exists():
        return None
    text = f.read_text()
    head = text.splitlines()[0] if text else ""
    if not head.rstrip().endswith(workload):
        return None
    m = re.search(rf"{key}:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, calibrated with a plain copy) of the same workload, or None."""
    return _profile_value(f"{kernel}_hbm_traffic.md", "traffic_bytes_per_launch", workload)


def measured_valu_instr(kernel: str, workload: str):
    """VALU instructions per launch of `kernel` from the committed rocprofv3 SQ summary of the same
    workload, or None."""
    return _profile_value(f"{kernel}_sq.md", "valu_instr_per_launch", workload)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _omp_threads(n: int) -> None:
    """Sets the OpenMP thread count of the oracle's parallel loops (libgomp, already loaded)."""
    ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))


def _median_runs(fn, runs: int) -> tuple[float, list]:
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def cpu_baseline_3d(scene, pose: int, runs: int, single_runs: int) -> dict:
    """The C oracle (the CPU restatement of the same rules) timed on the host: one full fwd+bwd of
    one view of the workload, all cores (median of `runs` after a warm-up) and one thread. The
    preprocess, the forward and backward blends (tile-parallel) and the preprocess backward run on
    OpenMP threads; the binning is serial (instances emitted, then one qsort)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    cam = scene.cameras[pose]
    p = [t.numpy() for t in scene.params()]
    gi = np.random.default_rng(0).standard_normal((3, cam.height, cam.width)).astype(np.float32)
    deg = int(round(scene.sh.shape[1] ** 0.5)) - 1

    def once():
        r = O.render(*p, cam, deg)
        g2 = O.blend_bwd(r["rec"], r["point_list"], r["ranges"], r["bucket_offsets"], cam.width, cam.height,
                         r["image"], gi, r["final_T"], r["n_contrib"], r["tile_max"], r["ckpt"], scene.n)
        O.preprocess_bwd(*p, cam, deg, r["rec"], r["touched"], g2)

    cores = os.cpu_count() or 1
    once()  # warm-up (also loads and builds the oracle)
    _omp_threads(cores)
    med, times = _median_runs(once, runs)
    out = {"value": round(med * 1000.0, 1), "unit": "ms/iter", "cores": cores, "kind": "port",
           "runs_s": [round(t, 2) for t in times], "nproc": os.cpu_count(), "cpu_model": cpu_model(),
           "sample": f"the C oracle's fwd+bwd of pose {pose} of this workload, all {scene.n} Gaussians: median of "
                     f"{runs} runs after a warm-up, {cores} OpenMP threads (preprocess, forward blend, "
                     f"backward blend and preprocess backward parallel; the binning serial: instance "
                     f"emission and one qsort)"}
    if single_runs > 0:
        _omp_threads(1)
        smed, stimes = _median_runs(once, single_runs)
        _omp_threads(cores)
        out["single_thread"] = {"value": round(smed * 1000.0, 1), "unit": "ms/iter", "cores": 1,
                                "runs_s": [round(t, 2) for t in stimes],
                                "sample": f"the same view, one thread, median of {single_runs} runs"}
    return out


# learning rates of the training-step workload (means, log-scales, quats, SH DC, SH rest, opacity)
TRAIN_LR = {"means": 1.6e-4, "scales": 5e-3, "quats": 1e-3, "sh_dc": 2.5e-3, "sh_rest": 1.25e-4, "opacity": 5e-2}


def _K(c):
    import torch

    return torch.tensor([[c.fx, 0.0, c.cx], [0.0, c.fy, c.cy], [0.0, 0.0, 1.0]])


def train_step_bench(scene, steps: int, warmup: int) -> dict:
    """The full training step on the same scene: forward, L1 + D-SSIM (lambda 0.2) against a
    seeded U(0,1) target, backward, fused Adam over all 59 parameters per Gaussian (dense, and
    masked to the Gaussians visible in the view). Poses cycle as in the main measurement."""
    import torch

    from amdsplat import FusedAdam, l1_ssim_loss, rasterize

    sc = scene.to("cuda")
    m, ls, q, op, sh = [t.contiguous() for t in sc.params()]
    P = {"means": m, "scales": ls, "quats": q, "opacity": op, "sh_dc": sh[:, :1].contiguous(),
         "sh_rest": sh[:, 1:].contiguous()}
    cams = sc.cameras
    g = torch.Generator().manual_seed(4321)
    targets = [torch.rand(3, c.height, c.width, generator=g).cuda() for c in cams]
    Ks = [_K(c) for c in cams]
    n = m.shape[0]
    n_par = sum(t[0].numel() for t in P.values())  # fp32 parameters per Gaussian
    deg = int(round(sh.shape[1] ** 0.5)) - 1
    # Adam moves 28 bytes per element: reads parameter, gradient and both moments, writes
    # parameter and both moments
    row_bytes = 28 * n_par
    out = {"workload": f"{n} Gaussians SH{deg} {cams[0].width}x{cams[0].height}: fwd, L1+D-SSIM (11x11, lambda 0.2), "
                       f"bwd, fused Adam over {n_par} fp32 parameters per Gaussian",
           "lr": TRAIN_LR}
    for mode in ("dense", "masked"):
        params = {k: torch.nn.Parameter(v.clone()) for k, v in P.items()}
        groups = [{"params": [params[k]], "lr": lr, "name": k} for k, lr in TRAIN_LR.items()]
        opt = FusedAdam(groups, lr=0.0, eps=1e-15, sparse=(mode == "masked"))

        def step(k, ev=None):
            c = cams[k % len(cams)]
            img, _, aux = rasterize(params["means"], params["scales"], params["quats"], params["opacity"],
                                    (params["sh_dc"], params["sh_rest"]), c.viewmat, Ks[k % len(cams)], c.width,
                                    c.height, near=c.near, far=c.far)
            loss = l1_ssim_loss(img, targets[k % len(cams)], 0.2)
            loss.backward()
            if ev:
                ev[0].record()
            opt.step(visibility=aux["visibility"])
            if ev:
                ev[1].record()
            opt.zero_grad(set_to_none=True)
            return aux["tiles_touched"]

        for k in range(warmup):
            step(k)
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        t0 = time.perf_counter()
        touched = []
        for k in range(steps):
            touched.append(step(k, evs[k]))
        torch.cuda.synchronize()
        step_ms = (time.perf_counter() - t0) * 1000.0 / steps
        adam_ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
        vis_sum = sum(int((t > 0).sum().item()) for t in touched) / steps
        nbytes = row_bytes * n if mode == "dense" else int(row_bytes * vis_sum) + 4 * n
        out[mode] = {"step_ms": round(step_ms, 4), "adam_ms": round(adam_ms, 4),
                     "adam_hbm_gbs": round(nbytes / (adam_ms * 1e6), 1),
                     "adam_hbm_frac": round(nbytes / (adam_ms * 1e6) / HBM_PEAK_GBS, 4),
                     "adam_algorithmic_bytes": nbytes, "visible_per_view": round(vis_sum)}
        from amdsplat.fastergs import _Rasterize
        from amdsplat.raster3d import _Rasterize3D

        _Rasterize3D.track_visibility = False
        _Rasterize.track_visibility = False
    out["loss_kernels"] = loss_kernel_times(targets[0], max(steps, 20))
    return out


def loss_kernel_times(target, reps: int) -> dict:
    """Event-timed gs_l1_ssim_fwd (with the backward's per-pixel map) and gs_l1_ssim_bwd on an
    image of the target's size, each launched `reps` times back to back. Algorithmic bytes: the
    forward reads both images and writes the map (3 floats per pixel and channel), the backward
    reads the images and the map and writes the image gradient."""
    import torch

    from amdsplat import _lib
    from amdsplat._lib import call, ptr

    C, H, W = target.shape
    x = torch.rand(C, H, W, generator=torch.Generator().manual_seed(5)).cuda()
    dmap = torch.empty(C, 3, H, W, device="cuda")
    loss = torch.empty(3, device="cuda")
    g = torch.empty_like(x)
    ws = torch.empty(max(_lib.size_call("gs_l1_ssim_workspace_size", C, H, W), 1), dtype=torch.uint8, device="cuda")
    st = _lib.stream_handle()
    fwd = _event_ms(lambda: call("gs_l1_ssim_fwd", ptr(x), ptr(target), C, H, W, 0.2, ptr(dmap), ptr(loss), ptr(ws),
                                 ws.numel(), st), reps)
    bwd = _event_ms(lambda: call("gs_l1_ssim_bwd", ptr(x), ptr(target), ptr(dmap), C, H, W, 0.2, None, ptr(g), st),
                    reps)
    px = C * H * W
    fb, bb = 4 * px * (2 + 3), 4 * px * (2 + 3 + 1)
    return {"image": [C, H, W],
            "fwd_ms": round(fwd, 4), "fwd_hbm_gbs": round(fb / (fwd * 1e6), 1), "fwd_algorithmic_bytes": fb,
            "bwd_ms": round(bwd, 4), "bwd_hbm_gbs": round(bb / (bwd * 1e6), 1), "bwd_algorithmic_bytes": bb}


def variants_bench(sc, grads, steps: int, warmup: int) -> dict:
    """ms per view of the path's variants on the same scene and poses: the inference forward (no
    backward state), the pruning-score blend (preprocess, binning, summed blending weights),
    fwd+bwd under proper antialiasing, and fwd+bwd with the |dL/dmean2d| sums that densification
    by absolute gradient reads."""
    import dataclasses

    import torch

    from amdsplat import raster3d as R

    params = sc.params()
    cams = sc.cameras
    Ks = [_K(c) for c in cams]
    scores = torch.zeros(params[0].shape[0], dtype=torch.float32, device="cuda")
    aa_cams = [dataclasses.replace(c, proper_antialiasing=True) for c in cams]

    def inference(k):
        c = cams[k % len(cams)]
        R.rasterize_inference(*params, c.viewmat, Ks[k % len(cams)], c.width, c.height, near=c.near, far=c.far)

    def pruning(k):
        c = cams[k % len(cams)]
        R.pruning_scores(*params, c.viewmat, Ks[k % len(cams)], c.width, c.height, near=c.near, far=c.far,
                         scores=scores)

    def aa_fwd_bwd(k):
        fs = R.forward_pass(*params, aa_cams[k % len(cams)])
        R.backward_pass(fs, *params, grads[k % len(cams)], abs_grad=False)

    def abs_fwd_bwd(k):
        fs = R.forward_pass(*params, cams[k % len(cams)])
        R.backward_pass(fs, *params, grads[k % len(cams)], abs_grad=True)

    out = {}
    for name, fn in (("inference_fwd", inference), ("pruning_scores", pruning),
                     ("proper_antialiasing_fwd_bwd", aa_fwd_bwd), ("abs_grad_fwd_bwd", abs_fwd_bwd)):
        for k in range(warmup):
            fn(k)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(steps):
            fn(k)
        torch.cuda.synchronize()
        out[name + "_ms"] = round((time.perf_counter() - t0) * 1000.0 / steps, 4)
    return out


def bench_3d(args, ceilings) -> dict:
    import dataclasses

    import torch

    from amdsplat import _lib
    from amdsplat import raster3d as R
    from amdsplat import rasterize, scenes

    make = {"sh3_1m": scenes.sh3_1m, "sh3_3m": scenes.sh3_3m, "sh_rgb_100k": scenes.sh_rgb_100k}[args.workload]
    scene = make()
    sc = scene.to("cuda")
    params = sc.params()
    R.BINNING = args.binning
    cams = [dataclasses.replace(c, binning=args.binning) for c in sc.cameras]
    Ks = [_K(c) for c in cams]
    g = torch.Generator().manual_seed(1234)
    grads = [torch.randn(3, c.height, c.width, generator=g).cuda() for c in cams]
    leaves = [t.clone().requires_grad_(True) for t in params]

    def autograd_step(k):
        """The headline operator: rasterize(...) -> image, then image.backward(grad)."""
        pose = k % len(cams)
        c = cams[pose]
        for t in leaves:
            t.grad = None
        img, _, _ = rasterize(*leaves, c.viewmat, Ks[pose], c.width, c.height, near=c.near, far=c.far)
        img.backward(grads[pose])

    def step(k, timer=None, counters=None):
        pose = k % len(cams)
        fs = R.forward_pass(*params, cams[pose], sh_degree=None, timing=timer if timer else False)
        out = R.backward_pass(fs, *params, grads[pose], timing=timer if timer else False, counters=counters,
                              abs_grad=False)
        return fs, out

    def timed(fn, k_steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(k_steps):
            fn(k)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1000.0 / k_steps

    for k in range(args.warmup):
        autograd_step(k)
        step(k)
    # the timed region: K autograd steps, nothing recorded between the stages
    wall_ms = timed(autograd_step, args.steps)
    # the same K steps through forward_pass / backward_pass (no autograd bookkeeping)
    low_ms = timed(lambda k: step(k), args.steps)

    # the per-stage breakdown: the same K steps again with HIP events between the stages (the
    # events cost a few microseconds each, so this pass is not the headline number)
    timers = [R.StageTimer(True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for k in range(args.steps):
        step(k, timers[k])
    torch.cuda.synchronize()
    staged_wall_ms = (time.perf_counter() - t1) * 1000.0 / args.steps

    # the binning chain's sub-stages, from the library's stage marks (HIP events between its
    # kernels), over one more pass of the same steps, each step waited for before the next
    mark_steps = max(len(cams), min(args.steps, 4 * len(cams)))
    sub_ms = substage_times(lambda k: step(k), mark_steps)

    per_stage = {}
    step_ms = []
    pose_ms = [[] for _ in cams]
    for k, tm in enumerate(timers):
        r = tm.result(sync=False)
        step_ms.append(sum(r.values()))
        pose_ms[k % len(cams)].append(step_ms[-1])
        for k2, v in r.items():
            per_stage.setdefault(k2, []).append(v)
    stage_ms = {k2: statistics.mean(v) for k2, v in per_stage.items()}
    # per pose: the median over its event-timed steps; then the median and the max over the poses
    pose_medians = [statistics.median(v) for v in pose_ms if v]

    # counts for the byte and operation models: one counting step per pose outside the timed
    # regions, averaged over the poses like the timings
    per_pose, paths = [], set()
    for pose in range(len(cams)):
        ctr = torch.zeros(3, dtype=torch.int64, device="cuda")
        fs, _ = step(pose, counters=ctr)
        torch.cuda.synchronize()
        nv = int((fs.touched > 0).sum().item())
        ab, ss, stg, ckw = bucket_stats(fs)
        up = int(ctr[0].item()) // 9
        ev = int(ctr[2].item())
        spans = span_count(fs) if fs.path == _lib.GS_BIN_PATH_SPANS else None
        paths.add("spans" if fs.path == _lib.GS_BIN_PATH_SPANS else "radix")
        per_pose.append({"visible": nv, "instances": fs.m, "buckets": int(fs.bucket_offsets[-1].item()),
                         "active_buckets": ab, "bucket_splat_steps": ss, "staged_entries": stg,
                         "ckpt_written": ckw, "reduced_bucket_splats": up, "bwd_pair_evals": ev,
                         "bwd_valu_ops": OPS_PER_PAIR * ev + OPS_PER_STEP_LANE * 64 * ss + OPS_PER_REDUCTION * up,
                         **({"row_spans": spans} if spans is not None else {}),
                         "bytes": stage_bytes(fs, nv, ab, ss, up, stg, ckw, spans=spans)})
    counts = {k2: round(statistics.mean(pp[k2] for pp in per_pose)) for k2 in per_pose[0] if k2 != "bytes"}
    sb = {k2: statistics.mean(pp["bytes"][k2] for pp in per_pose) for k2 in per_pose[0]["bytes"]
          if k2 != "substages"}
    sub_bytes = {k2: statistics.mean(pp["bytes"]["substages"].get(k2, 0) for pp in per_pose)
                 for k2 in per_pose[0]["bytes"]["substages"]}
    substages = {k2: {"ms": round(v, 4), "algorithmic_bytes": round(sub_bytes[k2]),
                      "hbm_gbs": round(sub_bytes[k2] / (v * 1e6), 1) if v > 0 else None,
                      "hbm_frac": round(sub_bytes[k2] / (v * 1e6) / HBM_PEAK_GBS, 4) if v > 0 else None}
                 for k2, v in sub_ms.items() if k2 in sub_bytes}
    stage_gbs = {k2: sb[k2] / (stage_ms[k2] * 1e6) for k2 in stage_ms if k2 in sb and stage_ms[k2] > 0}
    dominant = max((k2 for k2 in stage_ms if k2 in SINGLE_KERNEL), key=lambda k2: stage_ms[k2])
    kernel = SINGLE_KERNEL[dominant]
    t_dom = stage_ms[dominant]
    hbm = {"achieved": round(stage_gbs[dominant], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(stage_gbs[dominant] / HBM_PEAK_GBS, 4), "algorithmic_bytes": round(sb[dominant])}
    if ceilings:
        hbm["achievable"] = ceilings["copy_gbs"]
        hbm["frac_of_achievable"] = round(stage_gbs[dominant] / ceilings["copy_gbs"], 4)
    if dominant == "blend_bwd":
        ops = counts["bwd_valu_ops"]
        tops = ops / (t_dom * 1e-3) / 1e12
        roof = {"kernel": kernel, "bound": "valu", "achieved": round(tops, 3), "peak": VALU_PEAK_TOPS,
                "unit": "T FP32 lane-op/s (157.3 TFLOP/s with an FMA as 2)", "frac": round(tops / VALU_PEAK_TOPS, 4),
                "traffic": measured_traffic(kernel, args.workload), "algorithmic_ops": ops,
                "ops_model": f"{OPS_PER_PAIR} per evaluated pair + {OPS_PER_STEP_LANE} per lane and bucket-splat "
                             f"step + {OPS_PER_REDUCTION} per reduced bucket-splat",
                "avg_launch_ms": round(t_dom, 4), "hbm": hbm}
        if ceilings:
            roof["achievable"] = ceilings["fma_tops"]
            roof["frac_of_achievable"] = round(tops / ceilings["fma_tops"], 4)
    else:
        roof = {"kernel": kernel, "bound": "hbm", **{k: v for k, v in hbm.items() if k != "algorithmic_bytes"},
                "traffic": measured_traffic(kernel, args.workload), "algorithmic_bytes": hbm["algorithmic_bytes"],
                "avg_launch_ms": round(t_dom, 4)}
    valu_instr = measured_valu_instr(kernel, args.workload)
    if valu_instr:
        rate = valu_instr / (t_dom * 1e-3)
        roof["issue"] = {"valu_instr_per_launch": valu_instr, "achieved": round(rate / 1e12, 4),
                         "peak": round(VALU_ISSUE_PEAK_INSTR / 1e12, 4),
                         "unit": "T wave64 VALU instr/s (plain FP32 issue: 1 per 4 cycles per SIMD at 2.4 GHz)",
                         "frac": round(rate / VALU_ISSUE_PEAK_INSTR, 4)}
    atomics = _profile_value(f"{kernel}_atomics.md", "atomic_requests_per_launch", args.workload)
    if atomics:
        roof["atomic_requests_per_launch"] = atomics

    views = f"{len(cams)} orbit poses" if len(cams) > 1 else "one camera"
    fs_cam = cams[0]
    out = {
        "metric": METRIC,
        "value": round(wall_ms, 4),
        "unit": "ms/iter",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator; random-init Gaussians of the configured distribution)",
        "config": {"workload": f"{args.workload}: {scene.n} Gaussians SH{int(round(scene.sh.shape[1] ** 0.5)) - 1} "
                               f"{fs_cam.width}x{fs_cam.height}, fwd+bwd per view through rasterize(...) and "
                               f"autograd, {views}",
                   "gaussians": scene.n, "width": fs_cam.width, "height": fs_cam.height,
                   "tile_binning": "+".join(sorted(paths)),
                   "parallelism": "single GPU"},
        "low_level_ms_per_step": round(low_ms, 4),
        "stage_ms": {k2: round(v, 4) for k2, v in stage_ms.items()},
        "binning_substages": substages,
        "stage_hbm_gbs": {k2: round(v, 1) for k2, v in stage_gbs.items()},
        "stage_hbm_frac": {k2: round(v / HBM_PEAK_GBS, 4) for k2, v in stage_gbs.items()},
        "event_sum_ms": round(statistics.mean(step_ms), 4),
        "per_pose_ms": {"median": round(statistics.median(pose_medians), 4), "max": round(max(pose_medians), 4),
                        "steps_per_pose": args.steps // len(cams), "poses": [round(v, 4) for v in pose_medians]},
        "staged_pass_ms_per_step": round(staged_wall_ms, 4),
        "counts": counts,
        "roofline": roof,
    }
    if ceilings:
        out["achievable"] = ceilings
        out["stage_hbm_frac_of_achievable"] = {k2: round(v / ceilings["copy_gbs"], 4) for k2, v in stage_gbs.items()}
    if not args.no_variants:
        out["variants"] = variants_bench(sc, grads, steps=max(args.steps // 4, 16), warmup=4)
    if not args.no_train_step:
        out["train_step"] = train_step_bench(scene, steps=max(args.steps // 4, 16), warmup=4)
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline_3d(scene, 0, args.cpu_runs, args.cpu_single_runs)
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"error": repr(e)}
    return out


# ---------------------------------------------------------------------------------------
# 2D image fit (toy2d rules)
# ---------------------------------------------------------------------------------------
FIT_LR = lambda H, W: {"xy": 0.002 * max(H, W) / 10, "log_scale": 0.01, "theta": 0.01, "rgb_logit": 0.02,  # noqa: E731
                       "opacity_logit": 0.02}


def _fit_optimizer(model, H, W, fused: bool = False):
    """The fit's Adam: torch.optim.Adam's update (lr per parameter, eps 1e-8), as the reference's
    toy2d/fit.py:67-73 builds it; fused: the same update in one launch for all five groups
    (FusedAdam, gs_adam_step)."""
    import torch

    lr = FIT_LR(H, W)
    groups = [{"params": [getattr(model, k)], "lr": v, "name": k} for k, v in lr.items()]
    if fused:
        from amdsplat import FusedAdam

        return FusedAdam(groups, lr=0.0, eps=1e-8)
    return torch.optim.Adam(groups)


def cpu_baseline_toy2d(bins_cpu, runs: int, single_runs: int) -> dict:
    """The reference's CPU path of the fit, restated (gs2d.render_reference: every Gaussian
    against every pixel in PyTorch ops): activate, dense render, L1, autograd backward and Adam
    on the host cores, with the tile rectangles and depth order of the first step's binning (the
    binning is a small part of the step)."""
    import torch

    from gs2d import render_reference
    from gs2d.params import fit_model_4k

    model, target = fit_model_4k()
    opt = _fit_optimizer(model, 256, 256)

    def once():
        means, conic, color, opacity, _ = model.activated()
        img = render_reference(means, conic, color, opacity, bins_cpu)
        loss = (img - target).abs().mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()

    cores = torch.get_num_threads()
    once()
    med, times = _median_runs(once, runs)
    out = {"value": round(med * 1000.0, 1), "unit": "ms/iter", "cores": cores, "kind": "port",
           "runs_s": [round(t, 3) for t in times], "nproc": os.cpu_count(), "cpu_model": cpu_model(),
           "sample": f"one fit step of this workload on the dense reference path (render_reference, PyTorch CPU, "
                     f"{cores} threads): median of {runs} runs after a warm-up"}
    if single_runs > 0:
        torch.set_num_threads(1)
        smed, stimes = _median_runs(once, single_runs)
        torch.set_num_threads(cores)
        out["single_thread"] = {"value": round(smed * 1000.0, 1), "unit": "ms/iter", "cores": 1,
                                "runs_s": [round(t, 3) for t in stimes],
                                "sample": f"the same step, one thread, median of {single_runs} runs"}
    return out


def bench_toy2d(args, ceilings) -> dict:
    import torch

    from amdsplat import raster3d as R
    from gs2d import bin_gaussians, rasterize
    from gs2d.params import fit_model_4k, radii_from_cov
    from gs2d.raster import ext

    H = W = 256
    model, target = fit_model_4k()
    model = model.cuda()
    target = target.cuda()
    opt = _fit_optimizer(model, H, W, fused=True)

    def step(k, timer=None):
        tm = timer if timer is not None else R.StageTimer(False)
        tm.mark("start")
        # activate + radii_from_cov (toy2d/fit.py:77-78) in one launch, its backward in one more
        means, conic, color, opacity, cov, radii = model.activated_fused()
        bins = bin_gaussians(means, radii, model.depth, H, W)
        tm.mark("binning")
        img = rasterize(means, conic, color, opacity, bins, backend="splat")
        tm.mark("forward")
        loss = (img - target).abs().mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        tm.mark("backward")
        opt.step()
        tm.mark("adam")
        return bins

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        bins = step(k)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    timers = [R.StageTimer(True) for _ in range(args.steps)]
    for k in range(args.steps):
        step(k, timers[k])
    torch.cuda.synchronize()
    stage_ms = {}
    for tm in timers:
        for k2, v in tm.result(sync=False).items():
            stage_ms.setdefault(k2, []).append(v)
    stage_ms = {k2: statistics.mean(v) for k2, v in stage_ms.items()}

    # the kernels alone, as the reference's bench times them (toy2d/bench.py:48-73): forward with
    # checkpoints and the bucketed backward, on the current parameters
    with torch.no_grad():
        means, conic, color, opacity, cov = (t.contiguous() for t in model.activated())
        bins = bin_gaussians(means, radii_from_cov(cov), model.depth, H, W)
    e = ext()
    bg = torch.zeros(3, device="cuda")
    dout = torch.randn(3, H, W, generator=torch.Generator().manual_seed(7)).cuda()
    common = (means, conic, color, opacity, bg, bins.ranges, bins.point_list)
    out_s, final_T, n_contrib, bstate = e.forward(*common, bins.bucket_offsets, bins.num_buckets, H, W, True)
    fwd_ms = _event_ms(lambda: e.forward(*common, bins.bucket_offsets, bins.num_buckets, H, W, True), 50)
    bwd_ms = _event_ms(lambda: e.backward_splat(*common, bins.bucket_offsets, bins.bucket_to_tile, out_s, final_T,
                                                n_contrib, bstate, dout), 50)
    m = int(bins.point_list.numel())
    nb = int(bins.num_buckets)
    n = means.shape[0]
    P = H * W
    # algorithmic bytes: forward -- ids and 64-byte records of every list entry, image / final T /
    # n_contrib per pixel, 4 KiB of checkpoints per bucket; backward -- checkpoints, grad image,
    # image and n_contrib per bucket pixel, ids and records per entry, 9 atomics per entry
    fwd_bytes = m * (4 + 64) + P * 20 + nb * 4096
    bwd_bytes = nb * (4096 + 256 * 28) + m * (4 + 64) + m * 36 + n * 48
    dom, t_dom, by = ("backward_splat", bwd_ms, bwd_bytes) if bwd_ms >= fwd_ms else ("forward", fwd_ms, fwd_bytes)
    gbs = by / (t_dom * 1e6)
    roof = {"kernel": dom, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": by,
            "avg_launch_ms": round(t_dom, 4),
            "note": "a 256x256 frame with 4096 Gaussians keeps 256 workgroups busy for microseconds: the kernels "
                    "are launch- and latency-bound at this size, far from either roofline"}
    if ceilings:
        roof["achievable"] = ceilings["copy_gbs"]
        roof["frac_of_achievable"] = round(gbs / ceilings["copy_gbs"], 4)
    out = {
        "metric": "toy2d 2D image fit ms/iter (4096 Gaussians, 256x256, L1, Adam)",
        "value": round(wall_ms, 4), "unit": "ms/iter", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded: means U(0,256)^2, log-scales N(ln 2, 0.3), angle U(0, pi), "
                                "opacity sigmoid(N(0,1)), colour U(0,1), target U(0,1))",
        "config": {"workload": "toy2d_fit: 4096 2D Gaussians, 256x256, one fit step (activate, GPU binning, "
                               "forward, L1, bucketed backward, Adam: the activation and radii in one launch "
                               "(activate_fused), torch.optim.Adam's update for the five groups in one "
                               "FusedAdam launch)", "parallelism": "single GPU"},
        "stage_ms": {k2: round(v, 4) for k2, v in stage_ms.items()},
        "kernel_ms": {"forward_with_checkpoints": round(fwd_ms, 4), "backward_splat": round(bwd_ms, 4)},
        "counts": {"pairs": m, "buckets": nb},
        "roofline": roof,
    }
    if ceilings:
        out["achievable"] = ceilings
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline_toy2d(bins.to("cpu"), args.cpu_runs, args.cpu_single_runs)
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"error": repr(e)}
    return out


# The reference's own timings of the toy2d kernels (NVIDIA H100, CUDA events, median of 20 calls
# after 5 warm-ups): forward, forward saving the bucket checkpoints, per-pixel backward, bucketed
# backward, in ms, per (image size, Gaussians); toy2d/results/bench-cfda5b4-4473561.json:11-76.
TOY2D_REF_H100 = {
    (512, 10000): (0.07605, 0.08138, 0.30386, 0.16710),
    (512, 50000): (0.08946, 0.09562, 0.24104, 0.25720),
    (512, 200000): (0.19120, 0.22274, 0.28445, 0.49690),
    (1024, 10000): (0.08664, 0.10072, 1.10880, 0.36314),
    (1024, 50000): (0.12594, 0.14626, 0.86635, 0.49179),
    (1024, 200000): (0.22525, 0.26998, 0.79949, 0.82573),
}


def bench_toy2d_kernels(args) -> dict:
    """The reference's toy2d kernel benchmark (toy2d/bench.py:34-73) on the same scenes:
    Gaussians2D(n, size, size, seed=0), binned with the float32 depth, a N(0,1) upstream gradient;
    each of the extension's calls (forward, forward saving the bucket checkpoints, per-pixel
    backward, bucketed backward) timed alone with HIP events, median of --steps calls after
    --warmup. The pair and bucket counts must equal the reference's."""
    import torch

    from gs2d import Gaussians2D, bin_gaussians
    from gs2d.params import radii_from_cov
    from gs2d.raster import ext

    golden = json.loads((ROOT / "tests" / "golden" / "toy2d_bench_counts.json").read_text())["rows"]
    want = {(r["size"], r["n"]): (r["pairs"], r["buckets"]) for r in golden}

    def timed(fn, warmup, iters):
        for _ in range(warmup):
            fn()
        times = []
        for _ in range(iters):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        return statistics.median(times)

    rows = []
    e = ext()
    for (size, n), ref in TOY2D_REF_H100.items():
        H = W = size
        g = Gaussians2D(n, H, W, seed=0).cuda()
        with torch.no_grad():
            means, conic, color, opacity, cov = (t.contiguous() for t in g.activated())
            bins = bin_gaussians(means, radii_from_cov(cov), g.depth, H, W)
        bg = torch.zeros(3, device="cuda")
        dout = torch.randn(3, H, W, generator=torch.Generator().manual_seed(0)).cuda()
        common = (means, conic, color, opacity, bg, bins.ranges, bins.point_list)

        def fwd(save):
            return e.forward(*common, bins.bucket_offsets, bins.num_buckets, H, W, save)

        out, final_T, n_contrib, _ = fwd(False)
        out_s, final_T_s, n_contrib_s, bstate = fwd(True)
        pairs, buckets = int(bins.point_list.numel()), int(bins.num_buckets)
        if (pairs, buckets) != want[(size, n)]:
            raise RuntimeError(f"toy2d {size}^2 n={n}: {pairs} pairs, {buckets} buckets; the reference binned "
                               f"{want[(size, n)]}")
        r = {"size": size, "n": n, "pairs": pairs, "buckets": buckets,
             "forward_ms": timed(lambda: fwd(False), args.warmup, args.steps),
             "forward_save_buckets_ms": timed(lambda: fwd(True), args.warmup, args.steps),
             "backward_pixel_ms": timed(lambda: e.backward_pixel(*common, final_T, n_contrib, dout), args.warmup,
                                        args.steps),
             "backward_splat_ms": timed(lambda: e.backward_splat(*common, bins.bucket_offsets, bins.bucket_to_tile,
                                                                 out_s, final_T_s, n_contrib_s, bstate, dout),
                                        args.warmup, args.steps)}
        r = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        r["reference_h100_ms"] = dict(zip(("forward", "forward_save_buckets", "backward_pixel", "backward_splat"),
                                          ref))
        rows.append(r)
    value = statistics.mean(r["forward_ms"] + r["backward_splat_ms"] for r in rows)
    ref_value = statistics.mean(v[0] + v[3] for v in TOY2D_REF_H100.values())
    return {
        "metric": "toy2d kernels: forward + bucketed backward ms, mean over the reference's 6 bench scenes",
        "value": round(value, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(value, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (Gaussians2D(n, size, size, seed=0), the reference's bench scenes)",
        "config": {"workload": "toy2d_bench: 512^2 and 1024^2 x 10k, 50k, 200k 2D Gaussians; each extension call "
                               "timed alone (median of HIP-event-timed calls)", "parallelism": "single GPU"},
        "reference_h100_value": round(ref_value, 4),
        "rows": rows,
    }


# The reference's phase0 result on its bench scenes (bench/phase0/backward_bench.py defaults,
# 1920x1080, sigma 2-10 px, opacity 0.05-0.6): the bucketed backward (B) 8.3x faster than the
# per-pixel atomic backward (A) at 50k splats and 9.1x at 200k, on an A100 (phase1/PLAN.md:16;
# its raw logs are not in the tree).
PHASE0_REF_SPEEDUP = {50_000: 8.3, 200_000: 9.1}


def phase0_scene(n: int, h: int, w: int, seed: int = 0, sigma=(2.0, 10.0), opacity=(0.05, 0.6)):
    """The phase0 bench scene (bench/phase0/backward_bench.py:34-49): float64 draws from one seeded
    generator in the reference's order -- means x and y U(-2%, 102%) of the image, the two
    Cholesky diagonals 1 / U(sigma), the off-diagonal U(-0.5, 0.5) times the smaller diagonal,
    opacity U(opacity), colours U(0, 1) -- as (means, chol, opacity logit, colours); index order is
    depth order."""
    import torch

    g = torch.Generator().manual_seed(seed)

    def u(lo, hi, *shape):
        return lo + (hi - lo) * torch.rand(*shape, generator=g, dtype=torch.float64)

    means = torch.stack([u(-0.02 * w, 1.02 * w, n), u(-0.02 * h, 1.02 * h, n)], dim=-1)
    l0 = 1.0 / u(sigma[0], sigma[1], n)
    l2 = 1.0 / u(sigma[0], sigma[1], n)
    l1 = u(-0.5, 0.5, n) * torch.minimum(l0, l2)
    o = u(opacity[0], opacity[1], n)
    colors = u(0.0, 1.0, n, 3)
    return means, torch.stack([l0, l1, l2], dim=-1), torch.log(o / (1.0 - o)), colors


def bench_phase0_kernels(args) -> dict:
    """The reference's phase0 kernel benchmark (bench/phase0/backward_bench.py:81-175) on its
    scenes at 50k and 200k splats: forward, per-pixel backward (A) and bucketed backward (B) of
    the extension, each call timed alone with HIP events (median of --steps calls after --warmup,
    output allocation included, as the reference times them), without the GPU op counters the
    reference's CUDA kernels do not have; plus A-versus-B agreement per parameter group."""
    import torch

    from splat2d import bin_tiles, load_extension

    def timed(fn, warmup, iters):
        for _ in range(warmup):
            fn()
        times = []
        for _ in range(iters):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        return statistics.median(times)

    def rel(a, b):
        return float((a.double() - b.double()).norm() / max(float(b.double().norm()), 1e-12))

    h, w = 1080, 1920
    ext = load_extension(with_cuda=True)
    ext.counting = False
    rows = []
    try:
        for n, ref_speedup in PHASE0_REF_SPEEDUP.items():
            p64 = [t.cuda() for t in phase0_scene(n, h, w)]
            bins = bin_tiles(*p64[:3], h, w)
            tb = (bins.tile_offsets, bins.tile_ids, bins.bucket_offsets, bins.bucket_tile)
            p32 = [t.float().contiguous() for t in p64]
            g_img = torch.randn(h, w, 3, generator=torch.Generator().manual_seed(1)).cuda()
            image, t_final, n_contrib, last_contrib, ckpt = ext.forward(*p32, *tb, h, w)

            def fwd():
                return ext.forward(*p32, *tb, h, w)

            def bwd_a():
                return ext.backward_pixel(g_img, *p32, *tb, t_final, last_contrib, h, w)

            def bwd_b():
                return ext.backward_splat(g_img, *p32, *tb, image, ckpt, h, w)

            ga, gb = bwd_a(), bwd_b()
            counts = (bins.tile_offsets[1:] - bins.tile_offsets[:-1]).double()
            t_f, t_a, t_b = (timed(f, args.warmup, args.steps) for f in (fwd, bwd_a, bwd_b))
            rows.append({"width": w, "height": h, "n": n, "list_entries": int(counts.sum()),
                         "per_tile_mean": round(float(counts.mean()), 1), "per_tile_max": int(counts.max()),
                         "buckets": bins.num_buckets,
                         "contributors_per_pixel": round(float(n_contrib.double().mean()), 1),
                         "forward_ms": round(t_f, 4), "backward_pixel_ms": round(t_a, 4),
                         "backward_splat_ms": round(t_b, 4), "splat_speedup": round(t_a / t_b, 2),
                         "reference_a100_splat_speedup": ref_speedup,
                         "a_vs_b_rel": {k: float(f"{rel(b, a):.2e}") for k, a, b in
                                        zip(("means", "chol", "opacity_logit", "colors"), ga, gb)}})
    finally:
        ext.counting = True
    value = statistics.mean(r["backward_splat_ms"] for r in rows)
    return {
        "metric": "phase0 kernels: bucketed backward ms at 1920x1080, mean over the reference's 50k and 200k scenes",
        "value": round(value, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(value, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (the reference's seeded phase0 bench scene, seed 0)",
        "config": {"workload": "phase0_bench: 1920x1080, 50k and 200k 2D splats (sigma 2-10 px, opacity 0.05-0.6); "
                               "forward, per-pixel backward (A), bucketed backward (B), each call timed alone",
                   "parallelism": "single GPU"},
        "rows": rows,
    }


def bench_l1_ssim(args) -> dict:
    """The fused L1 + D-SSIM loss alone on a 3 x 840 x 1297 frame (the 1M workload's): the forward
    (with the backward's per-pixel map and the partial-sum reduction) and the backward, each
    launched --steps times back to back after --warmup and event-timed. The reference's
    fused-ssim kernels take 0.064 ms (fusedssimCUDA) + 0.093 ms (fusedssim_backwardCUDA) per
    training step on its H100 (results/phase1/README.md:46-47)."""
    import torch

    g = torch.Generator().manual_seed(4321)
    target = torch.rand(3, 840, 1297, generator=g).cuda()
    loss_kernel_times(target, max(args.warmup, 1))  # warm-up
    t = loss_kernel_times(target, args.steps)
    value = t["fwd_ms"] + t["bwd_ms"]
    return {
        "metric": "L1 + D-SSIM loss forward + backward ms on a 3x840x1297 frame",
        "value": round(value, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(value, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded U(0,1) image and target)",
        "config": {"workload": "l1_ssim: 11x11 Gaussian window (sigma 1.5), lambda 0.2, 3x840x1297",
                   "parallelism": "single GPU"},
        "kernels": t, "reference_h100_ms": {"fusedssimCUDA": 0.064, "fusedssim_backwardCUDA": 0.093},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark runs on one GPU; several GPUs are not supported",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.probes:
        print(json.dumps(probes()))
        return
    ceilings = None if args.no_probes else probes()
    if args.workload == "toy2d_fit":
        out = bench_toy2d(args, ceilings)
    elif args.workload == "toy2d_bench":
        out = bench_toy2d_kernels(args)
    elif args.workload == "phase0_bench":
        out = bench_phase0_kernels(args)
    elif args.workload == "l1_ssim":
        out = bench_l1_ssim(args)
    else:
        out = bench_3d(args, ceilings)
    line = json.dumps(out)
    print(line, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(line + "\n")


if __name__ == "__main__":
    main()
