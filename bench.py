"""Benchmark: 3D Gaussian-splat rasterizer fwd+bwd ms/iter on one MI355X.

Workload (default): 1M Gaussians, SH degree 3, 1297x840, fx=fy=1160, 8 seeded orbit poses
(radius U(3,5)); one step = forward + backward of one view (poses cycled) with a seeded
N(0,1) upstream image gradient. Inputs are resident in HBM before the timed region.

    python bench.py [--steps K] [--warmup W] [--workload sh3_1m|sh3_3m|sh_rgb_100k] [--no-cpu-baseline]
                    [--no-train-step] [--no-variants]
    python bench.py --copy-probe      # a plain 1 GiB device copy, to calibrate HBM counters

Prints ONE JSON line. `value` is the wall time of K plain steps; per-stage times come from
HIP events recorded on the launch stream in a second pass over the same K steps; `roofline` is for the kernel with the largest share of the step
(the bucketed blend backward), from its algorithmic bytes and its event-timed duration, plus
its VALU issue rate from the committed SQ counter summary. `train_step` (secondary) times the
full training step on the same scene: forward, L1 + D-SSIM loss, backward and fused Adam
(dense and visibility-masked), with the optimizer's HBM rate; `variants` the inference forward,
the pruning-score blend and fwd+bwd under proper antialiasing, per view.
"""
from __future__ import annotations

import argparse
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
# wave64 FP32 VALU instructions per second: the published 157.3 TFLOP/s FP32 vector peak, an FMA
# counting 2 FLOP on each of 64 lanes
VALU_PEAK_INSTR = 157.3e12 / 2 / 64
METRIC = "fwd+bwd ms/iter @1M Gaussians SH3 1297x840; per-stage HBM GB/s vs roofline"
# stages that are one kernel each (the others group several kernels)
SINGLE_KERNEL = {"preprocess": "preprocess_fwd_kernel", "blend_fwd": "blend_fwd_strip_kernel",
                 "blend_bwd": "blend_bwd_bucket_kernel", "preprocess_bwd": "preprocess_bwd_kernel"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="sh3_1m", choices=["sh3_1m", "sh3_3m", "sh_rgb_100k"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0, help="threads for the CPU baseline (0 = OMP default)")
    ap.add_argument("--copy-probe", action="store_true", help="time a plain 1 GiB device copy and exit")
    ap.add_argument("--no-train-step", action="store_true", help="skip the training-step measurement")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the inference / pruning-score / antialiasing variants (profiling runs)")
    ap.add_argument("--json-out", default=None)
    return ap.parse_args()


def stage_bytes(fs, n_visible, active_buckets, splat_steps, used_pairs, staged, ckpt_written,
                atomics_per_pair=9):
    """Algorithmic (compulsory) HBM bytes per stage for the measured counts: each datum read or
    written once (fp32)."""
    n, m, K = fs.n, fs.m, fs.sh_coeffs
    T = fs.cam.n_tiles
    P = fs.cam.width * fs.cam.height
    B = int(fs.bucket_offsets[-1].item())
    return {
        # params 44 B/Gaussian + tiles_touched and depth key 8 B; SH 12 K B and the 64 B record
        # per visible one
        "preprocess": 44 * n + 8 * n + n_visible * (12 * K + 64),
        # 3 radix passes over N (histogram read 4 B, key+value read and write 16 B), the counts
        # gathered into depth order (read + write), the scan (counts read, offsets written)
        "depth_order": 3 * 20 * n + 8 * n + 8 * n,
        # emission (48 B of the record of the visible, order and offset per Gaussian, key+value
        # per instance), tile sort pass 1 (histogram 4, key+value read and write 16) and pass 2
        # (histogram 4, key+value read 8, value write 4), ranges and bucket offsets per tile
        "binning": 48 * n_visible + 8 * n + 8 * m + 20 * m + 16 * m + 20 * T + 4 * B,
        # per staged list entry: id + 64 B record; per pixel: image 12 + final T 4 + n_contrib 4;
        # the checkpoints written (4 KiB per bucket reached); tile max, bucket_to_tile, and the
        # backward's screen-space gradient buffer the forward zeroes (48 B per Gaussian)
        "blend_fwd": staged * (4 + 64) + P * 20 + ckpt_written * 4096 + 4 * T + 4 * B + 48 * n,
        # per active bucket: checkpoints 4 KiB + grad image 12, image 12, n_contrib 4 per pixel;
        # per bucket-splat step: id + record; per reduced bucket-splat: 9 fp32 atomics (11 with
        # the |dL/dmean2d| sums)
        "blend_bwd": active_buckets * (4096 + 256 * 28) + splat_steps * (4 + 64) + used_pairs * 4 * atomics_per_pair,
        # params, SH, record and grad2d of the visible; every output row written
        "preprocess_bwd": n_visible * (44 + 12 * K + 64 + 48) + n * (44 + 12 * K),
    }


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


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, calibrated with a plain copy), or None."""
    f = ROOT / "profiles" / f"{kernel}_hbm_traffic.md"
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def measured_valu_instr(kernel: str):
    """VALU instructions per launch of `kernel` from the committed rocprofv3 SQ summary, or None."""
    f = ROOT / "profiles" / f"{kernel}_sq.md"
    if not f.exists():
        return None
    m = re.search(r"valu_instr_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(scene, pose, threads):
    """The C oracle (the CPU restatement of the same rules, OpenMP where the loops allow) timed
    on the host: one full fwd+bwd of one view of the workload (~10 s)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    if threads > 0:
        os.environ["OMP_NUM_THREADS"] = str(threads)
    import oracle as O

    cam = scene.cameras[pose]
    p = [t.numpy() for t in scene.params()]
    gi = np.random.default_rng(0).standard_normal((3, cam.height, cam.width)).astype(np.float32)
    t0 = time.perf_counter()
    r = O.render(*p, cam, 3)
    g2 = O.blend_bwd(r["rec"], r["point_list"], r["ranges"], r["bucket_offsets"], cam.width, cam.height,
                     r["image"], gi, r["final_T"], r["n_contrib"], r["tile_max"], r["ckpt"], scene.n)
    O.preprocess_bwd(*p, cam, 3, r["rec"], r["touched"], g2)
    dt = time.perf_counter() - t0
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    return {"value": round(dt * 1000.0, 1), "unit": "ms/iter", "cores": cores, "kind": "port",
            "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"C oracle fwd+bwd of pose {pose}, all {scene.n} Gaussians ({dt:.1f} s; preprocess and "
                      f"forward blend on {cores} OpenMP threads, sort and backward blend single-threaded)"}


# learning rates of the training-step workload (means, log-scales, quats, SH DC, SH rest, opacity)
TRAIN_LR = {"means": 1.6e-4, "scales": 5e-3, "quats": 1e-3, "sh_dc": 2.5e-3, "sh_rest": 1.25e-4, "opacity": 5e-2}


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
    Ks = [torch.tensor([[c.fx, 0.0, c.cx], [0.0, c.fy, c.cy], [0.0, 0.0, 1.0]]) for c in cams]
    n = m.shape[0]
    out = {"workload": f"{n} Gaussians SH3 {cams[0].width}x{cams[0].height}: fwd, L1+D-SSIM (11x11, lambda 0.2), "
                       f"bwd, fused Adam over 59 fp32 parameters per Gaussian",
           "lr": TRAIN_LR}
    for mode in ("dense", "masked"):
        params = {k: torch.nn.Parameter(v.clone()) for k, v in P.items()}
        groups = [{"params": [params[k]], "lr": lr, "name": k} for k, lr in TRAIN_LR.items()]
        opt = FusedAdam(groups, lr=0.0, eps=1e-15, sparse=(mode == "masked"))
        vis_sum = 0

        def step(k, ev=None):
            c = cams[k % len(cams)]
            img, _, aux = rasterize(params["means"], params["scales"], params["quats"], params["opacity"],
                                    (params["sh_dc"], params["sh_rest"]), c.viewmat, Ks[k % len(cams)], c.width,
                                    c.height, near=c.near, far=c.far)
            loss = l1_ssim_loss(img, targets[k % len(cams)], 0.2)
            loss.backward()
            if ev:
                ev[0].record()
            opt.step()
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
        nbytes = 1652 * n if mode == "dense" else int(1652 * vis_sum) + 4 * n
        out[mode] = {"step_ms": round(step_ms, 4), "adam_ms": round(adam_ms, 4),
                     "adam_hbm_gbs": round(nbytes / (adam_ms * 1e6), 1),
                     "adam_hbm_frac": round(nbytes / (adam_ms * 1e6) / HBM_PEAK_GBS, 4),
                     "adam_algorithmic_bytes": nbytes, "visible_per_view": round(vis_sum)}
        from amdsplat.raster3d import _Rasterize3D

        _Rasterize3D.track_visibility = False
    return out


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
    Ks = [torch.tensor([[c.fx, 0.0, c.cx], [0.0, c.fy, c.cy], [0.0, 0.0, 1.0]]) for c in cams]
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


def copy_probe():
    import torch

    n = 1 << 28  # 1 GiB of float32
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    reps = 10
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "ms": round(ms, 4),
                      "GBps_read_plus_write": round(8 * n / (ms * 1e6), 1)}))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark runs on one GPU; several GPUs are not supported",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.copy_probe:
        copy_probe()
        return
    import torch

    from amdsplat import raster3d as R
    from amdsplat import scenes

    make = {"sh3_1m": scenes.sh3_1m, "sh3_3m": scenes.sh3_3m, "sh_rgb_100k": scenes.sh_rgb_100k}[args.workload]
    scene = make()
    sc = scene.to("cuda")
    params = sc.params()
    cams = sc.cameras
    g = torch.Generator().manual_seed(1234)
    grads = [torch.randn(3, c.height, c.width, generator=g).cuda() for c in cams]

    def step(k, timer=None, counters=None):
        pose = k % len(cams)
        fs = R.forward_pass(*params, cams[pose], sh_degree=None, timing=timer if timer else False)
        out = R.backward_pass(fs, *params, grads[pose], timing=timer if timer else False, counters=counters,
                              abs_grad=False)
        return fs, out

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()

    # the timed region: K steps, nothing recorded between the stages
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(k)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / args.steps

    # the per-stage breakdown: the same K steps again with HIP events between the stages (the
    # events cost a few microseconds each, so this pass is not the headline number)
    timers = [R.StageTimer(True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for k in range(args.steps):
        step(k, timers[k])
    torch.cuda.synchronize()
    staged_wall_ms = (time.perf_counter() - t1) * 1000.0 / args.steps

    per_stage = {}
    step_ms = []
    pose_ms = [[] for _ in cams]
    for k, tm in enumerate(timers):
        r = tm.result(sync=False)
        step_ms.append(sum(r.values()))
        pose_ms[k % len(cams)].append(step_ms[-1])
        for k2, v in r.items():
            per_stage.setdefault(k2, []).append(v)
    stage_ms = {k2: statistics.mean(v) for k2, v in per_stage.items() if k2 != "start"}
    # per pose: the median over its event-timed steps; then the median and the max over the poses
    pose_medians = [statistics.median(v) for v in pose_ms if v]

    # counts for the byte model: one counting step per pose outside the timed regions, averaged
    # over the poses like the timings
    per_pose = []
    for pose in range(len(cams)):
        ctr = torch.zeros(3, dtype=torch.int64, device="cuda")
        fs, _ = step(pose, counters=ctr)
        torch.cuda.synchronize()
        nv = int((fs.touched > 0).sum().item())
        ab, ss, stg, ckw = bucket_stats(fs)
        up = int(ctr[0].item()) // 9
        per_pose.append({"visible": nv, "instances": fs.m, "buckets": int(fs.bucket_offsets[-1].item()),
                         "active_buckets": ab, "bucket_splat_steps": ss, "staged_entries": stg,
                         "ckpt_written": ckw, "reduced_bucket_splats": up,
                         "bwd_pair_evals": int(ctr[2].item()),
                         "bytes": stage_bytes(fs, nv, ab, ss, up, stg, ckw)})
    counts = {k2: round(statistics.mean(pp[k2] for pp in per_pose)) for k2 in per_pose[0] if k2 != "bytes"}
    sb = {k2: statistics.mean(pp["bytes"][k2] for pp in per_pose) for k2 in per_pose[0]["bytes"]}
    stage_gbs = {k2: sb[k2] / (stage_ms[k2] * 1e6) for k2 in stage_ms if k2 in sb and stage_ms[k2] > 0}
    dominant = max((k2 for k2 in stage_ms if k2 in SINGLE_KERNEL), key=lambda k2: stage_ms[k2])
    achieved = stage_gbs[dominant]
    traffic = measured_traffic(SINGLE_KERNEL[dominant])
    valu_instr = measured_valu_instr(SINGLE_KERNEL[dominant])
    valu = None
    if valu_instr:
        rate = valu_instr / (stage_ms[dominant] * 1e-3)
        valu = {"achieved": round(rate / 1e12, 4), "peak": round(VALU_PEAK_INSTR / 1e12, 4),
                "unit": "T wave64 instr/s", "frac": round(rate / VALU_PEAK_INSTR, 4), "instr_per_launch": valu_instr}

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
        "config": {"workload": f"{args.workload}: {scene.n} Gaussians SH{fs.sh_degree} "
                               f"{fs.cam.width}x{fs.cam.height}, fwd+bwd per view, 8 orbit poses",
                   "gaussians": scene.n, "width": fs.cam.width, "height": fs.cam.height,
                   "parallelism": "single GPU"},
        "stage_ms": {k2: round(v, 4) for k2, v in stage_ms.items()},
        "stage_hbm_gbs": {k2: round(v, 1) for k2, v in stage_gbs.items()},
        "stage_hbm_frac": {k2: round(v / HBM_PEAK_GBS, 4) for k2, v in stage_gbs.items()},
        "event_sum_ms": round(statistics.mean(step_ms), 4),
        "per_pose_ms": {"median": round(statistics.median(pose_medians), 4), "max": round(max(pose_medians), 4),
                        "poses": [round(v, 4) for v in pose_medians]},
        "staged_pass_ms_per_step": round(staged_wall_ms, 4),
        "counts": counts,
        "roofline": {"kernel": SINGLE_KERNEL[dominant], "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": round(sb[dominant]),
                     "avg_launch_ms": round(stage_ms[dominant], 4), "valu": valu},
    }
    if not args.no_variants:
        out["variants"] = variants_bench(sc, grads, steps=max(args.steps // 2, 5), warmup=3)
    if not args.no_train_step:
        out["train_step"] = train_step_bench(scene, steps=max(args.steps // 2, 5), warmup=3)
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(scene, 0, args.cpu_threads)
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"error": repr(e)}
    line = json.dumps(out)
    print(line, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(line + "\n")


if __name__ == "__main__":
    main()
