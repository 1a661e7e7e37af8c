"""Headline benchmark: ms per training iteration (fwd + L1/SSIM + bwd + Adam)
of the FastGS path at 1M Gaussians, 1920x1080, SH degree 3 with fp16 SH
storage, on one MI355X, plus the HBM roofline of the
dominant kernel and the CPU oracle's time on the same workload.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--image-dtype float32|float16]
                  [--no-cpu-baseline]
  python bench.py --config 4 [--stress-counts N ...]   (fwd+bwd stress sweep, its own JSON line)
  python bench.py --config 5 [--train-iters K]          (the training loop, its own JSON line)

Prints one JSON line on stdout; a per-stage table goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ms per fwd+bwd+Adam iter at 1M Gaussians 1080p; % of HBM roofline"
HBM_PEAK_GBS = 8000.0

STAGES = ["preprocess", "depth_sort", "emit_instances", "tile_sort", "blend_forward", "l1", "fused_ssim",
          "blend_backward", "preprocess_backward", "adam"]
# stages that are one kernel launch, and that kernel's symbol in rocprofv3
# output, per image dtype (fp16 images: the FGS16 blend kernels)
SINGLE_KERNEL = {"preprocess": "tgs::preprocess_kernel", "blend_forward": "tgs::blend_forward_kernel",
                 "l1": "tgs::l1_kernel", "blend_backward": "tgs::blend_backward_kernel",
                 "adam": "tgs::adam_kernel"}
SINGLE_KERNEL16 = dict(SINGLE_KERNEL, preprocess="tgs::preprocess16_kernel",
                       blend_forward="tgs::blend16_forward_kernel", blend_backward="tgs::blend16_backward_kernel")
# committed counter summaries of this workload ({} = config, then "_fp16" for fp16 images)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_config{}{}.md")
COUNTERS_FILE = os.path.join(ROOT, "profiles", "counters_config{}{}.md")
# VALU issue peak: one wave64 VALU instruction per CU per clock (4 SIMDs, 4
# cycles each), 256 CUs at the 2.4 GHz peak engine clock: 614.4 G wave
# instructions/s. The engine clock under load sits below its peak, by an
# amount that depends on the load, so two figures go beside it: the counter
# run's VALU-busy share (SQ_ACTIVE_INST_VALU over the GPU's own busy cycles)
# and the shader clock the library's probe measures under its own VALU load
# (tgs_selftest_clock).
VALU_PEAK_GINST_S = 256 * 2.4


def measured_clock_mhz():
    """The shader clock under a VALU load (MHz), from the library's probe, or None."""
    import ctypes as C
    from tinygs_amd import _lib
    mhz = C.c_double(0.0)
    if _lib.load().tgs_selftest_clock(C.byref(mhz), None) != 0:
        return None
    return mhz.value


def _suffix(image_dtype):
    return "_fp16" if image_dtype == "float16" else ""


def measured_valu(config, kernel, image_dtype="float32"):
    """(wave-level VALU instructions per launch (SQ_INSTS_VALU), VALU busy %)
    of `kernel` from the committed counter summary of this workload, or
    (None, None)."""
    path = COUNTERS_FILE.format(config, _suffix(image_dtype))
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        m = re.match(r"\|\s*`([^`]+)`\s*\|\s*([0-9.e+]+)\s*\|", line)
        if m and (m.group(1) == kernel or m.group(1).startswith(kernel + "<")):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            busy = float(cells[5].rstrip("%")) if len(cells) > 5 and cells[5].endswith("%") else None
            return float(m.group(2)), busy
    return None, None


def measured_traffic(config, kernel, image_dtype="float32"):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE /
    WRITE_SIZE summary of this workload (two rocprofv3 --pmc runs of this
    script, scaled by a copy of known size), or None if there is none."""
    path = TRAFFIC_FILE.format(config, _suffix(image_dtype))
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\|\s*`([^`]+)`\s*\|\s*\d+\s*\|[^|]*\|[^|]*\|\s*(\d+)\s*\|", line)
        if m and (m.group(1) == kernel or m.group(1).startswith(kernel + "<")):
            return int(m.group(2))
    return None


def algorithmic_bytes(stage, c):
    """Compulsory HBM bytes of one launch (each input read once, each output
    written once; implementation scratch excluded). With the sparse gradient
    handoff (TrainStep's default) only the L rows that receive a gradient are
    read / written by the preprocess backward and read by Adam; the dense
    formulas are the sparse ones with L = N."""
    N, V, I, T, P = c["N"], c["V"], c["I"], c["T"], c["P"]
    L = c["L"]
    s, K, e = c["sh_bytes"], c["sh_bases"], c["image_bytes"]
    if stage == "preprocess":
        return 44 * N + 3 * K * s * V + 4 * N + 52 * V
    if stage == "blend_forward":
        return 8 * T + 40 * c["I_f"] + P * (3 * e + 4)
    if stage == "blend_backward":
        return 8 * T + P * (6 * e + 4) + 40 * c["I_b"] + 44 * c["I_b"]
    if stage == "preprocess_backward":
        # per Gaussian: n_touched, row mask; per gradient row: means, scales, rotations, conic+opacity,
        # SH rest (45 scalars), the 2D gradient sums (11 floats) read, 59 fp32 gradients written
        return 5 * N + L * (12 + 12 + 16 + 16 + 45 * s + 44 + 236)
    if stage == "adam":
        # theta (11 fp32 + 48 SH scalars) and m, v (59 fp32 each) read and written; gradient rows read;
        # the row mask read
        theta = 11 * 4 + 48 * s
        return N * (2 * theta + 4 * 59 * 4 + 1) + 236 * L
    if stage == "l1":
        return 4 * 3 * P * e          # read pred, target; read-modify-write grad, loss
    if stage == "fused_ssim":
        # fused L1 + SSIM in assign mode: read pred, target; write loss, grad
        return 4 * 3 * P * e
    if stage == "depth_sort":
        return 8 * V + 8 * V + 8 * V   # read keys/values once, write one permutation
    if stage == "emit_instances":
        # per visible primitive: index and offset read, 16-byte emission record read, first slot written
        # (the 32-byte record only for primitives past 32 rect tiles: not counted); per instance: the
        # (tile, primitive) pair written
        return 28 * V + 8 * I
    if stage == "tile_sort":
        return 24 * I + 8 * I + 8 * T
    return 0


def host_threads():
    """Cores this process may run on (the GPU box's share), at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(scene_fn, config, all_core_iters=3):
    """The CPU oracle's full iteration on the same seeded scene: the median of
    `all_core_iters` iterations on all the host cores this process may use
    (the reported baseline; its results are identical for any thread count),
    and one iteration on one thread beside it."""
    from oracle import oracle as O
    scene = scene_fn()
    lr = {"means": 1.6e-4, "scene_scale": 1.0, "opacities": 5e-2, "rotations": 1e-3, "scales": 5e-3, "shs": 5e-3}
    O.lib()
    threads = host_threads()

    def one():
        t0 = time.perf_counter()
        O.run_iteration(scene, 0.8, 0.2, lr=lr, eps=1e-15)
        return (time.perf_counter() - t0) * 1e3

    O.set_threads(threads)
    all_ms = sorted(one() for _ in range(all_core_iters))
    O.set_threads(1)
    one_ms = one()
    O.set_threads(threads)
    med = all_ms[len(all_ms) // 2]
    return {"value": round(med, 1), "unit": "ms/iter", "cores": threads, "kind": "port",
            "one_thread_ms": round(one_ms, 1), "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"full config{config} iterations (preprocess, bin, blend fwd, L1+SSIM, blend bwd, preprocess "
                      f"bwd, SimpleAdam) of the C oracle on the same seeded scene: median of {all_core_iters} on "
                      f"{threads} OpenMP threads (value), one on 1 thread (one_thread_ms)"}


def calibrate_copy(mib):
    """Copies `mib` MiB device to device five times. Under `rocprofv3 --pmc
    FETCH_SIZE` (or WRITE_SIZE) each dispatch should read (write) exactly
    mib MiB; the ratio of the counter to that is the scale applied to the
    same counter of the path's kernels."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n * 4, "copies": 5}), flush=True)


STRESS_METRIC = "ms per fwd+bwd vs Gaussians per tile (config 4 stress, 3840x2160, fp32)"


def tile_histogram(rasterizer):
    """Instances per tile of the last forward (from the tile ranges only)."""
    import ctypes as C

    import numpy as np
    import torch

    from tinygs_amd import _lib
    dv = _lib.tgs_debug_view()
    _lib.check(_lib.load().tgs_rasterizer_debug_view(rasterizer._h, C.byref(dv)), "debug_view")
    t = torch.empty(2 * int(dv.n_tiles), dtype=torch.int32, device="cuda")
    _lib.copy_device(dv.tile_ranges, t.numel() * 4, t)
    r = t.cpu().numpy().view(np.uint32).reshape(-1, 2).astype(np.int64)
    return r[:, 1] - r[:, 0]


def stress_main(args):
    """Config 4: forward + backward (no loss, no optimiser) of the high-overlap
    scene at several Gaussian counts; per count the distribution of Gaussians
    per tile and the ms per fwd+bwd. The JSON value is the full 3M case."""
    import numpy as np
    import torch

    from tinygs_amd import scenes
    from tinygs_amd.core import GPUBatchInput, GPUGaussian3d, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer

    rows = []
    for n in args.stress_counts:
        t0 = time.time()
        scene = scenes.config4(n=n)
        g = GPUGaussian3d.from_scene(scene)
        grads = g.gradient_like()
        r = create_rasterizer("fastgs")
        r.set_gaussians(g)
        ctx = RasterizeContext()
        ctx.fwd_input = GPUBatchInput.from_camera(scene.camera)
        ctx.fwd_output.image = Image.empty(scene.camera.shape)
        ctx.gaussians_grad = grads
        gimg = scenes.grad_image(44, scene.camera.shape)
        ctx.grad_output.image = Image(scene.camera.shape, "float32", torch.from_numpy(gimg).cuda())
        print(f"[bench] config4 n={n}: scene in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

        def step():
            r.forward(ctx)
            r.backward(ctx, assign=True)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        fwd_ms = 0.0
        stream = torch.cuda.current_stream()
        a.record(stream)
        for _ in range(args.steps):
            step()
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / args.steps
        a.record(stream)
        for _ in range(args.steps):
            r.forward(ctx)
        b.record(stream)
        torch.cuda.synchronize()
        fwd_ms = a.elapsed_time(b) / args.steps
        per_tile = tile_histogram(r)
        V, I, T = r.counts()
        img = ctx.fwd_output.image.data
        ok = bool(torch.isfinite(img).all().item()) and all(
            bool(torch.isfinite(t).all().item()) for t in grads.tensors())
        row = {"n_gaussians": n, "n_instances": I, "n_tiles": T, "ms_fwd_bwd": round(ms, 3),
               "ms_fwd": round(fwd_ms, 3),
               "per_tile": {"median": int(np.median(per_tile)), "p90": int(np.percentile(per_tile, 90)),
                            "max": int(per_tile.max()), "mean": round(float(per_tile.mean()), 1),
                            "covered_tiles": int((per_tile > 0).sum()),
                            "median_covered": int(np.median(per_tile[per_tile > 0])) if (per_tile > 0).any() else 0},
               "finite": ok}
        rows.append(row)
        print(f"[bench] config4 n={n}: {ms:.3f} ms fwd+bwd ({fwd_ms:.3f} fwd), I={I}, Gaussians per tile "
              f"median {row['per_tile']['median']} (covered tiles {row['per_tile']['covered_tiles']}: median "
              f"{row['per_tile']['median_covered']}) p90 {row['per_tile']['p90']} max {row['per_tile']['max']}",
              file=sys.stderr, flush=True)
        del r, g, grads, ctx
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    last = rows[-1]
    out = {"metric": STRESS_METRIC, "value": last["ms_fwd_bwd"], "unit": "ms/iter", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": last["ms_fwd_bwd"], "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "config4: fwd + bwd (assign), seeded dL/dimage", "width": 3840, "height": 2160,
                      "sh_degree": 3, "parallelism": "single GPU"},
           "sweep": rows}
    print(json.dumps(out), flush=True)


TRAIN_METRIC = "iters/s of the config-5 training loop (fwd+bwd+L1/SSIM+Adam, densification every 100 iters)"


def train_main(args):
    """Config 5: the training loop (Orchestrator with SimpleAdam and
    DefaultStrategy) on a synthetic 200-view dataset. Reports iterations per
    second over the whole loop (densification steps included, targets
    resident in HBM), the Gaussian count, and the mean PSNR over all views at
    iteration 100 and at the end."""
    import torch

    from tinygs_amd import scenes
    from tinygs_amd.data import SimpleDataLoader, SyntheticViewDataset, gaussians_from_arrays
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.rasterizer import create_rasterizer
    from tinygs_amd.strategy import create_strategy
    from tinygs_amd.trainer import Orchestrator, OrchestratorConfig

    t0 = time.time()
    scene = scenes.config5(n_init=args.train_init, n_gt=args.train_gt, n_cameras=args.train_views)
    ds = SyntheticViewDataset(scene)
    g = gaussians_from_arrays(scene.init, 0)   # SH degree 0 at the start, as the loop's schedule has it
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    strat = create_strategy("default", g, grads, opt)
    strat.set_params({"refine_every": 100, "start_refine": 100, "end_refine": args.train_iters,
                      "duplicate_grad_threshold": 2e-4, "pruning_opacity_threshold": 0.005})
    orch = Orchestrator(OrchestratorConfig(), g, grads, create_rasterizer("fastgs"), opt, SimpleDataLoader(ds),
                        strategy=strat)
    orch.initialize()   # Morton reordering before step 0 (reorder_gaussians_interval > 0), as the loop does
    torch.cuda.synchronize()
    print(f"[bench] config5: {args.train_init} initial Gaussians, {args.train_gt} ground truth, "
          f"{args.train_views} views {scene.width}x{scene.height} (set up in {time.time() - t0:.1f}s)",
          file=sys.stderr, flush=True)
    psnr0 = orch.eval_psnr()
    orch.recompute_scene_scale()
    first = min(100, args.train_iters)
    t0 = time.time()
    for _ in range(first):
        orch.train_step()
    torch.cuda.synchronize()
    t_first = time.time() - t0
    psnr100 = orch.eval_psnr()
    n100 = g.size()
    t1 = time.time()
    for _ in range(args.train_iters - first):
        orch.train_step()
        if orch.m_state.current_step % 100 == 0:
            print(f"[bench] iter {orch.m_state.current_step}: {g.size()} Gaussians", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    elapsed = t_first + (time.time() - t1)
    psnr_end = orch.eval_psnr()
    ips = args.train_iters / elapsed
    print(f"[bench] {args.train_iters} iterations in {elapsed:.2f}s = {ips:.1f} it/s; PSNR {psnr0:.3f} -> "
          f"{psnr100:.3f} (iter 100) -> {psnr_end:.3f} dB; {g.size()} Gaussians", file=sys.stderr, flush=True)
    out = {"metric": TRAIN_METRIC, "value": round(ips, 2), "unit": "iters/s", "n_gpus": 1,
           "steps": args.train_iters, "warmup": 0, "ms_per_step": round(1e3 / ips, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "config5: Orchestrator loop (Morton reorder at initialize), SimpleAdam, "
                                  "DefaultStrategy (refine every 100)",
                      "initial_gaussians": args.train_init, "ground_truth_gaussians": args.train_gt,
                      "views": args.train_views, "width": scene.width, "height": scene.height,
                      "parallelism": "single GPU"},
           "psnr_db": {"start": round(psnr0, 3), "iter100": round(psnr100, 3), "final": round(psnr_end, 3)},
           "gaussians": {"start": args.train_init, "iter100": n100, "final": g.size()}}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3,
                    help="3: the headline training iteration; 1, 2: the smaller scenes; 4: the fwd+bwd stress sweep; "
                         "5: the training loop")
    ap.add_argument("--stress-counts", type=int, nargs="+", default=[375_000, 750_000, 1_500_000, 3_000_000],
                    help="Gaussian counts of the config-4 sweep")
    ap.add_argument("--train-iters", type=int, default=1000, help="config 5: training iterations")
    ap.add_argument("--train-init", type=int, default=500_000, help="config 5: initial Gaussians")
    ap.add_argument("--train-gt", type=int, default=400_000, help="config 5: ground-truth Gaussians")
    ap.add_argument("--train-views", type=int, default=200, help="config 5: views")
    ap.add_argument("--image-dtype", choices=["float32", "float16"], default="float32",
                    help="config 1-3: image data type; float16 runs the fp16-image rasterizer (FGS16) and the fp16 "
                         "losses, the reference's train_data_type float16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run 5 device-to-device copies of MIB MiB (the known-size kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters of a --pmc run)")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)

    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); this build measures one GPU's "
              "share of the path, and sharding across GPUs is not implemented", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from tinygs_amd import _lib, scenes
    from tinygs_amd.train import TrainStep

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    if args.config == 4:
        return stress_main(args)
    if args.config == 5:
        return train_main(args)
    scene_fn = {1: scenes.config1, 2: scenes.config2, 3: scenes.config3}[args.config]
    t0 = time.time()
    scene = scene_fn()
    print(f"[bench] scene config{args.config}: N={scene.n} {scene.camera.width}x{scene.camera.height} "
          f"sh_degree={scene.sh_degree} sh_storage={scene.sh_dtype} (generated in {time.time() - t0:.1f}s)",
          file=sys.stderr, flush=True)
    f16 = args.image_dtype == "float16"
    # the no-sync step (no host waits inside the step; the first warmup step
    # sizes the buffers and reserves 1.25x its instance count), checked for a
    # capacity overflow after the timed steps: the same kernels and results
    # as the waiting step (tests/test_gpu_forward_modes.py)
    ts = TrainStep(scene, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, image_dtype=args.image_dtype,
                   no_sync=True)
    L = _lib.load()
    stream = torch.cuda.current_stream()

    for _ in range(args.warmup):
        ts.step()
    torch.cuda.synchronize()

    import ctypes as C

    # the timed region: K uninstrumented steps
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        ts.step()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    ts.check_status()   # raises if a timed step outgrew the reserved instance capacity

    # per-stage breakdown: K more steps with one event pair per stage per step
    # (the events add gaps of their own, so these steps are not the timed ones)
    L.tgs_profiling_set((1 << len(STAGES)) - 1)
    for k in range(len(STAGES)):
        L.tgs_profiling_read(k, None, None, 1)
    for _ in range(args.steps):
        ts.step()
    torch.cuda.synchronize()
    L.tgs_profiling_set(0)
    stage_ms = {}
    for k, name in enumerate(STAGES):
        tot, cnt = C.c_double(), C.c_int64()
        _lib.check(L.tgs_profiling_read(k, C.byref(tot), C.byref(cnt), 1))
        stage_ms[name] = (tot.value / cnt.value) if cnt.value else 0.0
    fl, bp = C.c_int64(), C.c_int64()
    _lib.check(L.tgs_rasterizer_work_stats(ts.rasterizer._h, C.byref(fl), C.byref(bp), 1))
    V, I, T = ts.rasterizer.counts()
    cam = scene.camera
    if ts.sparse_grads:
        mask = torch.empty(scene.n, dtype=torch.uint8, device="cuda")
        _lib.copy_device(ts.rasterizer.grad_row_mask(), scene.n, mask)
        live = int(mask.sum().item())
    else:
        live = scene.n
    counts = {"N": scene.n, "V": V, "I": I, "T": T, "P": cam.width * cam.height, "L": live,
              "I_f": fl.value, "I_b": bp.value,
              "sh_bytes": 2 if scene.sh_dtype == "float16" else 4, "sh_bases": (scene.sh_degree + 1) ** 2,
              "image_bytes": 2 if f16 else 4}
    single = SINGLE_KERNEL16 if f16 else SINGLE_KERNEL

    print(f"[bench] {ms:.3f} ms/iter over {args.steps} steps; V={V} I={I} T={T} "
          f"I_f={counts['I_f']:.0f} I_b={counts['I_b']:.0f} gradient rows L={live}", file=sys.stderr)
    print(f"[bench] {'stage':22s} {'ms':>8s} {'GB/s':>8s} {'%HBM':>6s}", file=sys.stderr)
    rows = []
    for name in STAGES:
        t = stage_ms[name]
        b = algorithmic_bytes(name, counts)
        gbs = b / (t * 1e-3) / 1e9 if t > 0 else 0.0
        rows.append((name, t, b, gbs))
        print(f"[bench] {name:22s} {t:8.4f} {gbs:8.1f} {100 * gbs / HBM_PEAK_GBS:6.1f}", file=sys.stderr)
    print(f"[bench] sum of stages {sum(r[1] for r in rows):.3f} ms", file=sys.stderr, flush=True)

    dom = max((r for r in rows if r[0] in single), key=lambda r: r[1])
    roofline = {"bound": "hbm", "kernel": dom[0], "achieved": round(dom[3], 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dom[3] / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(args.config, single[dom[0]], args.image_dtype),
                "algorithmic_bytes": int(dom[2]), "avg_launch_ms": round(dom[1], 5)}

    # VALU roofline of the VALU-bound blend kernels: wave instructions per
    # launch (counter summary) over the live launch time, and the counter
    # run's own VALU-busy figure beside it
    valu = {}
    clk = measured_clock_mhz()
    if clk:
        print(f"[bench] shader clock under the probe's VALU load {clk:.0f} MHz (a kernel's own clock depends on its "
              "load)", file=sys.stderr)
    for name in ("blend_forward", "blend_backward"):
        insts, busy = measured_valu(args.config, single[name], args.image_dtype)
        t = stage_ms[name]
        if insts is None or t <= 0:
            valu[name] = None
            continue
        ach = insts / (t * 1e-3) / 1e9
        valu[name] = {"bound": "valu", "achieved": round(ach, 1), "peak": VALU_PEAK_GINST_S,
                      "unit": "G wave-instructions/s", "frac": round(ach / VALU_PEAK_GINST_S, 4),
                      "insts_per_launch": insts, "avg_launch_ms": round(t, 5),
                      "counter_valu_busy_pct": busy, "probe_clock_mhz": round(clk, 1) if clk else None}
        print(f"[bench] {name}: {ach:.0f} G VALU wave-instructions/s = {100 * ach / VALU_PEAK_GINST_S:.1f}% of the "
              f"issue peak at 2.4 GHz; counter run VALU busy {busy}%", file=sys.stderr)

    cpu = None
    if not args.no_cpu_baseline and not f16:
        print(f"[bench] cpu baseline: full iterations of the CPU oracle on the same scene ({host_threads()} "
              "threads, then 1)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(scene_fn, args.config)
        print(f"[bench] cpu baseline {cpu['value']:.0f} ms/iter on {cpu['cores']} threads "
              f"({cpu['value'] / ms:.0f}x the GPU), {cpu['one_thread_ms']:.0f} ms on 1 thread; "
              f"{cpu['cpu_model']}, nproc {cpu['nproc']}", file=sys.stderr)

    out = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms/iter", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 images (half blending and losses), f32 geometry and Adam" if f16 else "f32",
        "data": "synthetic",
        "config": {"workload": f"config{args.config}: fwd + 0.8 L1 + 0.2 (1-SSIM) + bwd + SimpleAdam"
                               + (", float16 images (FGS16)" if f16 else ""),
                   "n_gaussians": scene.n, "width": cam.width, "height": cam.height, "sh_degree": scene.sh_degree,
                   "sh_storage": scene.sh_dtype, "image_dtype": args.image_dtype, "n_visible": V,
                   "n_instances": I, "n_tiles": T,
                   "gradient_rows": live, "sparse_gradients": ts.sparse_grads,
                   "step_mode": "no-sync (reserved instance capacity, no host wait inside a step)",
                   "parallelism": "single GPU"},
        "stages_ms": {r[0]: round(r[1], 5) for r in rows},
        "roofline": roofline,
        "valu_roofline": valu,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
