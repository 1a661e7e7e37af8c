"""Writes config5_iter100.json: the CPU oracle's full-size config-5 training
run (500k initial Gaussians, 400k ground truth, 200 views of 1600x1060) up to
iteration 100 -- the mean PSNR over views 0..19 and the parameter checksums --
which tests/test_gpu_train.py compares the GPU loop against.

Takes about half an hour of one CPU core plus the target renders, which run
in a process pool:

  python tests/golden/make_config5_iter100.py [--workers 6]
"""
import argparse
import json
import os
import sys
import time
from multiprocessing import Pool

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import train as T  # noqa: E402
from tinygs_amd import scenes  # noqa: E402

ITERS = 100
EVAL_VIEWS = tuple(range(20))
STRATEGY = {"refine_every": 100, "start_refine": 100, "end_refine": 1000}


def _render(i):
    sc = scenes.config5()
    return i, T.render_targets(sc.gt, [sc.cameras[i]])[0]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workers", type=int, default=6)
    args = ap.parse_args()
    sc = scenes.config5()
    ld = T.Loader(len(sc.cameras))
    used = sorted(set(ld.next() for _ in range(ITERS)) | set(EVAL_VIEWS))
    t0 = time.time()
    targets = [None] * len(sc.cameras)
    with Pool(args.workers) as pool:
        for i, img in pool.imap_unordered(_render, used):
            targets[i] = img
    print(f"{len(used)} targets in {time.time() - t0:.0f}s", flush=True)
    tr = T.Trainer(sc, STRATEGY, targets=targets)
    t0 = time.time()
    for it in range(ITERS):
        tr.train_step()
        if (it + 1) % 10 == 0:
            print(f"iter {it + 1} ({time.time() - t0:.0f}s)", flush=True)
    psnr = tr.eval_psnr(EVAL_VIEWS)
    print("psnr", psnr, flush=True)
    out = {"iters": ITERS, "eval_views": list(EVAL_VIEWS), "strategy": STRATEGY, "scene_scale": tr.scale,
           "psnr": psnr, "gaussians": int(tr.p["means"].shape[0]),
           "param_means": {k: float(np.asarray(v, np.float64).mean()) for k, v in tr.p.items()},
           "param_abs_means": {k: float(np.abs(np.asarray(v, np.float64)).mean()) for k, v in tr.p.items()}}
    with open(os.path.join(HERE, "config5_iter100.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
