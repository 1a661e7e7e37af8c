"""Writes config5_reduced.json: the CPU oracle's training trajectory on a
reduced config-5 scene (oracle/train.py), the fixture that
tests/test_gpu_train.py compares the GPU Orchestrator against.

  python tests/golden/make_config5_reduced.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import train as T  # noqa: E402
from tinygs_amd import scenes  # noqa: E402

SCENE = {"n_init": 3000, "n_gt": 4000, "width": 256, "height": 168, "n_cameras": 16}
STRATEGY = {"refine_every": 10, "start_refine": 10, "end_refine": 40, "reset_every": 30, "seed": 42}
ITERS = 40
CHECKPOINTS = (10, 20, 30, 40)
EVAL_VIEWS = (0, 5, 10, 15)


def main():
    sc = scenes.config5(**SCENE)
    tr = T.Trainer(sc, STRATEGY)
    traj = {"psnr": {}, "gaussians": {}, "counts": {}}
    for it in range(1, ITERS + 1):
        tr.train_step()
        if tr.strategy.counts:
            traj["counts"][str(it)] = dict(tr.strategy.counts)
            tr.strategy.counts = {}
        if it in CHECKPOINTS:
            traj["psnr"][str(it)] = tr.eval_psnr(EVAL_VIEWS)
            traj["gaussians"][str(it)] = int(tr.p["means"].shape[0])
            print(it, traj["psnr"][str(it)], traj["gaussians"][str(it)], flush=True)
    traj["psnr"]["0"] = None
    out = {"scene": SCENE, "strategy": STRATEGY, "iters": ITERS, "eval_views": list(EVAL_VIEWS),
           "scene_scale": tr.scale, "trajectory": traj}
    with open(os.path.join(HERE, "config5_reduced.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
