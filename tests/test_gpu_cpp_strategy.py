"""The C++ class surface's densification (include/tinygs_amd/tinygs.hpp:
create_optimizer / create_strategy / DefaultStrategy / GPUGaussian3d::append,
remove / SimpleAdam::remove, duplicate, reset_opacity) end to end: a C++
program runs DefaultStrategy steps with given densification info, and its
parameters, moments, counts and RNG state must be the CPU restatement's
(oracle/strategy.py), bit for bit."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from oracle import strategy as S

pytestmark = pytest.mark.gpu

F = np.float32
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORDER = ("means", "opacities", "rotations", "scales", "sh0", "sh_rest")
WIDTH = {"means": 3, "opacities": 1, "rotations": 4, "scales": 3, "sh0": 3, "sh_rest": 45}


def _binary():
    from tinygs_amd import build as hb
    path = hb.cpp_test_bin("densify_step")
    if not os.path.exists(path):
        hb.build_cpp_test()
    return path


def _info(n, seed):
    g = np.random.default_rng(seed)
    info = np.zeros((n, 4), F)
    info[:, 0] = g.integers(0, 5, n)
    info[:, 1] = (g.random(n) * 8e-4).astype(F)
    info[:, 2] = (g.random(n) * 1.6e-3).astype(F)
    info[:, 3] = (g.random(n) * 900.0).astype(F)
    return info


@pytest.mark.parametrize("sh_half", [0, 1])
def test_cpp_default_strategy_matches_oracle(hip, tmp_path, sh_half):
    n = 5000
    g = np.random.default_rng(31)
    p = {"means": g.normal(0, 1, (n, 3)).astype(F), "scales": g.normal(-4.3, 1.0, (n, 3)).astype(F),
         "rotations": (g.standard_normal((n, 4)) * 1.2).astype(F), "opacities": g.normal(0, 2.5, n).astype(F),
         "sh0": g.random((n, 3)).astype(F), "sh_rest": g.normal(0, 0.1, (n, 45)).astype(F)}
    if sh_half:
        p["sh0"] = p["sh0"].astype(np.float16).astype(F)
        p["sh_rest"] = p["sh_rest"].astype(np.float16).astype(F)
    m1 = {k: g.normal(0, 1, (n, WIDTH[k]) if WIDTH[k] > 1 else n).astype(F) for k in ORDER}
    m2 = {k: g.random((n, WIDTH[k]) if WIDTH[k] > 1 else n).astype(F) for k in ORDER}
    cfg = {"refine_every": 2, "start_refine": 2, "end_refine": 5, "reset_every": 4, "seed": 91,
           "duplicate_grad_threshold": 3e-4, "duplicate_scale_threshold": 0.012, "pruning_scale_threshold": 0.3,
           "max_screen_size": 0.5}
    steps, scale, W, H = 6, 1.5, 320, 240
    # the oracle first: it fixes the row count (and so the info size) of every step
    ref = S.DefaultStrategy(cfg)
    q = {k: v.copy() for k, v in p.items()}
    r1 = {k: v.copy() for k, v in m1.items()}
    r2 = {k: v.copy() for k, v in m2.items()}
    infos, counts = [], []
    for st in range(steps):
        info = _info(q["means"].shape[0], 200 + st)
        infos.append(info)
        ref.counts = {}
        ref.step(q, r1, r2, info, 1.0, scale, W, H)
        counts.append(dict(ref.counts))
    fin = tmp_path / "in.bin"
    with open(fin, "wb") as f:
        f.write(np.int64(n).tobytes())
        f.write(np.int32(sh_half).tobytes())
        f.write(np.array([scale, 1.0], F).tobytes())
        f.write(np.array([W, H], np.uint32).tobytes())
        f.write(np.int32(len(cfg)).tobytes())
        for k, v in cfg.items():
            f.write(k.encode().ljust(48, b"\0"))
            f.write(np.float64(v).tobytes())
        f.write(np.int32(steps).tobytes())
        for k in ORDER:
            f.write(np.ascontiguousarray(p[k], F).tobytes())
        for m in (m1, m2):
            for k in ORDER:
                f.write(np.ascontiguousarray(m[k], F).tobytes())
        for info in infos:
            f.write(np.int64(info.shape[0]).tobytes())
            f.write(np.ascontiguousarray(info, F).tobytes())
    fout = tmp_path / "out.bin"
    print(f"[cpp strategy] sh_half={sh_half}", flush=True)
    r = subprocess.run([_binary(), str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    buf = open(fout, "rb").read()
    off = 0

    def take(count, dtype):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a

    nf = int(take(1, np.int64)[0])
    assert nf == q["means"].shape[0] and nf != n
    for k in ORDER:
        got = take(WIDTH[k] * nf, F)
        assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(q[k], F).reshape(-1).view(np.uint32)), k
    for m in (r1, r2):
        for k in ORDER:
            got = take(WIDTH[k] * nf, F)
            assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(m[k], F).reshape(-1).view(np.uint32)), k
    c = take(3 * steps, np.int64).reshape(steps, 3)
    for st in range(steps):
        want = counts[st]
        if "duplicate" in want:
            assert (c[st, 0], c[st, 1]) == (want["duplicate"], want["split"]), st
        if "kept" in want:
            assert c[st, 2] == want["kept"], st
    rng = take(2, np.uint64)
    assert (int(rng[0]), int(rng[1])) == (ref.rng.state, ref.rng.inc)
