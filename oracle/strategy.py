"""TEST INFRASTRUCTURE — CPU restatement of the densification step.

Only tests/ may import this module; the product (tinygs_amd) never does.

Restates, in float32 numpy with the oracle's deterministic exp / log:
  pcg32 seed / next / advance / next_float   tinygs/include/tinygs/random/pcg32.hpp:35-160
  generate_random_logistic                    tinygs/include/tinygs/random/device.cuh:38-84
  logit / logistic                            tinygs/include/tinygs/common.hpp:358-364
  DefaultStrategy::duplicate (select, apply)  tinygs/src/strategy/default.cu:71-297
  DefaultStrategy::prune (alive flags)        default.cu:300-341
  reset_opacity                               default.cu:26-37
  DefaultStrategy::step_impl                  default.cu:40-69
  GPUGaussian3d::append / remove              tinygs/src/core/gpu_gaussian.cu:117-170
  SimpleAdam::remove / duplicate /
  reset_opacity                               tinygs/src/optim/simple_adam.cu:841-985
  StrategyBase::on_remove / on_duplicate      tinygs/src/strategy/strategy.cpp:19-63

Every float32 expression follows the kernel's operation order; NaN-aware
min / max are np.fmin / np.fmax (C fminf / fmaxf).
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

M64 = (1 << 64) - 1
PCG_MULT = 0x5851F42D4C957F2D
PCG32_DEFAULT_STATE = 0x853C49E6748FEA9B
PCG32_DEFAULT_STREAM = 0xDA3E39CB94B95BDB
F = np.float32


class Pcg32:
    def __init__(self, state=PCG32_DEFAULT_STATE, inc=PCG32_DEFAULT_STREAM):
        self.state, self.inc = state, inc

    def seed(self, initstate: int, initseq: int = 1):
        self.state = 0
        self.inc = ((initseq << 1) | 1) & M64
        self.next_uint()
        self.state = (self.state + initstate) & M64
        self.next_uint()

    def next_uint(self) -> int:
        old = self.state
        self.state = (old * PCG_MULT + self.inc) & M64
        xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
        rot = old >> 59
        return ((xs >> rot) | (xs << ((-rot) & 31))) & 0xFFFFFFFF

    def next_float(self) -> np.float32:
        bits = np.uint32((self.next_uint() >> 9) | 0x3F800000)
        return bits.view(np.float32) - F(1.0)

    def advance(self, delta: int):
        cur_mult, cur_plus, acc_mult, acc_plus = PCG_MULT, self.inc, 1, 0
        delta &= M64
        while delta > 0:
            if delta & 1:
                acc_mult = (acc_mult * cur_mult) & M64
                acc_plus = (acc_plus * cur_mult + cur_plus) & M64
            cur_plus = ((cur_mult + 1) * cur_plus) & M64
            cur_mult = (cur_mult * cur_mult) & M64
            delta >>= 1
        self.state = (acc_mult * self.state + acc_plus) & M64


def logit(x):
    x = np.asarray(x, F)
    c = np.fmin(np.fmax(x, F(1e-9)), F(1.0) - F(1e-9))
    return (-O.logf(F(1.0) / c - F(1.0))).astype(F)


def logistic(x):
    x = np.asarray(x, F)
    return (F(1.0) / (F(1.0) + O.expf(-x))).astype(F)


def random_logistic(rng: Pcg32, n: int, mean=0.0, stddev=1.0) -> np.ndarray:
    """generate_random_logistic: element i + T j (T = ceil(n / 4) threads)
    takes stream position 4 i + j; the stream is then advanced by n."""
    if n <= 0:
        return np.zeros(0, F)
    threads = (n + 3) // 4
    # positions up to 4 * threads - 1 may be read
    r = Pcg32(rng.state, rng.inc)
    u = np.array([r.next_float() for _ in range(4 * threads)], F)
    idx = np.arange(n)
    pos = 4 * (idx % threads) + idx // threads
    out = (logit(u[pos]) * F(stddev) * F(0.551328895) + F(mean)).astype(F)
    rng.advance(n)
    return out


def densify_select(info: np.ndarray, scales: np.ndarray, grow_grad, grow_scale, absgrad: bool) -> np.ndarray:
    info = np.asarray(info, F).reshape(-1, 4)
    s = np.asarray(scales, F).reshape(-1, 3)
    accum = info[:, 2] if absgrad else info[:, 1]
    grad = (accum / np.fmax(info[:, 0], F(1.0))).astype(F)
    es = O.expf(s.reshape(-1)).reshape(-1, 3)
    smax = np.fmax(np.fmax(es[:, 0], es[:, 1]), es[:, 2])
    grow = (grad > F(grow_grad)) & (info[:, 0] > F(0.0))
    flags = np.where(grow, np.where(smax > F(grow_scale), 2, 1), 0).astype(np.uint8)
    return flags


def densify_apply(p: dict, n_old: int, src: np.ndarray, flags: np.ndarray, rnd: np.ndarray):
    """In place on the (already appended) parameter arrays of p: means (N,3),
    scales (N,3), rotations (N,4), opacities (N,), sh0 (N,3), sh_rest (N,45)."""
    for i, s in enumerate(src):
        t = n_old + i
        f = flags[s]
        if f == 0:
            continue
        r, x, y, z = [F(v) for v in p["rotations"][s]]
        p["rotations"][t] = p["rotations"][s]
        p["sh0"][t] = p["sh0"][s]
        p["sh_rest"][t] = p["sh_rest"][s]
        if f == 1:
            p["means"][t] = p["means"][s]
            p["scales"][t] = p["scales"][s]
            p["opacities"][t] = p["opacities"][s]
            continue
        two, one = F(2.0), F(1.0)
        m00 = one - two * (y * y + z * z)
        m01 = two * (x * y - r * z)
        m02 = two * (x * z + r * y)
        m10 = two * (x * y + r * z)
        m11 = one - two * (x * x + z * z)
        m12 = two * (y * z - r * x)
        m20 = two * (x * z - r * y)
        m21 = two * (y * z + r * x)
        m22 = one - two * (x * x + y * y)
        act = O.expf(p["scales"][s].astype(F))
        new_o = one - np.sqrt(one - logistic(p["opacities"][s:s + 1])[0])
        o_logit = logit(np.array([new_o], F))[0]
        r1 = rnd[6 * i:6 * i + 3].astype(F)
        r2 = rnd[6 * i + 3:6 * i + 6].astype(F)
        v1 = (r1 * (act + F(1e-5))).astype(F)
        v2 = (r2 * (act + F(1e-5))).astype(F)

        def mv(v):
            return np.array([(m00 * v[0] + m10 * v[1]) + m20 * v[2], (m01 * v[0] + m11 * v[1]) + m21 * v[2],
                             (m02 * v[0] + m12 * v[1]) + m22 * v[2]], F)

        o1, o2 = mv(v1), mv(v2)
        ls = O.logf((act / F(1.6)).astype(F))
        m = p["means"][s].astype(F).copy()
        p["means"][t] = m + o1
        p["scales"][t] = ls
        p["means"][s] = m + o2
        p["scales"][s] = ls
        p["opacities"][t] = o_logit
        p["opacities"][s] = o_logit


def prune_alive(p: dict, info: np.ndarray, n_info: int, min_opacity, scale_limit, radius_limit,
                prune_large: bool) -> np.ndarray:
    n = p["means"].shape[0]
    es = O.expf(p["scales"].astype(F).reshape(-1)).reshape(-1, 3)
    smax = np.fmax(np.fmax(es[:, 0], es[:, 1]), es[:, 2])
    not_large_ws = smax < F(scale_limit)
    rad = np.zeros(n, F)
    m = min(n, n_info)
    rad[:m] = np.asarray(info, F).reshape(-1, 4)[:m, 3]
    not_large_ss = (np.arange(n) >= n_info) | (rad < F(radius_limit))
    not_transparent = logistic(p["opacities"]) > F(min_opacity)
    q = np.abs(p["rotations"].astype(F))
    qs = ((q[:, 0] + q[:, 1]) + q[:, 2]) + q[:, 3]
    not_degenerate = qs > F(1.1920928955078125e-07)
    alive = not_transparent & ((not_large_ws & not_large_ss) | (not prune_large)) & not_degenerate
    return alive.astype(np.uint8)


def reset_opacity(opac: np.ndarray, max_opacity) -> np.ndarray:
    return logit(np.fmin(logistic(opac), F(max_opacity)))


def adam_remove_rows(alive: np.ndarray, num_kept: int) -> np.ndarray:
    """SimpleAdam::remove's mapping: copy_if over the first num_kept flags
    (the optimiser's Gaussians are already shrunk), zero-initialised tail."""
    rows = np.zeros(num_kept, np.int64)
    k = np.nonzero(alive[:num_kept])[0]
    rows[:k.size] = k
    return rows


class DefaultStrategy:
    """default.cu:40-69 on host arrays: p (parameters, as in densify_apply),
    m1 / m2 (Adam moments per group: means (N,3), opacities (N,), rotations
    (N,4), scales (N,3), sh0 (N,3), sh_rest (N,45)), info (N,4)."""

    def __init__(self, params: dict | None = None):
        self.prm = dict(pruning_opacity_threshold=0.005, pruning_scale_threshold=0.1, max_screen_size=10.0,
                        duplicate_grad_threshold=0.0002, duplicate_scale_threshold=0.01,
                        reset_reset_optimizer=False, absgrad=False, refine_every=100, start_refine=500,
                        end_refine=15000, max_num_gaussians=10_000_000, reset_every=3000, seed=42)
        self.rng = Pcg32()
        if params is not None:
            self.prm.update(params)
            self.rng.seed(int(self.prm["seed"]))
        self.step_count = 0
        self.counts = {}

    def step(self, p, m1, m2, info, grad_scaler, scene_scale, width, height):
        q = self.prm
        step = self.step_count
        if info is None:
            info = np.zeros((p["means"].shape[0], 4), F)
        if step % q["refine_every"] == 0 and q["start_refine"] <= step <= q["end_refine"]:
            if p["means"].shape[0] < q["max_num_gaussians"]:
                self._duplicate(p, m1, m2, info, grad_scaler, scene_scale)
            self._prune(p, m1, m2, info, scene_scale, width, height)
            info = np.zeros((p["means"].shape[0], 4), F)
        if q["reset_every"] > 0 and step % q["reset_every"] == 0 and q["start_refine"] <= step < q["end_refine"]:
            p["opacities"][:] = reset_opacity(p["opacities"], F(2.0) * F(q["pruning_opacity_threshold"]))
            m1["opacities"][:] = 0
            m2["opacities"][:] = 0
            if q["reset_reset_optimizer"]:
                for k in m1:
                    m1[k][:] = 0
                    m2[k][:] = 0
        self.step_count += 1
        return info

    def _duplicate(self, p, m1, m2, info, grad_scaler, scene_scale):
        q = self.prm
        n = p["means"].shape[0]
        flags = densify_select(info, p["scales"], F(q["duplicate_grad_threshold"]) * F(grad_scaler),
                               F(q["duplicate_scale_threshold"]) * F(scene_scale), q["absgrad"])
        src = np.nonzero(flags)[0]
        self.counts = {"duplicate": int((flags == 1).sum()), "split": int((flags == 2).sum())}
        g = src.size
        if g == 0:
            return
        for k in p:
            p[k] = np.concatenate([p[k], np.zeros((g,) + p[k].shape[1:], p[k].dtype)])
        for k in m1:
            m1[k] = np.concatenate([m1[k], np.zeros((g,) + m1[k].shape[1:], F)])
            m2[k] = np.concatenate([m2[k], np.zeros((g,) + m2[k].shape[1:], F)])
        rnd = random_logistic(self.rng, 6 * g, 0.0, 1.0)
        densify_apply(p, n, src, flags, rnd)

    def _prune(self, p, m1, m2, info, scene_scale, width, height):
        q = self.prm
        n_info = info.shape[0]
        alive = prune_alive(p, info, n_info, q["pruning_opacity_threshold"],
                            F(q["pruning_scale_threshold"]) * F(scene_scale),
                            F(max(width, height)) * F(q["max_screen_size"]),
                            self.step_count > q["reset_every"])
        kept = np.nonzero(alive)[0]
        nk = kept.size
        self.counts["kept"] = int(nk)
        if nk <= 0:
            return
        for k in p:
            p[k] = p[k][kept]
        rows = adam_remove_rows(alive, nk)
        for k in m1:
            m1[k] = m1[k][rows]
            m2[k] = m2[k][rows]
