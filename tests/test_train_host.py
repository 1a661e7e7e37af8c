"""Host logic of the training loop (no GPU): data-loader order, LR
schedulers, SH-degree schedule, scene scale."""
import math

import numpy as np

from oracle import train as T


class _DS:
    def __init__(self, n):
        self.n = n

    def size(self):
        return self.n

    def __getitem__(self, i):
        return i


def test_data_loader_permutation_matches_oracle():
    """SimpleDataLoader's order is the Fisher-Yates permutation drawn from
    pcg32 seeded 0 (simple.cpp:17-35), renewed every epoch; the library's
    bounded pcg32 and the oracle's agree."""
    from tinygs_amd.data import SimpleDataLoader
    ld = SimpleDataLoader(_DS(37))
    ref = T.Loader(37)
    assert ld.m_permutation == [ref.next() for _ in range(37)]
    assert sorted(ld.m_permutation) == list(range(37))
    ld.generate_permutation()
    assert ld.m_permutation == [ref.next() for _ in range(37)]


def test_bounded_pcg32_is_unbiased_rejection():
    from oracle import strategy as S
    r = S.Pcg32()
    r.seed(1)
    # bound 3: threshold (2^32 - 3) % 3 = 1, so only the output 0 is rejected
    assert ((~3 + 1) & 0xFFFFFFFF) % 3 == 1
    vals = [T.next_bounded(r, 3) for _ in range(3000)]
    counts = np.bincount(vals, minlength=3)
    assert counts.min() > 900


class _Opt:
    def __init__(self):
        self.lr = None

    def set_lr(self, lr):
        self.lr = lr


def test_exponential_lr():
    from tinygs_amd.trainer import ExponentialLR, create_lr_scheduler
    o = _Opt()
    s = ExponentialLR(o, 0.01, 0.9)
    assert o.lr == np.float32(0.01)
    seq = [s.step() for _ in range(4)]
    want = [float(np.float32(np.float32(0.01) * math.pow(np.float32(0.9), k))) for k in range(4)]
    assert seq == want and o.lr == want[-1]
    s.reset()
    assert o.lr == np.float32(0.01)
    c = create_lr_scheduler("constant", o, {"lr": 0.5})
    assert c.step() == 0.5


def test_sh_degree_schedule():
    from tinygs_amd.trainer import Orchestrator, OrchestratorConfig, TrainingState

    class G:
        d = 3

        def set_sh_degree(self, d):
            self.d = d

    o = Orchestrator.__new__(Orchestrator)
    o.m_config = OrchestratorConfig(sh_degree_interval=10, max_sh_degree=2)
    o.m_gaussians = G()
    o.m_state = TrainingState()
    seen = []
    for step in range(45):
        o.m_state.current_step = step
        o.update_sh_degree()
        seen.append(o.m_gaussians.d)
    assert seen[0] == 0 and seen[9] == 0 and seen[10] == 1 and seen[20] == 2 and seen[44] == 2


def test_scene_scale_restatement():
    pts = np.random.default_rng(0).normal(0, 1, (1000, 3)).astype(np.float32)
    cams = np.array([[4, 0, 0], [0, -5, 0]], np.float32)
    s = T.scene_scale(pts, cams)
    m = pts.mean(0)
    assert abs(s - max(np.linalg.norm(c - m) for c in cams)) < 1e-4


def test_oracle_psnr_closed_form():
    from tinygs_amd.image import ImageShape
    shape = ImageShape(13, 9)
    g = np.random.default_rng(3)
    pred = g.uniform(-0.5, 1.5, shape.padded_size).astype(np.float32)
    target = g.uniform(0.0, 1.0, shape.padded_size).astype(np.float32)
    d = np.clip(pred.astype(np.float64), 0.0, 1.0) - target
    want = -10.0 * math.log10((d * d).sum() / shape.size())
    assert abs(T.psnr(pred, target, shape) - want) < 1e-4
    assert T.psnr(target, target, shape) == 100.0
