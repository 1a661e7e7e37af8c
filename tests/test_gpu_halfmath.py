"""The fp16 rasterizer's canonical half operations on the GPU
(tinygs_amd/csrc/halfmath.h) against the oracle's (oracle/halfmath.h, pinned
by tests/test_halfmath_host.py): exp2 over all 65,536 inputs, the arithmetic
and conversions on random inputs with subnormals, packed and scalar; the
rounding of exact fixed-point sums; the lane layout of the DPP shift the fp16
blend backward uses."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _gpu(op, a, b=None, c=None):
    import torch
    from tinygs_amd import _lib
    view = {np.dtype(np.uint16): np.int16, np.dtype(np.int64): np.int64}.get(a.dtype, np.float32)
    ta = torch.from_numpy(np.ascontiguousarray(a).view(view)).cuda()
    tb = None if b is None else torch.from_numpy(b.view(np.int16)).cuda()
    tc = None if c is None else torch.from_numpy(c.view(np.int16)).cuda()
    out = torch.zeros(a.size, dtype=torch.int16, device="cuda")
    _lib.check(_lib.load().tgs_selftest_half(op, ta.data_ptr(), None if tb is None else tb.data_ptr(),
                                             None if tc is None else tc.data_ptr(), out.data_ptr(), a.size, None))
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


def _same(x, y):
    nan = (np.isnan(x.view(np.float16)) & np.isnan(y.view(np.float16)))
    return (x == y) | nan


def test_exp2_all_inputs(hip, orc):
    x = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = _gpu(0, x)
    want = orc.half_op(0, x)
    hw = _gpu(1, x)   # the hardware v_exp_f16, for the record
    bad_hw = ~_same(hw, want)
    print(f"[halfmath] v_exp_f16 differs from the correctly rounded exp2 on {np.count_nonzero(bad_hw)} "
          f"of 65536 inputs: {x[bad_hw][:8]}", flush=True)
    ok = _same(got, want)
    assert ok.all(), (np.count_nonzero(~ok), x[~ok][:8], got[~ok][:8], want[~ok][:8])


@pytest.mark.parametrize("op", [2, 3, 4, 5, 6, 9, 10])
def test_arithmetic(hip, orc, op):
    rng = np.random.default_rng(op)
    n = 1 << 20
    a, b, c = (rng.integers(0, 1 << 16, n).astype(np.uint16) for _ in range(3))
    # a quarter near cancellation for the fma forms
    if op in (2, 6):
        with np.errstate(all="ignore"):
            ab = (a.view(np.float16).astype(np.float32) * b.view(np.float16).astype(np.float32)).astype(np.float16)
        c[::4] = (-ab[::4]).view(np.uint16)
    got, want = _gpu(op, a, b, c), orc.half_op(op, a, b, c)
    ok = _same(got, want)
    assert ok.all(), (op, np.count_nonzero(~ok), a[~ok][:4], b[~ok][:4], c[~ok][:4], got[~ok][:4], want[~ok][:4])


@pytest.mark.parametrize("op", [7, 8])
def test_conversions(hip, orc, op):
    rng = np.random.default_rng(op)
    f = np.concatenate([rng.normal(0, 1, 1 << 19), rng.uniform(-70000, 70000, 1 << 17),
                        rng.uniform(-1e-6, 1e-6, 1 << 17), np.array([0.0, -0.0, 65504.0, 65520.0, -65520.0])]
                       ).astype(np.float32)
    got, want = _gpu(op, f), orc.half_op(op, f)
    assert np.array_equal(got, want), (op, np.count_nonzero(got != want))


def test_fixed_point_rounding(hip, orc):
    """half_of_fixed: the nearest half of S * 2^-24 (exact integer sums of halves)."""
    rng = np.random.default_rng(11)
    mag = rng.integers(0, 43, 1 << 18)
    s = (rng.integers(0, 1 << 62, 1 << 18) >> (62 - mag)) * rng.choice([-1, 1], 1 << 18)
    # exact halfway points and their neighbours at several binades
    q = rng.integers(1 << 10, 1 << 11, 4096)
    sh = rng.integers(1, 30, 4096)
    ties = (q << sh) + (1 << (sh - 1))
    s = np.concatenate([s, ties, ties - 1, ties + 1, -ties, [0, 1, -1, (65520 << 24) - 1, 65520 << 24]]).astype(np.int64)
    got, want = _gpu(11, s), orc.half_op(11, s)
    assert np.array_equal(got, want), (np.count_nonzero(got != want), s[got != want][:4])


def test_dpp_wave_shift_lane_layout(hip, orc):
    rng = np.random.default_rng(12)
    n = 64 * 64
    a = rng.integers(0, 1 << 16, n).astype(np.uint16)
    b = rng.integers(0, 1 << 16, n).astype(np.uint16)
    got, want = _gpu(12, a, b), orc.half_op(12, a, b)
    assert np.array_equal(got, want), np.count_nonzero(got != want)
