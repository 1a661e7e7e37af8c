"""The fp16 rasterizer's canonical half operations on the GPU
(tinygs_amd/csrc/halfmath.h) against the oracle's (oracle/halfmath.h, pinned
by tests/test_halfmath_host.py): exp2 over all 65,536 inputs in both lanes of
the packed form, the arithmetic and conversions on random inputs with
subnormals, packed and scalar; the rounding of exact fixed-point and double
sums; the lane layout of the DPP shift the fp16 blend backward uses."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _gpu(op, a, b=None, c=None):
    import torch
    from tinygs_amd import _lib
    view = {np.dtype(np.uint16): np.int16, np.dtype(np.int64): np.int64,
            np.dtype(np.float64): np.float64}.get(a.dtype, np.float32)
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


def test_packed_exp2_both_lanes(hip, orc):
    """The packed exp2 (two v_exp_f16, the second written into the high half)
    equals the canonical exp2 in both lanes for every input: element i takes
    lane i & 1 of exp2((a[i], b[i])); the second call swaps the roles, so
    every input passes through each lane."""
    x = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    xr = np.roll(x, 1)
    odd = (np.arange(x.size) & 1).astype(bool)
    for a, b in ((x, xr), (xr, x)):
        got = _gpu(13, a, b)
        want = orc.half_op(0, np.where(odd, b, a))
        ok = _same(got, want)
        assert ok.all(), (np.count_nonzero(~ok), a[~ok][:4], b[~ok][:4], got[~ok][:4], want[~ok][:4])


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


def test_double_sum_rounding(hip, orc):
    """half_of_double_sum (the fp16 preprocess backward's rounding of its exact
    double sums of half records) equals the correctly rounded half of the
    same value as an exact fixed-point integer, including sums a float ulp
    (or less) from a half midpoint, where rounding through float would round
    twice: m + 2^-24 for a midpoint m in [1, 2) is a float midpoint."""
    rng = np.random.default_rng(14)
    e = rng.integers(-13, 16, 4096)   # binade of the midpoint (sums of halves: multiples of 2^-24)
    q = rng.integers(1 << 10, 1 << 11, 4096)   # half significand
    mid = (2 * q + 1).astype(np.float64) * np.exp2(e - 11.0)   # a half midpoint
    k = rng.integers(-3, 4, 4096)
    near = np.concatenate([mid + k * 2.0 ** -24, mid, -(mid + 2.0 ** -24), mid + 2.0 ** -24])
    near = near[np.abs(near) < 2.0 ** 29]
    rand = rng.integers(-(1 << 52), 1 << 52, 1 << 16) >> rng.integers(0, 50, 1 << 16)
    s = np.concatenate([near, rand.astype(np.float64) * 2.0 ** -24, [0.0, 65519.0, 65520.0, -65520.0]])
    fixed = np.rint(s * 2.0 ** 24).astype(np.int64)
    assert np.array_equal(fixed.astype(np.float64) * 2.0 ** -24, s)   # exact: multiples of 2^-24
    got, want = _gpu(14, s), orc.half_op(11, fixed)
    assert np.array_equal(got, want), (np.count_nonzero(got != want), s[got != want][:4])
    # through float the midpoint cases round twice; at least one of them differs
    with np.errstate(over="ignore"):
        twice = s.astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.count_nonzero(twice != want) > 0
    special = _gpu(14, np.array([np.inf, -np.inf, np.nan]))
    assert special[0] == 0x7c00 and special[1] == 0xfc00 and np.isnan(special[2:].view(np.float16)).all()


def test_dpp_wave_shift_lane_layout(hip, orc):
    rng = np.random.default_rng(12)
    n = 64 * 64
    a = rng.integers(0, 1 << 16, n).astype(np.uint16)
    b = rng.integers(0, 1 << 16, n).astype(np.uint16)
    got, want = _gpu(12, a, b), orc.half_op(12, a, b)
    assert np.array_equal(got, want), np.count_nonzero(got != want)
