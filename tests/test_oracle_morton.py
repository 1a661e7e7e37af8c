"""The Morton-order restatement (oracle/morton.py) pinned on the CPU: the
bit interleave against its definition and known answers, the quantisation
against hand-worked boxes, and the order's sortedness and stability."""
import numpy as np

from oracle import morton as M


def test_interleave_known_answers():
    assert M.interleave_bits(1, 0, 0) == 1
    assert M.interleave_bits(0, 1, 0) == 2
    assert M.interleave_bits(0, 0, 1) == 4
    assert M.interleave_bits(2, 0, 0) == 8
    assert M.interleave_bits(0, 0, 512) == 1 << 29
    assert M.interleave_bits(1023, 1023, 1023) == (1 << 30) - 1
    # de-interleaving gives the coordinates back
    rng = np.random.default_rng(0)
    for qx, qy, qz in rng.integers(0, 1024, (200, 3)):
        c = M.interleave_bits(int(qx), int(qy), int(qz))
        back = [sum(((c >> (3 * k + a)) & 1) << k for k in range(10)) for a in range(3)]
        assert back == [qx, qy, qz]


def test_vectorised_codes_equal_the_definition():
    rng = np.random.default_rng(1)
    means = rng.normal(0, 1, (500, 3)).astype(np.float32)
    q = M.quantise(means)
    c = M.codes(means)
    for i in range(len(means)):
        assert int(c[i]) == M.interleave_bits(int(q[i, 0]), int(q[i, 1]), int(q[i, 2]))


def test_quantise_box_corners_and_degenerate_axis():
    means = np.array([[0.0, 5.0, -2.0], [1.0, 5.0, 2.0], [0.5, 5.0, 0.0]], np.float32)
    q = M.quantise(means)
    # x in [0, 1]: 0, 1023 and truncate(0.5 * 1023) = 511; y constant: the
    # extent is clamped to 1e-8 and every (y - min) is 0; z in [-2, 2]
    assert q[:, 0].tolist() == [0, 1023, 511]
    assert q[:, 1].tolist() == [0, 0, 0]
    assert q[:, 2].tolist() == [0, 1023, 511]


def test_order_is_a_stable_sort_of_the_codes():
    rng = np.random.default_rng(2)
    means = rng.uniform(-3, 3, (3000, 3)).astype(np.float32)
    means[1000:1100] = means[5]          # duplicates: equal codes keep their index order
    order = M.morton_order(means)
    c = M.codes(means)
    assert sorted(order.tolist()) == list(range(len(means)))
    assert np.all(np.diff(c[order].astype(np.int64)) >= 0)
    same = [i for i in order.tolist() if c[i] == c[5]]
    assert same == sorted(same)
    info = rng.normal(0, 1, (3000, 4)).astype(np.float32)
    assert np.array_equal(M.densification_reorder(info, order), info[order])
