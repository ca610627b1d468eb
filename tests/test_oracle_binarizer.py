"""The binarizer oracle (oracle/binarizer.py) pinned on the CPU: hand-computed known answers,
np.searchsorted (a library routine independent of the oracle) for every bin index, and the
invariants of the codes.  src/tm_utils/binarizer.py holds no tests or fixtures of its own;
its call sites (test/cutm/fmnist_conv.py:40-43, octmnist.py:14-17, celeba_conv.py:48-49)
fix the uses covered here: uint8 images, 8 uniform thermometer bins, gray and RGB levels."""
import numpy as np
import pytest

from oracle import binarizer as ob


def test_thermometer_levels_known_answers():
    t = ob.thermometer_thresholds(8)
    np.testing.assert_array_equal(t, np.array([255 * j / 9 for j in range(1, 9)]))
    assert t[2] == 85.0 and t[5] == 170.0  # exact levels: pixel 85 reaches level 3, 84 does not
    X = np.array([0, 28, 29, 84, 85, 170, 254, 255], dtype=np.uint8)
    expect = np.array([[0] * 8, [0] * 8, [1] + [0] * 7, [1, 1] + [0] * 6, [1, 1, 1] + [0] * 5,
                       [1] * 6 + [0] * 2, [1] * 8, [1] * 8], dtype=np.uint32)
    np.testing.assert_array_equal(ob.thermometer(X, t), expect)


def test_fit_thresholds_known_answers():
    X = np.array([[0, 10], [4, 7]], dtype=np.uint8)
    np.testing.assert_array_equal(ob.fit_thresholds(X, 4), [0, 2, 4, 6, 8, 10])
    Q = np.arange(101, dtype=np.float64).reshape(1, -1)  # percentiles of 0..100 are the values themselves
    np.testing.assert_array_equal(ob.fit_thresholds(Q, 3, "quantile"), [0, 25, 50, 75, 100])
    np.testing.assert_array_equal(ob.fit_thresholds(X, 2, thresholds=[3, 5]), [0, 3, 5, 10])
    np.testing.assert_array_equal(ob.fit_thresholds(X, 1, min_val=-5, max_val=5), [-5, 0, 5])
    with pytest.raises(ValueError):
        ob.fit_thresholds(X, 2, "nope")


def test_onehot_known_answers():
    t = np.array([0.0, 2.0, 4.0, 6.0])
    X = np.array([-1.0, 0.0, 1.9, 2.0, 5.0, 6.0, 7.0])
    no_edge = np.array([[0, 0, 0], [1, 0, 0], [1, 0, 0], [0, 1, 0], [0, 0, 1], [0, 0, 0], [0, 0, 0]])
    np.testing.assert_array_equal(ob.onehot(X, t, False), no_edge)
    edge = np.concatenate([(X < 0)[:, None], no_edge, (X >= 6)[:, None]], axis=1)
    np.testing.assert_array_equal(ob.onehot(X, t, True), edge)
    assert ob.onehot(X, t, True).dtype == np.uint32


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_codes_against_searchsorted(seed):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(50, 7))
    X[0, :3] = [-10.0, 10.0, 0.0]
    t = np.sort(rng.normal(size=6))
    X[1, :6] = t  # ties: values equal to thresholds
    level = np.searchsorted(t, X, side="right")  # thresholds <= X
    th = ob.thermometer(X, t)
    np.testing.assert_array_equal(th.sum(-1), level)
    assert np.all(np.diff(th.astype(np.int64), axis=-1) <= 0)  # a prefix of ones
    np.testing.assert_array_equal(ob.collapse(th, "thermometer", False), level)
    oh = ob.onehot(X, t, True)
    assert np.all(oh.sum(-1) == 1)  # with edge bins every value has exactly one bin
    np.testing.assert_array_equal(np.argmax(oh, -1), level)  # bin 0: below t[0]; last: >= t[-1]
    np.testing.assert_array_equal(ob.collapse(oh, "onehot", True), level - 1)
    oh0 = ob.onehot(X, t, False)
    inside = (X >= t[0]) & (X < t[-1])
    assert np.all(oh0.sum(-1) == inside)
    np.testing.assert_array_equal(ob.collapse(oh0, "onehot", False)[inside], (level - 1)[inside])


def test_collapse_edge_cases():
    B = np.array([[0, 0, 0], [1, 0, 0], [1, 1, 1], [0, 1, 0]], dtype=np.uint32)
    np.testing.assert_array_equal(ob.collapse(B, "thermometer", False), [0, 1, 3, 2])
    np.testing.assert_array_equal(ob.collapse(B, "thermometer", True), [-1, 0, 2, 1])
    np.testing.assert_array_equal(ob.collapse(B, "onehot", False), [0, 0, 0, 1])  # first maximum
    np.testing.assert_array_equal(ob.collapse(B, "onehot", True), [-1, -1, -1, 0])
