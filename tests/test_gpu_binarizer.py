"""ytm_amd.binarizer (HIP kernels ytm_binarize / ytm_collapse_bins) against the numpy
oracle (oracle/binarizer.py), bit for bit: every input type the kernels take, integer and
float thresholds, thermometer and one-hot with and without edge bins, ties at the
thresholds, NaN, empty and ragged shapes, and the reference's own uses (uint8 images, 8
thermometer levels)."""
import zlib

import numpy as np
import pytest

from oracle import binarizer as ob

pytestmark = pytest.mark.gpu

ytm_amd = pytest.importorskip("ytm_amd")
from ytm_amd.binarizer import Binarizer, ThermometerBinarizer  # noqa: E402

DTYPES = ["uint8", "int8", "uint16", "int16", "uint32", "int32", "int64", "float32", "float64", "float16", "bool",
          "uint64"]


def sample(dtype, shape, rng):
    if dtype == "bool":
        return rng.random(shape) < 0.5
    if dtype.startswith("float"):
        X = rng.normal(scale=40.0, size=shape).astype(dtype)
        X.flat[:4] = [0.0, -0.0, 25.0, 50.0][: X.size]
        return X
    info = np.iinfo(dtype)
    lo, hi = max(int(info.min), -100), min(int(info.max), 300)
    return rng.integers(lo, hi, size=shape, endpoint=True).astype(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("method", ["uniform", "quantile"])
def test_binarizer_matches_oracle(dtype, method):
    rng = np.random.default_rng(zlib.crc32(f"{dtype}/{method}".encode()))
    X = sample(dtype, (37, 5, 3), rng)
    if dtype == "bool" and method == "quantile":  # numpy's percentile rejects booleans, as in the reference
        with pytest.raises(TypeError):
            Binarizer(4, method=method).fit(X)
        return
    for bins in (1, 4, 9):
        for edge in (False, True):
            for kind in ("thermometer", "onehot"):
                b = Binarizer(bins, edge_bins=edge, method=method, type=kind)
                b.fit(X)
                t = ob.fit_thresholds(X, bins, method)
                np.testing.assert_array_equal(b.thresholds, t)
                got = b.transform(X)
                want = ob.thermometer(X, t if edge else t[1:-1]) if kind == "thermometer" else ob.onehot(X, t, edge)
                assert got.dtype == np.uint32 and got.shape == want.shape
                np.testing.assert_array_equal(got, want, err_msg=f"{dtype} {method} {bins} {edge} {kind}")
                np.testing.assert_array_equal(b.collapse_bins(got), ob.collapse(want, kind, edge))


@pytest.mark.parametrize("dtype", ["uint8", "int16", "int32", "int64", "float32"])
def test_given_thresholds_integer_and_float(dtype):
    rng = np.random.default_rng(5)
    X = sample(dtype, (64, 11), rng)
    for thr in ([-7, 0, 3, 50], [-7.5, 0.0, 3.25, 50.0]):
        for kind in ("thermometer", "onehot"):
            b = Binarizer(4, edge_bins=True, type=kind)
            b.fit(X, thresholds=thr)
            t = ob.fit_thresholds(X, 4, thresholds=thr)
            assert b.thresholds.dtype == t.dtype
            want = ob.thermometer(X, t) if kind == "thermometer" else ob.onehot(X, t, True)
            np.testing.assert_array_equal(b.transform(X), want)
    # integers compared as int64, not double: 2**53 < 2**53 + 1 although both round to 2**53
    Xi = np.array([[-7, 0, 3, 50, 2**53, 2**53 + 1]], dtype=np.int64)
    b = Binarizer(1, edge_bins=False)
    b.fit(Xi, thresholds=[2**53 + 1], min_val=-7, max_val=2**53 + 2)
    assert b.thresholds.dtype == np.int64
    got = b.transform(Xi)
    np.testing.assert_array_equal(got, ob.thermometer(Xi, b.thresholds[1:-1]))
    np.testing.assert_array_equal(got[0, :, 0], [0, 0, 0, 0, 0, 1])


def test_nan_and_non_native_byte_order():
    X = np.array([[np.nan, 1.0, -np.inf, np.inf, 2.5]], dtype=np.float64)
    for kind in ("thermometer", "onehot"):
        b = Binarizer(3, edge_bins=True, type=kind)
        b.fit(X, min_val=0.0, max_val=4.0)
        t = ob.fit_thresholds(X, 3, min_val=0.0, max_val=4.0)
        want = ob.thermometer(X, t) if kind == "thermometer" else ob.onehot(X, t, True)
        np.testing.assert_array_equal(b.transform(X), want)
        np.testing.assert_array_equal(b.transform(X.astype(">f8")), want)


def test_thermometer_binarizer_gray_rgb():
    rng = np.random.default_rng(9)
    for ch in (1, 8, 13):
        tb = ThermometerBinarizer(ch)
        t = ob.thermometer_thresholds(ch)
        gray = rng.integers(0, 256, size=(6, 28, 28), dtype=np.uint8)
        gray[0, 0, :9] = [0, 28, 29, 84, 85, 170, 254, 255, 128]
        out = tb.binarize_gray(gray)
        assert out.dtype == np.uint32 and out.shape == (6, 28, 28, ch)
        np.testing.assert_array_equal(out, ob.thermometer(gray, t))
        rgb = rng.integers(0, 256, size=(4, 8, 9, 3), dtype=np.uint8)
        out = tb.binarize_rgb(rgb)
        assert out.shape == (4, 8, 9, 3 * ch)
        np.testing.assert_array_equal(out, ob.thermometer(rgb, t).reshape(4, 8, 9, 3 * ch))
    with pytest.raises(AssertionError):
        ThermometerBinarizer(8).binarize_gray(np.zeros((2, 3), np.uint8))


def test_reference_pipeline_and_edge_shapes():
    """fmnist_conv.py:40-43: Binarizer(8) fitted on uint8 images, transformed and flattened."""
    rng = np.random.default_rng(3)
    imgs = rng.integers(0, 256, size=(40, 28, 28), dtype=np.uint8)
    b = Binarizer(8)
    b.fit(imgs)
    flat = b.transform(imgs).reshape((imgs.shape[0], -1)).astype(np.uint32)
    want = ob.thermometer(imgs, ob.fit_thresholds(imgs, 8)[1:-1]).reshape((40, -1))
    np.testing.assert_array_equal(flat, want)
    # empty input, 2-D input, one row
    for X in (np.zeros((0, 5), np.float32), rng.normal(size=(1, 1)), rng.normal(size=(3, 1, 2, 1, 2))):
        b = Binarizer(3, edge_bins=True, type="onehot")
        b.fit(X, min_val=-1.0, max_val=1.0)
        t = ob.fit_thresholds(X, 3, min_val=-1.0, max_val=1.0)
        np.testing.assert_array_equal(b.transform(X), ob.onehot(X, t, True))
    with pytest.raises(AssertionError):
        b.collapse_bins(np.zeros((2, 5), np.uint32))
    with pytest.raises(TypeError):
        b.collapse_bins(np.zeros((2, 3, 6), np.float32))


def test_large_transform_properties():
    """A config-4-sized RGB batch (CIFAR-shaped, 8 levels: dim (32, 32, 24)): the thermometer
    count per pixel equals the level from np.searchsorted."""
    rng = np.random.default_rng(4)
    rgb = rng.integers(0, 256, size=(2000, 32, 32, 3), dtype=np.uint8)
    out = ThermometerBinarizer(8).binarize_rgb(rgb).reshape(2000, 32, 32, 3, 8)
    level = np.searchsorted(ob.thermometer_thresholds(8), rgb, side="right")
    np.testing.assert_array_equal(out.sum(-1, dtype=np.int64), level)
    assert np.all(np.diff(out.astype(np.int8), axis=-1) <= 0)


# ------------------------------------------------------------------ binning fused into encode
@pytest.mark.parametrize("case", ["rgb", "gray", "thermometer", "thermometer_edges", "onehot", "onehot_edges",
                                  "int_thresholds"])
def test_encode_binarized(case):
    """encode_binarized (ytm_encode_binarized: the binning done where encode reads each value)
    gives the words of encode() on the binarizer's output, and of the oracle's encode of the
    oracle's binning: ThermometerBinarizer on uint8 images (config 4's CIFAR shape, 3x3
    patches; a gray config-3 shape, 10x10 patches), and Binarizer thermometer / one-hot codes,
    with and without edge bins, on a one-patch model, float data and integer data with integer
    thresholds."""
    from ytm_amd import MultiClassTM
    from oracle import oracle as orc

    rng = np.random.default_rng(zlib.crc32(case.encode()))
    if case == "rgb":
        X = rng.integers(0, 256, (5, 32, 32, 3)).astype(np.uint8)
        b = ThermometerBinarizer(8)
        kw = dict(dim=(32, 32, 24), patch_dim=(3, 3))
        binned = ob.thermometer(X, ob.thermometer_thresholds(8))
    elif case == "gray":
        X = rng.integers(0, 256, (4, 28, 28)).astype(np.uint8)
        b = ThermometerBinarizer(3)
        kw = dict(dim=(28, 28, 3), patch_dim=(10, 10))
        binned = ob.thermometer(X, ob.thermometer_thresholds(3))
    else:
        edge = case.endswith("edges")
        kind = "onehot" if case.startswith("onehot") else "thermometer"
        if case == "int_thresholds":
            X = rng.integers(-50, 50, (30, 40)).astype(np.int16)
            b = Binarizer(3, type="thermometer")
            b.fit(X, thresholds=np.array([-10, 0, 25], dtype=np.int64))
            t = ob.fit_thresholds(X, 3, thresholds=np.array([-10, 0, 25], dtype=np.int64))
        else:
            X = rng.normal(size=(30, 40)).astype(np.float32)
            b = Binarizer(4, edge_bins=edge, type=kind)
            b.fit(X)
            t = ob.fit_thresholds(X, 4)
        binned = (ob.thermometer(X, t if edge else t[1:-1]) if kind == "thermometer" or case == "int_thresholds"
                  else ob.onehot(X, t, edge))
        kw = dict(dim=(40 * binned.shape[-1], 1, 1))
    N = X.shape[0]
    tm = MultiClassTM(4, 10, 3.0, n_classes=2, seed=1, **kw)
    ref = orc.OracleTM(4, 10, 3.0, n_classes=2, seed=1, **kw)
    got = tm.encode_binarized(X, b)
    binned = np.ascontiguousarray(binned.reshape(N, -1), dtype=np.uint32)
    np.testing.assert_array_equal(got, tm.encode(binned), err_msg=f"{case}: against encode of the binned rows")
    np.testing.assert_array_equal(got, ref.encode(binned), err_msg=f"{case}: against the oracle")


def test_encode_binarized_checks_the_size():
    from ytm_amd import MultiClassTM

    tm = MultiClassTM(4, 10, 3.0, (32, 32, 24), 2, patch_dim=(3, 3), seed=1)
    with pytest.raises(AssertionError):
        tm.encode_binarized(np.zeros((2, 32, 32, 3), dtype=np.uint8), ThermometerBinarizer(4))
