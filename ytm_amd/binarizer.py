"""Binarizers of src/tm_utils/binarizer.py (ThermometerBinarizer, Binarizer) with the binning
on the GPU.

The same classes, constructor arguments, methods, asserts and uint32 outputs as the
reference.  Fitting (min, max, percentiles) stays on the host in numpy, as in the reference.
The element-wise binning (transform, binarize_gray / binarize_rgb) and collapse_bins run in
libytm's HIP kernels (ytm_binarize, ytm_collapse_bins).  The comparisons use the type numpy
promotes the operands to, so results are bit-identical to the reference's:
  - int64 when data and thresholds are integers;
  - double otherwise, after exact widening of float16 / bool data; uint64 and other types are
    converted to float64, which is numpy's promotion against float64 thresholds.
"""
from __future__ import annotations

from typing import Literal

import numpy as np

from ._lib import DTYPES, check, lib, ptr

_THERMOMETER, _ONEHOT = 0, 1


def _dtype_code(Xd: np.ndarray) -> int:
    """YTM_DTYPE_* code of an array _device_input returned."""
    return DTYPES[Xd.dtype.name]


def _device_input(X: np.ndarray) -> np.ndarray:
    """X as a contiguous array of a type the GPU kernels take, with the same values."""
    X = np.asarray(X)
    if not X.dtype.isnative:
        X = X.astype(X.dtype.newbyteorder("="))
    if X.dtype == np.bool_:
        X = X.astype(np.uint8)
    elif X.dtype == np.float16:
        X = X.astype(np.float32)
    elif X.dtype.name not in DTYPES:
        X = X.astype(np.float64)
    return np.ascontiguousarray(X)


def _device_levels(X, thresholds, kind: int, edge_bins: bool):
    """(X for the kernels, threshold array, whether the comparison is in int64, levels per
    value) of a binning: the comparison type numpy promotes X and the thresholds to."""
    Xd = _device_input(X)
    t = np.asarray(thresholds)
    int_thr = (np.issubdtype(t.dtype, np.integer) and t.dtype != np.uint64
               and np.issubdtype(Xd.dtype, np.integer))
    t = np.ascontiguousarray(t, dtype=np.int64 if int_thr else np.float64)
    width = t.size if kind == _THERMOMETER else t.size - 1 + (2 if edge_bins else 0)
    return Xd, t, int_thr, width


def _binarize(X, thresholds, kind: int, edge_bins: bool) -> np.ndarray:
    Xd, t, int_thr, width = _device_levels(X, thresholds, kind, edge_bins)
    nthr = t.size
    out = np.empty(Xd.shape + (width,), dtype=np.uint32)
    check(lib.ytm_binarize(ptr(Xd), DTYPES[Xd.dtype.name], Xd.size, ptr(t), int(int_thr), nthr, kind,
                           int(bool(edge_bins)), ptr(out)))
    return out


def _collapse(B, kind: int, edge_bins: bool) -> np.ndarray:
    B = np.asarray(B)
    if B.dtype not in (np.bool_, np.uint8, np.uint16, np.uint32):
        raise TypeError(f"collapse_bins takes the binarizer's uint32 output (or bool / uint8 / uint16), got {B.dtype}")
    B = np.ascontiguousarray(B, dtype=np.uint32)
    width = B.shape[-1]
    rows = B.size // width if width else int(np.prod(B.shape[:-1]))
    out = np.empty(B.shape[:-1], dtype=np.int64)
    check(lib.ytm_collapse_bins(ptr(B), rows, width, kind, int(bool(edge_bins)), ptr(out)))
    return out


class ThermometerBinarizer:
    """src/tm_utils/binarizer.py:5-22: ch thermometer levels of 8-bit intensities, thresholds
    j * 255 / (ch + 1) for j = 1..ch."""

    def __init__(self, ch: int = 8):
        self.ch = ch

    def _thresholds(self) -> np.ndarray:
        return np.arange(1, self.ch + 1) * 255 / (self.ch + 1)

    def _levels(self):
        """Thresholds, kind and edge flag of the binning (for encode_binarized)."""
        return self._thresholds(), _THERMOMETER, False

    def binarize_gray(self, X):
        """(N, H, W) -> uint32 (N, H, W, ch)."""
        assert X.ndim == 3, "Input should be a 3D array (N, H, W)"
        return _binarize(X, self._thresholds(), _THERMOMETER, False)

    def binarize_rgb(self, X):
        """(N, H, W, C) -> uint32 (N, H, W, C * ch), channel-major: index c * ch + j."""
        assert X.ndim == 4, "Input should be a 4D array (N, H, W, C)"
        out = _binarize(X, self._thresholds(), _THERMOMETER, False)
        return out.reshape((X.shape[0], X.shape[1], X.shape[2], X.shape[3] * self.ch))


class Binarizer:
    """src/tm_utils/binarizer.py:25-136: bins thresholds between the data's min and max,
    evenly spaced (uniform) or at evenly spaced percentiles (quantile), or given; thermometer
    or one-hot codes, with optional edge bins."""

    def __init__(
        self,
        bins: int,
        edge_bins: bool = False,
        method: Literal["uniform", "quantile"] = "uniform",
        type: Literal["thermometer", "onehot"] = "thermometer",
    ):
        self.bins = bins
        self.edge_bins = edge_bins
        self.method = method
        self.type = type

    def fit(self, X, thresholds=None, min_val=None, max_val=None):
        assert X.ndim >= 2
        self.min_val = np.min(X) if min_val is None else min_val
        self.max_val = np.max(X) if max_val is None else max_val
        if thresholds is not None:
            assert len(thresholds) == self.bins
            inner = thresholds
        elif self.method == "quantile":
            inner = np.percentile(X, np.linspace(0, 100, self.bins + 2)[1:-1])
        elif self.method == "uniform":
            inner = np.linspace(self.min_val, self.max_val, self.bins + 2)[1:-1]
        else:
            raise ValueError(f"Unknown method: {self.method}")
        self.thresholds = np.concatenate(([self.min_val], inner, [self.max_val]))
        assert len(self.thresholds) == self.bins + 2

    def _levels(self):
        """Thresholds, kind and edge flag of transform (for encode_binarized)."""
        if self.type == "thermometer":
            return (self.thresholds if self.edge_bins else self.thresholds[1:-1]), _THERMOMETER, False
        if self.type == "onehot":
            return self.thresholds, _ONEHOT, self.edge_bins
        raise ValueError(f"Unknown type: {self.type}")

    def _transform_thermometer(self, X):
        t = self.thresholds if self.edge_bins else self.thresholds[1:-1]
        return _binarize(X, t, _THERMOMETER, False)

    def _transform_onehot(self, X):
        return _binarize(X, self.thresholds, _ONEHOT, self.edge_bins)

    def collapse_bins(self, X):
        assert X.ndim >= 3, "Input should be at least a 3D array (N, ... , binned_dim)"
        if self.type == "thermometer":
            if self.edge_bins:
                assert X.shape[-1] == self.bins + 2, (
                    f"Last dim should contain {self.bins + 2} elements, got {X.shape[-1]}"
                )
            else:
                assert X.shape[-1] == self.bins, f"Last dim should contain {self.bins} elements, got {X.shape[-1]}"
            return _collapse(X, _THERMOMETER, self.edge_bins)
        elif self.type == "onehot":
            if self.edge_bins:
                assert X.shape[-1] == self.bins + 3, (
                    f"Last dim should contain {self.bins + 3} elements, got {X.shape[-1]}"
                )
            else:
                assert X.shape[-1] == self.bins + 1, (
                    f"Last dim should contain {self.bins + 1} elements, got {X.shape[-1]}"
                )
            return _collapse(X, _ONEHOT, self.edge_bins)
        else:
            raise ValueError(f"Unknown type: {self.type}")

    def transform(self, X):
        if self.type == "thermometer":
            return self._transform_thermometer(X)
        elif self.type == "onehot":
            return self._transform_onehot(X)
        else:
            raise ValueError(f"Unknown type: {self.type}")

    def fit_transform(self, X):
        self.fit(X)
        return self.transform(X)
