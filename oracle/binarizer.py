"""Test infrastructure: a numpy restatement of the reference's binarizers
(src/tm_utils/binarizer.py), the checker for ytm_amd.binarizer.  Only tests/ may use it.

Each function states the reference lines it follows.  Pinned by tests/test_oracle_binarizer.py:
hand-computed known answers, np.searchsorted (a library routine independent of this code)
for every bin index, and the invariants of the encodings (thermometer rows are prefixes of
ones, one-hot rows hold at most one 1).
"""
from __future__ import annotations

import numpy as np


def thermometer_thresholds(ch: int) -> np.ndarray:
    """ThermometerBinarizer thresholds j * 255 / (ch + 1), j = 1..ch, float64
    (binarizer.py:10,17)."""
    return np.arange(1, ch + 1) * 255 / (ch + 1)


def fit_thresholds(X, bins: int, method: str = "uniform", thresholds=None, min_val=None, max_val=None) -> np.ndarray:
    """Binarizer.fit (binarizer.py:39-54): [min, inner..., max], bins + 2 values; inner is the
    given list, the bins evenly spaced percentiles strictly between 0 and 100 (quantile), or
    the bins evenly spaced values strictly between min and max (uniform)."""
    lo = np.min(X) if min_val is None else min_val
    hi = np.max(X) if max_val is None else max_val
    if thresholds is not None:
        assert len(thresholds) == bins
        inner = thresholds
    elif method == "quantile":
        inner = np.percentile(X, np.linspace(0, 100, bins + 2)[1:-1])
    elif method == "uniform":
        inner = np.linspace(lo, hi, bins + 2)[1:-1]
    else:
        raise ValueError(f"Unknown method: {method}")
    return np.concatenate(([lo], inner, [hi]))


def thermometer(X, t) -> np.ndarray:
    """Thermometer bits (binarizer.py:12-15,19-21,63-73): out[..., j] = X >= t[j], uint32."""
    X = np.asarray(X)
    t = np.asarray(t)
    out = np.zeros(X.shape + (len(t),), dtype=np.uint32)
    for j in range(len(t)):
        out[..., j] = X >= t[j]
    return out


def onehot(X, t, edge_bins: bool) -> np.ndarray:
    """One-hot bits (binarizer.py:75-86): the len(t) - 1 intervals t[j] <= X < t[j + 1], with
    X < t[0] before and X >= t[-1] after them when edge_bins; uint32."""
    X = np.asarray(X)
    t = np.asarray(t)
    cols = [(X >= t[j]) & (X < t[j + 1]) for j in range(len(t) - 1)]
    if edge_bins:
        cols = [X < t[0]] + cols + [X >= t[-1]]
    return np.stack(cols, axis=-1).astype(np.uint32)


def collapse(B, kind: str, edge_bins: bool) -> np.ndarray:
    """Binarizer.collapse_bins (binarizer.py:88-105): thermometer -> 1 + index of the last
    non-zero value along the last axis (0 if none); one-hot -> index of the first maximum;
    minus 1 with edge bins."""
    B = np.asarray(B)
    if kind == "thermometer":
        nz = B != 0
        width = B.shape[-1]
        last = width - np.argmax(nz[..., ::-1], axis=-1)
        out = np.where(nz.any(axis=-1), last, 0).astype(np.int64)
    else:
        out = np.argmax(B, axis=-1).astype(np.int64)
    return out - 1 if edge_bins else out
