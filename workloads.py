"""Seeded synthetic workloads of the five benchmark configurations.

Each generator returns raw (un-encoded) uint32 inputs of shape (N, dim0*dim1*dim2) with
values 0/1 as BaseTM.encode requires (src/cutm/base.py:229-230), integer labels, and the
constructor arguments of the model the configuration names.  No network, no datasets:
everything is drawn from numpy generators with fixed seeds.
"""
from __future__ import annotations

import numpy as np

CONFIGS = {
    1: dict(name="noisy_xor", n_train=5000, n_test=5000, epochs=10,
            model=dict(number_of_clauses_per_class=10, T=15, s=3.9, dim=(12, 1, 1), n_classes=2)),
    2: dict(name="mnist_shaped", n_train=60000, n_test=10000,
            model=dict(number_of_clauses_per_class=2000, T=50, s=10.0, dim=(28, 28, 1), n_classes=10)),
    3: dict(name="conv28_10x10", n_train=60000, n_test=10000,
            model=dict(number_of_clauses_per_class=8000, T=10000, s=5.0, dim=(28, 28, 1), n_classes=10,
                       patch_dim=(10, 10))),
    4: dict(name="cifar_shaped_3x3", n_train=50000, n_test=10000,
            model=dict(number_of_clauses_per_class=20000, T=15000, s=10.0, dim=(32, 32, 24), n_classes=10,
                       patch_dim=(3, 3))),
    5: dict(name="text_bow", n_train=25000, n_test=25000,
            model=dict(number_of_clauses_per_class=10000, T=8000, s=2.0, dim=(10000, 1, 1), n_classes=2)),
}

DATA_SEED = 2024
MODEL_SEED = 7


def _noisy_xor(rng, n_train, n_test):
    X = rng.integers(0, 2, (n_train, 12)).astype(np.uint32)
    y = (X[:, 0] ^ X[:, 1]).astype(np.uint32)
    flips = rng.choice(n_train, size=min(n_train, round(0.4 * n_train)), replace=False)
    y[flips] ^= 1
    Xt = rng.integers(0, 2, (n_test, 12)).astype(np.uint32)
    yt = (Xt[:, 0] ^ Xt[:, 1]).astype(np.uint32)
    return X, y, Xt, yt


def _templates(rng, n_classes=10, size=28, sigma=3.0):
    from scipy.ndimage import gaussian_filter

    out = np.empty((n_classes, size, size))
    for k in range(n_classes):
        f = gaussian_filter(rng.standard_normal((size, size)), sigma)
        f = (f - f.min()) / (f.max() - f.min())
        out[k] = 0.02 + 0.93 * f
    return out.reshape(n_classes, size * size)


def _bernoulli_images(rng, templates, n):
    y = rng.integers(0, templates.shape[0], n)
    X = (rng.random((n, templates.shape[1])) < templates[y]).astype(np.uint32)
    return X, y.astype(np.uint32)


def _mnist_shaped(rng, n_train, n_test):
    t = _templates(rng)
    X, y = _bernoulli_images(rng, t, n_train)
    Xt, yt = _bernoulli_images(rng, t, n_test)
    return X, y, Xt, yt


def _cifar_images(rng, means, labels):
    """uint8 images (n, 32, 32, 3) of the given classes: the class's colour field plus noise."""
    n = labels.shape[0]
    return np.clip(means[labels] + rng.normal(0.0, 32.0, (n, 32, 32, 3)), 0, 255).astype(np.uint8)


def _cifar_rows(rng, means, labels):
    # thermometer j = 0..7: x >= (j+1)*255/9, layout [y][x][channel*8 + j]
    # (the closed form of src/tm_utils/binarizer.py:11,19)
    img = _cifar_images(rng, means, labels)
    thr = (np.arange(1, 9) * 255.0 / 9.0)
    return (img[..., None] >= thr).reshape(labels.shape[0], 32 * 32 * 24).astype(np.uint32)  # (n, 32, 32, 3, 8)


def _cifar_set(rng, means, n, chunk=1024):
    # The noise is drawn chunk by chunk, which gives the same values as one draw of the whole
    # (n, 32, 32, 3) array while the temporaries stay in cache.
    y = rng.integers(0, means.shape[0], n)
    X = np.empty((n, 32 * 32 * 24), dtype=np.uint32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        X[s:e] = _cifar_rows(rng, means, y[s:e])
    return X, y.astype(np.uint32)


def _cifar_means(rng):
    from scipy.ndimage import gaussian_filter

    means = np.empty((10, 32, 32, 3))
    for k in range(10):
        for ch in range(3):
            f = gaussian_filter(rng.standard_normal((32, 32)), 4.0)
            means[k, :, :, ch] = 255.0 * (f - f.min()) / (f.max() - f.min())
    return means


def _cifar_shaped(rng, n_train, n_test):
    means = _cifar_means(rng)
    X, y = _cifar_set(rng, means, n_train)
    Xt, yt = _cifar_set(rng, means, n_test)
    return X, y, Xt, yt


class CifarStream:
    """Configuration 4's samples (the values of make(4, n_train, n_test)) generated on demand
    in consecutive row ranges, training rows first, then test rows, so that the 4.9 GB of
    raw uint32 training inputs never exist at once.  Labels: .y now, .yt once the test rows
    are started."""

    def __init__(self, n_train, n_test, seed=None):
        self._rng = np.random.default_rng(DATA_SEED + 4 if seed is None else seed)
        self._means = _cifar_means(self._rng)
        self.n_train, self.n_test = n_train, n_test
        self._y = self._rng.integers(0, 10, n_train)
        self.y = self._y.astype(np.uint32)
        self._yt = None
        self.yt = None
        self._pos = 0  # rows generated so far (training, then test)

    def train_rows(self, s, e):
        assert s == self._pos and e <= self.n_train, "rows must be generated in order"
        self._pos = e
        return _cifar_rows(self._rng, self._means, self._y[s:e])

    def test_rows(self, s, e):
        self._start_test(s)
        self._pos = self.n_train + e
        return _cifar_rows(self._rng, self._means, self._yt[s:e])

    def train_images(self, s, e):
        """The uint8 images (e - s, 32, 32, 3) behind train_rows(s, e): their rows are
        ThermometerBinarizer(8).binarize_rgb of these, flattened."""
        assert s == self._pos and e <= self.n_train, "rows must be generated in order"
        self._pos = e
        return _cifar_images(self._rng, self._means, self._y[s:e])

    def test_images(self, s, e):
        self._start_test(s)
        self._pos = self.n_train + e
        return _cifar_images(self._rng, self._means, self._yt[s:e])

    def _start_test(self, s):
        if self._yt is None:
            assert self._pos == self.n_train, "the training rows come first"
            self._yt = self._rng.integers(0, 10, self.n_test)
            self.yt = self._yt.astype(np.uint32)
        assert s == self._pos - self.n_train, "rows must be generated in order"


def _docs(rng, probs, n, length=150):
    V = probs.shape[1]
    y = rng.integers(0, probs.shape[0], n)
    X = np.zeros((n, V), dtype=np.uint32)
    cdf = np.cumsum(probs, axis=1)
    for k in range(probs.shape[0]):
        idx = np.nonzero(y == k)[0]
        draws = np.searchsorted(cdf[k], rng.random((idx.size, length)))
        draws = np.minimum(draws, V - 1)
        X[idx[:, None], draws] = 1
    return X, y.astype(np.uint32)


def _text_bow(rng, n_train, n_test, V=10000):
    base = np.arange(1, V + 1, dtype=np.float64) ** -1.1
    perm = rng.permutation(V)
    probs = np.empty((2, V))
    for k in range(2):
        p = base.copy()
        p[perm[200 * k:200 * (k + 1)]] *= 3.0
        probs[k] = p / p.sum()
    X, y = _docs(rng, probs, n_train)
    Xt, yt = _docs(rng, probs, n_test)
    return X, y, Xt, yt


_GEN = {1: _noisy_xor, 2: _mnist_shaped, 3: _mnist_shaped, 4: _cifar_shaped, 5: _text_bow}


def make(cfg: int, n_train: int | None = None, n_test: int | None = None, seed: int | None = None):
    """(X_train, y_train, X_test, y_test, model_kwargs) of configuration cfg (1..5)."""
    c = CONFIGS[cfg]
    n_train = c["n_train"] if n_train is None else n_train
    n_test = c["n_test"] if n_test is None else n_test
    rng = np.random.default_rng(DATA_SEED + cfg if seed is None else seed)
    X, y, Xt, yt = _GEN[cfg](rng, n_train, n_test)
    return X, y, Xt, yt, dict(c["model"])
