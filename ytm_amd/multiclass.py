"""MultiClassTM: drop-in counterpart of cutm.MultiClassTM (src/cutm/multiclass.py:6-59)."""
from __future__ import annotations

from typing import Any

import numpy as np

from .base import BaseTM


class MultiClassTM(BaseTM):
    def __init__(self, number_of_clauses_per_class: int, T: int, s: float, dim: tuple[int, int, int],
                 n_classes: int, **opt_args: Any):
        super().__init__(
            number_of_clauses_per_class=number_of_clauses_per_class,
            T=T,
            s=s,
            dim=dim,
            n_classes=n_classes,
            **opt_args,
        )

    def fit(self, X: np.ndarray, Y: np.ndarray, is_X_encoded: bool = False, **opt_args: Any) -> None:
        assert Y.ndim == 1, "Y must be 1D array (samples,)"
        assert X.shape[0] == Y.shape[0], "X and Y must have the same number of samples."
        # One-vs-rest targets +-T (multiclass.py:35-37).
        encoded_Y = np.empty((Y.shape[0], self.number_of_outputs), dtype=np.int32)
        for i in range(self.number_of_outputs):
            encoded_Y[:, i] = np.where(Y == i, self.T, -self.T)
        encoded_X = self.encode(X) if not is_X_encoded else X
        self._fit(encoded_X, encoded_Y, **opt_args)

    def device_data(self, X: np.ndarray, Y: np.ndarray | None = None, is_X_encoded: bool = False):
        """Copy (encoded) samples and their one-vs-rest targets into HBM once, for
        fit_device / score_device epochs that do not re-copy the data."""
        encoded_X = self.encode(X) if not is_X_encoded else X
        encoded_Y = None
        if Y is not None:
            encoded_Y = np.empty((Y.shape[0], self.number_of_outputs), dtype=np.int32)
            for i in range(self.number_of_outputs):
                encoded_Y[:, i] = np.where(Y == i, self.T, -self.T)
        return self._device_data(encoded_X, encoded_Y)

    def score(self, X: np.ndarray, is_X_encoded: bool, block_size: int | None = None) -> np.ndarray:
        encoded_X = self.encode(X) if not is_X_encoded else X
        return self._score_batch(encoded_X, block_size=block_size)

    def predict(self, X: np.ndarray, is_X_encoded: bool = False, block_size: int | None = None):
        class_sums = self.score(X, is_X_encoded, block_size=block_size)
        preds = np.argmax(class_sums, axis=1)  # first maximum on ties (multiclass.py:58)
        return preds, class_sums
