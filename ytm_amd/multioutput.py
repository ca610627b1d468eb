"""MultiOutputTM: drop-in counterpart of cutm.MultiOutputTM (src/cutm/multioutput.py:6-57)."""
from __future__ import annotations

from typing import Any

import numpy as np

from .base import BaseTM


class MultiOutputTM(BaseTM):
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
        assert Y.ndim == 2, f"Y must be 2D array (samples, outputs), got {Y.ndim}D"
        assert X.shape[0] == Y.shape[0], "X and Y must have the same number of samples"
        encoded_Y = np.where(Y == 1, self.T, -self.T).astype(np.int32)  # multioutput.py:36
        encoded_X = self.encode(X) if not is_X_encoded else X
        self._fit(encoded_X, encoded_Y, **opt_args)

    def score(self, X: np.ndarray, is_X_encoded: bool, block_size: int | None = None) -> np.ndarray:
        encoded_X = X if is_X_encoded else self.encode(X)
        return self._score_batch(encoded_X, block_size=block_size)

    def predict(self, X: np.ndarray, is_X_encoded: bool = False, block_size: int | None = None):
        class_sums = self.score(X, is_X_encoded, block_size=block_size)
        preds = (class_sums >= 0).astype(np.uint32)  # multioutput.py:56
        return preds, class_sums
