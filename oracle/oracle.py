"""ctypes wrapper of the C oracle (liboracle.so built from oracle/ytm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker / CPU baseline, never as the product path.

OracleTM keeps the reference's own state layout on the host (uint32 TA states (C, L),
float32 weights (C, K), int32 patch weights (C, P)) and restates the reference's
hyperparameter resolution (src/cutm/base.py:60-121,129-152) independently of ytm_amd.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


class OrcParams(ctypes.Structure):
    _fields_ = [
        ("clauses", ctypes.c_int32),
        ("classes", ctypes.c_int32),
        ("dim0", ctypes.c_int32),
        ("dim1", ctypes.c_int32),
        ("dim2", ctypes.c_int32),
        ("patch_dim0", ctypes.c_int32),
        ("patch_dim1", ctypes.c_int32),
        ("number_of_ta_states", ctypes.c_int32),
        ("max_included_literals", ctypes.c_int32),
        ("append_negated", ctypes.c_int32),
        ("encode_loc", ctypes.c_int32),
        ("coalesced", ctypes.c_int32),
        ("negative_polarity", ctypes.c_int32),
        ("init_neg_weights", ctypes.c_int32),
        ("thresh", ctypes.c_int32),
        ("s_inv", ctypes.c_double),
        ("q_prob", ctypes.c_double),
        ("seed", ctypes.c_uint64),
    ]


_P = ctypes.c_void_p
_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        sig = {
            "orc_geometry": (None, [ctypes.POINTER(OrcParams), _P]),
            "orc_set_threads": (None, [ctypes.c_int]),
            "orc_philox4x32_10": (None, [_P, _P, _P]),
            "orc_uniform_from_word": (ctypes.c_float, [ctypes.c_uint32]),
            "orc_u_lit": (ctypes.c_float, [ctypes.POINTER(OrcParams), ctypes.c_uint64, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_int64]),
            "orc_init_weights": (None, [ctypes.POINTER(OrcParams), _P]),
            "orc_encode": (None, [ctypes.POINTER(OrcParams), _P, ctypes.c_int64, _P]),
            "orc_score": (None, [ctypes.POINTER(OrcParams), _P, _P, _P, _P, ctypes.c_int64, _P]),
            "orc_transform": (None, [ctypes.POINTER(OrcParams), _P, _P, ctypes.c_int64, ctypes.c_int, _P]),
            "orc_fit": (None, [ctypes.POINTER(OrcParams), _P, _P, _P, _P, _P, _P, ctypes.c_int64, _P,
                               ctypes.c_uint64, _P, _P, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def set_threads(n: int) -> None:
    load().orc_set_threads(int(n))


def _addr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    load().orc_philox4x32_10(_addr(c), _addr(k), _addr(out))
    return out


def uniform_from_word(z: int) -> float:
    return float(load().orc_uniform_from_word(ctypes.c_uint32(z)))


# ---------------------------------------------------------------- constant typing
def _is_int(v) -> bool:
    return isinstance(v, (int, np.integer)) and not isinstance(v, (bool, np.bool_))


def s_inv_of(s) -> float:
    """`#define S {s}` then S_INV = (1.0f / S): float maths for an int literal, double
    maths for a floating literal (src/cutm/base.py:132, kernel.cu:31)."""
    if _is_int(s) or isinstance(s, (bool, np.bool_)):
        return float(np.float32(1.0) / np.float32(int(s)))
    return 1.0 / float(str(s))


def q_prob_of(q, K: int) -> float:
    """`#define Q {q}` then Q_PROB = (1.0f * Q / max(1, CLASSES - 1)) (kernel.cu:32)."""
    d = max(1, K - 1)
    if _is_int(q):
        return float(np.float32(np.float32(1.0) * np.float32(q)) / np.float32(d))
    return float(str(q)) / d


class OracleTM:
    """CPU model with the reference's semantics and the build's canonical random stream."""

    def __init__(self, number_of_clauses_per_class, T, s, dim, n_classes, *, q=1.0, patch_dim=None,
                 number_of_ta_states=256, max_included_literals=None, append_negated=True,
                 init_neg_weights=True, negative_polarity=True, encode_loc=True, coalesced=True,
                 seed=0, **_ignored):
        self.lib = load()
        patch_dim = patch_dim if patch_dim is not None else (dim[0], dim[1])
        K = n_classes
        banks = 1 if coalesced else K
        C = banks * number_of_clauses_per_class
        p = OrcParams()
        p.clauses = C
        p.classes = K
        p.dim0, p.dim1, p.dim2 = dim
        p.patch_dim0, p.patch_dim1 = patch_dim
        p.number_of_ta_states = number_of_ta_states
        p.append_negated = int(append_negated)
        p.encode_loc = int(encode_loc)
        p.coalesced = int(coalesced)
        p.negative_polarity = int(negative_polarity)
        p.init_neg_weights = int(init_neg_weights)
        p.thresh = int(T)
        p.s_inv = s_inv_of(s)
        p.q_prob = q_prob_of(min(q, float(K)), K)
        p.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        geo = np.zeros(4, dtype=np.int64)
        p.max_included_literals = 0
        self.lib.orc_geometry(ctypes.byref(p), _addr(geo))
        self.L, self.W, self.P, self.Lh = (int(v) for v in geo)
        p.max_included_literals = self.L if max_included_literals is None else int(max_included_literals)
        self.p = p
        self.C, self.K, self.T = C, K, int(T)
        self.number_of_ta_states = number_of_ta_states
        self.step = 0
        self.ta = np.full((C, self.L), number_of_ta_states // 2, dtype=np.uint32)
        self.w = np.zeros((C, K), dtype=np.float32)
        self.lib.orc_init_weights(ctypes.byref(p), _addr(self.w))
        self.pw = np.zeros((C, self.P), dtype=np.int32)
        self.bias = np.zeros(K, dtype=np.float32)
        self.updates = 0
        self.last_feedback_samples = 0

    def load_state(self, ta, w, pw, step: int) -> None:
        """Continue from another model's state: TA states (C, L), weights (C, K), patch
        weights (C, P) and the step of the random stream (samples trained so far)."""
        self.ta[...] = np.asarray(ta, dtype=np.uint32).reshape(self.ta.shape)
        self.w[...] = np.asarray(w, dtype=np.float32).reshape(self.w.shape)
        self.pw[...] = np.asarray(pw, dtype=np.int32).reshape(self.pw.shape)
        self.step = int(step)

    def encode(self, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.uint32)
        out = np.zeros((X.shape[0], self.P, self.W), dtype=np.uint32)
        self.lib.orc_encode(ctypes.byref(self.p), _addr(X), X.shape[0], _addr(out))
        return out

    def fit_encoded(self, encX: np.ndarray, encY: np.ndarray, drop: np.ndarray | None = None,
                    inject: np.ndarray | None = None) -> int:
        encX = np.ascontiguousarray(encX, dtype=np.uint32)
        encY = np.ascontiguousarray(encY, dtype=np.int32)
        N = encX.shape[0]
        drop = np.zeros(self.C, dtype=np.uint32) if drop is None else np.ascontiguousarray(drop, dtype=np.uint32)
        if inject is not None:
            inject = np.ascontiguousarray(inject, dtype=np.float32)
            assert inject.size == N * (self.C * self.P + 2 * self.C * self.K + self.C * self.K * self.L)
        upd = np.zeros(1, dtype=np.uint64)
        fb = np.zeros(1, dtype=np.uint64)
        self.lib.orc_fit(ctypes.byref(self.p), _addr(self.ta), _addr(self.w), _addr(self.pw), _addr(self.bias),
                         _addr(encX), _addr(encY), N, _addr(drop), ctypes.c_uint64(self.step), _addr(inject),
                         _addr(upd), _addr(fb))
        self.step += N
        self.updates += int(upd[0])
        # samples of this call at which some class had an update probability above zero
        self.last_feedback_samples = int(fb[0])
        return int(upd[0])

    def encode_y_multiclass(self, Y: np.ndarray) -> np.ndarray:
        out = np.empty((Y.shape[0], self.K), dtype=np.int32)
        for i in range(self.K):
            out[:, i] = np.where(Y == i, self.T, -self.T)
        return out

    def score(self, encX: np.ndarray) -> np.ndarray:
        encX = np.ascontiguousarray(encX, dtype=np.uint32)
        out = np.zeros((encX.shape[0], self.K), dtype=np.float32)
        self.lib.orc_score(ctypes.byref(self.p), _addr(self.ta), _addr(self.w), _addr(self.bias), _addr(encX),
                           encX.shape[0], _addr(out))
        return out

    def transform(self, encX: np.ndarray, patchwise: bool = False) -> np.ndarray:
        encX = np.ascontiguousarray(encX, dtype=np.uint32)
        N = encX.shape[0]
        shape = (N, self.C, self.P) if patchwise else (N, self.C)
        out = np.zeros(shape, dtype=np.uint32)
        self.lib.orc_transform(ctypes.byref(self.p), _addr(self.ta), _addr(encX), N, int(patchwise), _addr(out))
        return out

    def u_lit(self, t: int, c: int, k: int, l: int) -> float:
        return float(self.lib.orc_u_lit(ctypes.byref(self.p), t, c, k, l))


def default_threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", "1"))
