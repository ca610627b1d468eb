"""BaseTM: drop-in counterpart of cutm.base.BaseTM (src/cutm/base.py:41-593).

Same constructor arguments, public attributes, methods, return dtypes/shapes, assertion
and OverflowError behaviour and pickle dictionary as the reference.  The compute runs in
libytm.so (hand-written HIP kernels for gfx950) through the C-ABI of include/ytm.h;
there is no CPU fallback.

Deliberate differences, each raised as an error rather than silently diverging:
  * ``bias=True`` (documented "Does not work" in the reference, base.py:27, and racy in
    kernel.cu:593,601) raises NotImplementedError;
  * T must be integer-valued (the reference types it ``int``);
  * loaded clause weights must be integer-valued (what the reference itself produces);
  * encode() checks that X has dim0*dim1*dim2 columns (the reference would read past
    the end of X).
Randomness: the reference's cuRAND XORWOW streams depend on the launch grid and cannot
be reproduced; this model draws from a counter-based Philox4x32-10 stream keyed by the
seed, or from an injected buffer passed as ``fit(..., random_stream=...)``.
"""
from __future__ import annotations

import atexit
import ctypes
import sys
import weakref
from typing import Any

import numpy as np

from . import _lib
from ._lib import check, lib, ptr

_OPT_DEFAULTS = (
    ("q", 1.0),
    ("patch_dim", None),
    ("number_of_ta_states", 256),
    ("max_included_literals", None),
    ("append_negated", True),
    ("init_neg_weights", True),
    ("negative_polarity", True),
    ("encode_loc", True),
    ("coalesced", True),
    ("h", 1.0),
    ("bias", False),
    ("seed", None),
    ("block_size", 128),
)


def _is_int(v: Any) -> bool:
    return isinstance(v, (int, np.integer)) and not isinstance(v, (bool, np.bool_))


def typed_s_inv(s: Any) -> float:
    """S_INV = (1.0f / S) with S pasted as ``str(s)`` (base.py:132; kernel.cu:31):
    float arithmetic for an integer s, double arithmetic for a floating-point s."""
    if isinstance(s, (bool, np.bool_)):
        s = int(s)
    if _is_int(s):
        return float(np.float32(1.0) / np.float32(s))
    return 1.0 / float(str(s))


def typed_q_prob(q: Any, n_classes: int) -> float:
    """Q_PROB = (1.0f * Q / max(1, CLASSES - 1)) with Q pasted as ``str(q)`` (base.py:133;
    kernel.cu:32)."""
    d = max(1, n_classes - 1)
    if _is_int(q):
        return float(np.float32(np.float32(1.0) * np.float32(q)) / np.float32(d))
    return (1.0 * float(str(q))) / d


# Live models and datasets, released in that order (datasets first) by shutdown().
_live_data: "weakref.WeakSet[DeviceData]" = weakref.WeakSet()
_live_models: "weakref.WeakSet[BaseTM]" = weakref.WeakSet()


def shutdown() -> None:
    """Frees every live dataset and model (they are unusable afterwards), then unloads the
    training kernels compiled at run time (ytm_shutdown).  Registered with atexit, so the
    device memory, streams, events, pinned buffers and kernel modules of the library are
    all released while the interpreter and the HIP runtime are still whole, not left to the
    runtime's own exit handlers."""
    for d in list(_live_data):
        d.release()
    for m in list(_live_models):
        m.release()
    check(lib.ytm_shutdown())


def _shutdown_at_exit() -> None:
    try:
        shutdown()
    except Exception as exc:  # an exit handler must not raise; report and go on
        print(f"ytm_amd: teardown at exit failed: {exc}", file=sys.stderr)


atexit.register(_shutdown_at_exit)


class DeviceData:
    """Encoded samples (and encoded targets) copied once into HBM and owned by libytm."""

    def __init__(self, tm: "BaseTM", encoded_X: np.ndarray, encoded_Y: np.ndarray | None):
        self.n = int(encoded_X.shape[0])
        self._tm = tm  # keeps the model alive while the data exists
        handle = ctypes.c_void_p()
        check(lib.ytm_dataset_create(tm._handle, ptr(encoded_X), ptr(encoded_Y), self.n, ctypes.byref(handle)))
        self.handle = handle
        _live_data.add(self)

    def release(self) -> None:
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            lib.ytm_dataset_destroy(handle)
        self.handle = None

    def __del__(self):
        # shutdown() has released everything still alive before the interpreter finalizes
        if not sys.is_finalizing():
            self.release()


class BaseTM:
    def __init__(self, number_of_clauses_per_class: int, T: int, s: float, dim: tuple[int, int, int],
                 n_classes: int, **opt_args: Any):
        self.init_args = {
            "number_of_clauses_per_class": number_of_clauses_per_class,
            "T": T,
            "s": s,
            "dim": dim,
            "n_classes": n_classes,
        }
        defaults = dict(_OPT_DEFAULTS)
        defaults["patch_dim"] = (dim[0], dim[1])
        self.opt_args = {k: opt_args.get(k, v) for k, v in defaults.items()}

        self.number_of_clauses_per_class = number_of_clauses_per_class
        self.T = T
        self.s = s
        self.dim = dim
        self.number_of_outputs = n_classes
        self.q = min(self.opt_args["q"], float(self.number_of_outputs))
        self.patch_dim = self.opt_args["patch_dim"]
        self.number_of_ta_states = self.opt_args["number_of_ta_states"]
        self.max_included_literals = self.opt_args["max_included_literals"]
        self.append_negated = self.opt_args["append_negated"]
        self.init_neg_weights = self.opt_args["init_neg_weights"]
        self.negative_clauses = self.opt_args["negative_polarity"]
        self.encode_loc = self.opt_args["encode_loc"]
        self.coalesced = self.opt_args["coalesced"]
        self.bias = self.opt_args["bias"]
        self.seed = self.opt_args["seed"]
        self.block_size = self.opt_args["block_size"]

        self.number_of_clause_banks = 1 if self.coalesced else self.number_of_outputs
        self.number_of_clauses = self.number_of_clause_banks * self.number_of_clauses_per_class

        if isinstance(self.opt_args["h"], list):
            assert len(self.opt_args["h"]) == n_classes, "If h is a list, it must have length equal to n_classes."
            self.h = np.asarray(self.opt_args["h"], dtype=np.float64)
        else:
            self.h = np.asarray([self.opt_args["h"]] * n_classes, dtype=np.float64)

        if not hasattr(self, "min_y"):
            self.min_y = None
        if not hasattr(self, "max_y"):
            self.max_y = None

        if self.encode_loc:
            self.number_of_literals = int(
                self.patch_dim[0] * self.patch_dim[1] * self.dim[2]
                + (self.dim[0] - self.patch_dim[0])
                + (self.dim[1] - self.patch_dim[1])
            )
        else:
            self.number_of_literals = int(self.patch_dim[0] * self.patch_dim[1] * self.dim[2])
        if self.append_negated:
            self.number_of_literals *= 2
        self.number_of_literal_chunks = ((self.number_of_literals - 1) // 32) + 1
        self.number_of_patches = int((self.dim[0] - self.patch_dim[0] + 1) * (self.dim[1] - self.patch_dim[1] + 1))

        self.rng = np.random.default_rng(self.seed)
        self._gpu_init()

    # ------------------------------------------------------------------ device state
    def _params(self) -> _lib.YtmParams:
        if self.bias:
            raise NotImplementedError("bias=True is racy in the reference (kernel.cu:593,601) and is not supported")
        if float(self.T) != int(self.T):
            raise ValueError("T must be integer-valued")
        maxinc = self.number_of_literals if self.max_included_literals is None else self.max_included_literals
        if self.seed is None:
            key = int(np.random.SeedSequence().generate_state(1, np.uint64)[0])
        else:
            key = int(self.seed) & 0xFFFFFFFFFFFFFFFF
        p = _lib.YtmParams()
        p.clauses = self.number_of_clauses
        p.classes = self.number_of_outputs
        p.dim0, p.dim1, p.dim2 = (int(v) for v in self.dim)
        p.patch_dim0, p.patch_dim1 = (int(v) for v in self.patch_dim)
        p.number_of_ta_states = int(self.number_of_ta_states)
        p.max_included_literals = int(maxinc)
        p.append_negated = int(bool(self.append_negated))
        p.encode_loc = int(bool(self.encode_loc))
        p.coalesced = int(bool(self.coalesced))
        p.negative_polarity = int(bool(self.negative_clauses))
        p.init_neg_weights = int(bool(self.init_neg_weights))
        p.thresh = int(self.T)
        p.s_inv = typed_s_inv(self.s)
        p.q_prob = typed_q_prob(self.q, self.number_of_outputs)
        p.seed = key
        return p

    @classmethod
    def compile_kernels(cls, *args, injected: bool = False, compute_units: int = 0, **kwargs) -> list[int]:
        """Compile and cache, for this process, the training kernels specialised for a model
        built with these arguments, for a device with `compute_units` CUs (0: an MI355X's
        256); needs no GPU (the counterpart of the per-model compile in the reference's
        BaseTM.__init__, src/cutm/base.py:129-159).  Fitting compiles on first use anyway.
        Returns the training-kernel kinds compiled."""
        tm = cls.__new__(cls)
        tm._skip_gpu_init = True
        tm.__init__(*args, **kwargs)
        params = tm._params()
        if not tm.coalesced or tm.number_of_outputs > 64:
            return []  # clause banks and more than 64 classes: built-in kernels, a launch per sample (train_kind 4)
        P = tm.number_of_patches
        kinds = [0, 1] if P == 1 else ([0, 2] if (P + 31) // 32 <= 64 else [2])
        for kind in kinds:
            check(lib.ytm_compile_train_kernel(ctypes.byref(params), kind, int(bool(injected)), int(compute_units)))
        # the streaming kernel (one patch, counter stream), when the model fits its shape
        if P == 1 and not injected and lib.ytm_compile_train_kernel(ctypes.byref(params), 3, 0,
                                                                     int(compute_units)) == _lib.YTM_OK:
            kinds.append(3)
        return kinds

    def load_kernels(self) -> list[int]:
        """Compile (when not cached) and load onto this model's GPU every training kernel its
        fits may switch between, so that no fit pays for the load (about half a second the
        first time).  Returns the training-kernel kinds loaded (none for clause banks)."""
        kinds = (ctypes.c_int32 * 4)()
        n = ctypes.c_int32(0)
        check(lib.ytm_load_train_kernels(self._handle, kinds, ctypes.byref(n)))
        return list(kinds[:n.value])

    def _gpu_init(self) -> None:
        if getattr(self, "_skip_gpu_init", False):
            self._handle = None
            return
        self._params_c = self._params()
        handle = ctypes.c_void_p()
        check(lib.ytm_create(ctypes.byref(self._params_c), ctypes.byref(handle)))
        self._handle = handle
        _live_models.add(self)

    def release(self) -> None:
        """Free the model's device memory now (the object is unusable afterwards)."""
        handle = getattr(self, "_handle", None)
        if handle is not None and handle.value:
            lib.ytm_destroy(handle)
        self._handle = None

    def __del__(self):
        if not sys.is_finalizing():
            self.release()

    def stats(self) -> dict:
        """Counters and kernel timings of the most recent calls."""
        st = _lib.YtmStats()
        check(lib.ytm_get_stats(self._handle, ctypes.byref(st)))
        out = {name: getattr(st, name) for name, _ in st._fields_}
        out["last_fit_phase_us"] = list(out["last_fit_phase_us"])
        out["last_fit_draws"] = list(out["last_fit_draws"])
        return out

    # ------------------------------------------------------------------ encode
    def encode(self, X: np.ndarray, block_size: int | None = None) -> np.ndarray:
        assert X.ndim == 2, "X must be a 2D array (samples, dim0 * dim1 * dim2)."
        assert X.dtype == np.uint32, "X must be of type np.uint32."
        assert X.shape[1] == self.dim[0] * self.dim[1] * self.dim[2], "X must have dim0 * dim1 * dim2 columns."
        X = np.ascontiguousarray(X)
        N = X.shape[0]
        out = np.empty((N, self.number_of_patches, self.number_of_literal_chunks), dtype=np.uint32)
        check(lib.ytm_encode(self._handle, ptr(X), N, ptr(out)))
        return out

    def encode_binarized(self, X: np.ndarray, binarizer) -> np.ndarray:
        """encode() of the binarizer's output for X in one pass on the GPU, without the binned
        array: X holds N samples of raw values (any shape (N, ...)), binned by a
        ThermometerBinarizer or a fitted Binarizer (src/tm_utils/binarizer.py), whose levels
        of a value are consecutive in the binned row.  The result equals
        ``self.encode(binned.reshape(N, -1))`` where binned is binarize_gray / binarize_rgb /
        transform of X (not in the reference, which bins on the host: 1/width of the input
        bytes to move, and no binned array)."""
        from .binarizer import _device_levels, _dtype_code

        thresholds, kind, edge = binarizer._levels()
        Xd, t, int_thr, width = _device_levels(X, thresholds, kind, edge)
        assert Xd.ndim >= 2, "X must hold samples along its first axis."
        N = Xd.shape[0]
        F = self.dim[0] * self.dim[1] * self.dim[2]
        assert Xd[0].size * width == F, (
            f"X's samples bin to {Xd[0].size} x {width} values; the model takes dim0 * dim1 * dim2 = {F}.")
        out = np.empty((N, self.number_of_patches, self.number_of_literal_chunks), dtype=np.uint32)
        check(lib.ytm_encode_binarized(self._handle, ptr(Xd), _dtype_code(Xd), N, ptr(t), int(int_thr), t.size,
                                       kind, int(bool(edge)), ptr(out)))
        return out

    def _check_encoded(self, encoded_X: np.ndarray) -> np.ndarray:
        assert encoded_X.dtype == np.uint32, "encoded X must be of type np.uint32."
        assert encoded_X.shape[1:] == (self.number_of_patches, self.number_of_literal_chunks), (
            "encoded X must have shape (samples, number_of_patches, number_of_literal_chunks)."
        )
        return np.ascontiguousarray(encoded_X)

    # ------------------------------------------------------------------ fit / score
    def _drop_mask(self, clause_drop_p: float) -> np.ndarray:
        # base.py:288-293
        if clause_drop_p > 0.0:
            return (self.rng.random(self.number_of_clauses) <= clause_drop_p).astype(np.uint32)
        return np.zeros(self.number_of_clauses, dtype=np.uint32)

    def random_stream_size(self, n_samples: int) -> int:
        """Floats of an injected random stream for n_samples training samples."""
        C, K, P, L = self.number_of_clauses, self.number_of_outputs, self.number_of_patches, self.number_of_literals
        return n_samples * (C * P + 2 * C * K + C * K * L)

    def _fit(self, encoded_X, encoded_Y, **opt_args: Any) -> None:
        # block_size, true_mod, false_mod and norm_* are accepted like the reference; the
        # reference kernel never reads their values (kernel.cu:508-529,576-577).
        clause_drop_p = opt_args.get("clause_drop_p", 0.0)
        stream = opt_args.get("random_stream", None)
        encoded_X = self._check_encoded(encoded_X)
        encoded_Y = np.ascontiguousarray(encoded_Y, dtype=np.int32)
        N = encoded_X.shape[0]
        assert encoded_Y.shape == (N, self.number_of_outputs), "encoded Y must have shape (samples, n_outputs)."
        drop = self._drop_mask(clause_drop_p)
        if stream is not None:
            stream = np.ascontiguousarray(stream, dtype=np.float32)
            assert stream.size == self.random_stream_size(N), "random_stream has the wrong size."
        check(lib.ytm_fit(self._handle, ptr(encoded_X), ptr(encoded_Y), N, ptr(drop), ptr(stream)))

    # ------------------------------------------------------------------ HBM-resident data
    def _device_data(self, encoded_X, encoded_Y=None) -> "DeviceData":
        encoded_X = self._check_encoded(encoded_X)
        if encoded_Y is not None:
            encoded_Y = np.ascontiguousarray(encoded_Y, dtype=np.int32)
            assert encoded_Y.shape == (encoded_X.shape[0], self.number_of_outputs)
        return DeviceData(self, encoded_X, encoded_Y)

    def fit_device(self, data: "DeviceData", first: int = 0, count: int | None = None, **opt_args: Any) -> None:
        """_fit over samples [first, first+count) of data already resident in HBM."""
        count = data.n - first if count is None else count
        drop = self._drop_mask(opt_args.get("clause_drop_p", 0.0))
        check(lib.ytm_fit_dataset(self._handle, data.handle, first, count, ptr(drop), None))

    def score_device(self, data: "DeviceData") -> np.ndarray:
        class_sums = np.empty((data.n, self.number_of_outputs), dtype=np.float32)
        check(lib.ytm_score_dataset(self._handle, data.handle, ptr(class_sums)))
        return class_sums

    def _score_batch(self, encoded_X, block_size: int | None = None) -> np.ndarray:
        encoded_X = self._check_encoded(encoded_X)
        N = encoded_X.shape[0]
        class_sums = np.empty((N, self.number_of_outputs), dtype=np.float32)
        check(lib.ytm_score(self._handle, ptr(encoded_X), N, ptr(class_sums)))
        return class_sums

    # ------------------------------------------------------------------ state
    def _bank_shape(self, last: int) -> tuple[int, ...]:
        if self.coalesced:
            return (self.number_of_clauses, last)
        return (self.number_of_clause_banks, self.number_of_clauses_per_class, last)

    def get_ta_state(self) -> np.ndarray:
        ta = np.empty(self.number_of_clauses * self.number_of_literals, dtype=np.uint32)
        check(lib.ytm_get_ta_state(self._handle, ptr(ta)))
        return ta.reshape(self._bank_shape(self.number_of_literals))

    def get_literals(self) -> np.ndarray:
        return (self.get_ta_state() > (self.number_of_ta_states // 2)).astype(np.uint32)

    def get_weights(self) -> np.ndarray:
        w = np.empty(self.number_of_clauses * self.number_of_outputs, dtype=np.float32)
        check(lib.ytm_get_weights(self._handle, ptr(w)))
        return w.reshape(self._bank_shape(self.number_of_outputs))

    def get_patch_weights(self) -> np.ndarray:
        pw = np.empty(self.number_of_clauses * self.number_of_patches, dtype=np.int32)
        check(lib.ytm_get_patch_weights(self._handle, ptr(pw)))
        return pw.reshape(self._bank_shape(self.number_of_patches))

    def get_bias_weights(self) -> np.ndarray:
        b = np.empty(self.number_of_outputs, dtype=np.float32)
        check(lib.ytm_get_bias(self._handle, ptr(b)))
        return b

    # ------------------------------------------------------------------ transform
    def transform(self, X, is_X_encoded: bool = False, block_size: int | None = None) -> np.ndarray:
        encoded_X = X if is_X_encoded else self.encode(X)
        N = encoded_X.shape[0]
        max_safe_N = np.iinfo(np.uint32).max // self.number_of_clauses
        if N > max_safe_N:
            raise OverflowError(
                f"X has too many samples ({N}). Maximum of {max_safe_N} samples can be processed with current "
                "number_of_clauses. Call this method multiple times with smaller batches of X."
            )
        encoded_X = self._check_encoded(encoded_X)
        out = np.empty((N, self.number_of_clauses), dtype=np.uint32)
        check(lib.ytm_transform(self._handle, ptr(encoded_X), N, 0, ptr(out)))
        return out

    def transform_patchwise(self, X, is_X_encoded: bool = False, block_size: int | None = None,
                            packed: bool = False) -> np.ndarray:
        """Per-patch clause outputs (src/cutm/base.py:510-542): uint32 (N, clauses, patches).

        ``packed=True`` (not in the reference) returns the same values bit-packed, uint32
        (N, clauses, ceil(patches / 32)) with bit b of word j = patch 32j + b and zero bits
        beyond the last patch -- 1/32 of the memory.  ``np.unpackbits(out.view(np.uint8),
        axis=-1, bitorder="little")[..., :patches]`` recovers the unpacked array on a
        little-endian host.
        """
        encoded_X = X if is_X_encoded else self.encode(X)
        N = encoded_X.shape[0]
        P = self.number_of_patches
        per_clause = (P + 31) // 32 if packed else P
        max_safe_N = np.iinfo(np.uint32).max // (self.number_of_clauses * per_clause)
        if N > max_safe_N:
            raise OverflowError(
                f"X has too many samples ({N}). Maximum of {max_safe_N} samples can be processed with current "
                + ("number_of_clauses * ceil(number_of_patches / 32)" if packed
                   else "number_of_clauses * number_of_patches")
                + ". Call this method multiple times with smaller batches of X."
            )
        encoded_X = self._check_encoded(encoded_X)
        out = np.empty((N, self.number_of_clauses, per_clause), dtype=np.uint32)
        check(lib.ytm_transform(self._handle, ptr(encoded_X), N, 2 if packed else 1, ptr(out)))
        return out

    # ------------------------------------------------------------------ serialisation
    def __getstate__(self):
        args = {**self.init_args, **self.opt_args}
        return {"args": args, "state": self.get_state_dict()}

    def __setstate__(self, state):
        args = state["args"]
        self.__init__(**args)
        self.load_state_dict(state)

    def get_state_dict(self) -> dict:
        ta = np.empty(self.number_of_clauses * self.number_of_literals, dtype=np.uint32)
        w = np.empty(self.number_of_clauses * self.number_of_outputs, dtype=np.float32)
        pw = np.empty(self.number_of_clauses * self.number_of_patches, dtype=np.int32)
        check(lib.ytm_get_ta_state(self._handle, ptr(ta)))
        check(lib.ytm_get_weights(self._handle, ptr(w)))
        check(lib.ytm_get_patch_weights(self._handle, ptr(pw)))
        return {"ta_state": ta, "clause_weights": w, "patch_weights": pw, "min_y": self.min_y, "max_y": self.max_y}

    def load_state_dict(self, state) -> None:
        state_dict = state["state"]
        ta = np.ascontiguousarray(np.asarray(state_dict["ta_state"]).reshape(-1), dtype=np.uint32)
        w = np.ascontiguousarray(np.asarray(state_dict["clause_weights"]).reshape(-1), dtype=np.float32)
        pw = np.ascontiguousarray(np.asarray(state_dict["patch_weights"]).reshape(-1), dtype=np.int32)
        assert ta.size == self.number_of_clauses * self.number_of_literals, "ta_state has the wrong size."
        assert w.size == self.number_of_clauses * self.number_of_outputs, "clause_weights has the wrong size."
        assert pw.size == self.number_of_clauses * self.number_of_patches, "patch_weights has the wrong size."
        self.min_y = state_dict["min_y"]
        self.max_y = state_dict["max_y"]
        check(lib.ytm_set_ta_state(self._handle, ptr(ta)))
        check(lib.ytm_set_weights(self._handle, ptr(w)))
        check(lib.ytm_set_patch_weights(self._handle, ptr(pw)))
