"""ctypes binding of libytm.so, the C-ABI declared in include/ytm.h.

The HIP library is the only compute path: importing this module fails loudly when the
library has not been built (``python -c "import __graft_entry__ as g; g.build()"``).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("YTM_LIB", _HERE / "libytm.so"))

YTM_OK, YTM_EINVAL, YTM_EHIP, YTM_ETIMEOUT, YTM_ERANGE = range(5)


class YtmParams(ctypes.Structure):
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


class YtmStats(ctypes.Structure):
    _fields_ = [
        ("step", ctypes.c_uint64),
        ("last_fit_samples", ctypes.c_uint64),
        ("last_fit_updates", ctypes.c_uint64),
        ("total_updates", ctypes.c_uint64),
        ("last_fit_kernel_ms", ctypes.c_double),
        ("last_fit_launches", ctypes.c_int32),
        ("train_workgroups", ctypes.c_int32),
        ("last_score_kernel_ms", ctypes.c_double),
        ("last_encode_kernel_ms", ctypes.c_double),
        ("last_fit_wait_frac", ctypes.c_double),
        ("train_kind", ctypes.c_int32),
        ("train_specialised", ctypes.c_int32),
        ("last_fit_phase_us", ctypes.c_double * 8),
        ("last_fit_feedback_samples", ctypes.c_uint64),
        ("last_fit_evaluations", ctypes.c_uint64),
        ("last_fit_stream", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("last_fit_draws", ctypes.c_uint64 * 3),
    ]


# Every exported entry point of include/ytm.h with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
SIGNATURES = {
    "ytm_last_error": (ctypes.c_char_p, []),
    "ytm_shutdown": (ctypes.c_int, []),
    "ytm_create": (ctypes.c_int, [ctypes.POINTER(YtmParams), ctypes.POINTER(_P)]),
    "ytm_destroy": (None, [_P]),
    "ytm_geometry": (ctypes.c_int, [_P, _P]),
    "ytm_get_stats": (ctypes.c_int, [_P, ctypes.POINTER(YtmStats)]),
    "ytm_set_seed": (ctypes.c_int, [_P, ctypes.c_uint64]),
    "ytm_compile_train_kernel": (ctypes.c_int, [ctypes.POINTER(YtmParams), ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "ytm_load_train_kernels": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
    "ytm_encode": (ctypes.c_int, [_P, _P, _I64, _P]),
    "ytm_encode_binarized": (ctypes.c_int, [_P, _P, ctypes.c_int, _I64, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _P]),
    "ytm_dataset_create": (ctypes.c_int, [_P, _P, _P, _I64, ctypes.POINTER(_P)]),
    "ytm_dataset_destroy": (None, [_P]),
    "ytm_fit_dataset": (ctypes.c_int, [_P, _P, _I64, _I64, _P, _P]),
    "ytm_fit": (ctypes.c_int, [_P, _P, _P, _I64, _P, _P]),
    "ytm_score_dataset": (ctypes.c_int, [_P, _P, _P]),
    "ytm_score_dataset_noalloc": (ctypes.c_int, [_P, _P, _P]),
    "ytm_score": (ctypes.c_int, [_P, _P, _I64, _P]),
    "ytm_transform": (ctypes.c_int, [_P, _P, _I64, ctypes.c_int, _P]),
    "ytm_get_ta_state": (ctypes.c_int, [_P, _P]),
    "ytm_set_ta_state": (ctypes.c_int, [_P, _P]),
    "ytm_get_weights": (ctypes.c_int, [_P, _P]),
    "ytm_set_weights": (ctypes.c_int, [_P, _P]),
    "ytm_get_patch_weights": (ctypes.c_int, [_P, _P]),
    "ytm_set_patch_weights": (ctypes.c_int, [_P, _P]),
    "ytm_get_bias": (ctypes.c_int, [_P, _P]),
    "ytm_binarize": (ctypes.c_int, [_P, ctypes.c_int, _I64, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    _P]),
    "ytm_collapse_bins": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_int, ctypes.c_int, _P]),
}

# Element types of ytm_binarize (YTM_DTYPE_* of include/ytm.h).
DTYPES = {"uint8": 0, "int8": 1, "uint16": 2, "int16": 3, "uint32": 4, "int32": 5, "int64": 6, "float32": 7,
          "float64": 8}


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"libytm.so not found at {LIB_PATH}; build the HIP extension first "
            "(python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = _load()


class YtmError(RuntimeError):
    """A failure reported by libytm (HIP error, timeout, invalid argument)."""


def check(rc: int) -> None:
    if rc != YTM_OK:
        msg = lib.ytm_last_error().decode(errors="replace")
        if rc in (YTM_EINVAL, YTM_ERANGE):
            raise ValueError(msg)
        raise YtmError(msg)


def ptr(a: np.ndarray | None) -> int | None:
    """Address of a C-contiguous numpy array (None for NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data
