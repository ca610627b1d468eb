"""ytm_score_dataset_noalloc (the allocation-free scorer) against ytm_score_dataset and the
C oracle.

Both are called through the C-ABI on the same model and device-resident dataset; the
allocation-free one writes into a caller-owned device buffer, and the oracle, loaded with
the GPU model's state, scores the same samples.  Two calls in a row, the
second on fewer samples, so a stale scratch array from the first call would show.  Every
scoring kernel path is covered: wide one-patch clauses (literal lists), several patches
(literal-major samples), narrow one-patch clauses (per-chunk sums, several passes over the
scratch), and the plain scorer (more classes than the tiled scorers hold).
"""
import ctypes

import numpy as np
import pytest

import workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ytm_amd = pytest.importorskip("ytm_amd")
from ytm_amd import MultiClassTM  # noqa: E402
from ytm_amd._lib import check, lib, ptr  # noqa: E402

_hip = ctypes.CDLL("libamdhip64.so")
_hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
_hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
_hip.hipFree.argtypes = [ctypes.c_void_p]
_D2H = 2


def score_both(tm, data, n_classes):
    """(ytm_score_dataset, ytm_score_dataset_noalloc) class sums of one device dataset."""
    n = data.n
    ref = np.empty((n, n_classes), dtype=np.float32)
    check(lib.ytm_score_dataset(tm._handle, data.handle, ptr(ref)))
    d_out = ctypes.c_void_p()
    nbytes = max(4, n * n_classes * 4)
    assert _hip.hipMalloc(ctypes.byref(d_out), nbytes) == 0
    try:
        check(lib.ytm_score_dataset_noalloc(tm._handle, data.handle, d_out))
        got = np.empty((n, n_classes), dtype=np.float32)
        assert _hip.hipMemcpy(got.ctypes.data, d_out, n * n_classes * 4, _D2H) == 0
    finally:
        _hip.hipFree(d_out)
    return ref, got


def random_state(tm, rng, include_p):
    C, L, K = tm.number_of_clauses, tm.number_of_literals, tm.number_of_outputs
    inc = rng.random((C, L)) < include_p
    ta = np.where(inc, 200, 60).astype(np.uint32)
    w = rng.integers(-30, 31, (C, K)).astype(np.float32)
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w,
                                  "patch_weights": np.zeros((C, tm.number_of_patches), np.int32),
                                  "min_y": None, "max_y": None}})


@pytest.mark.parametrize("case", ["wide_one_patch", "several_patches", "narrow_one_patch_passes", "plain"])
def test_noalloc_matches_score_dataset(case):
    print(f"[noalloc] case {case}", flush=True)
    rng = np.random.default_rng(23)
    if case == "wide_one_patch":  # config 2: 49-word clauses
        X, y, Xt, _, kw = workloads.make(2, 300, 3000)
        tm = MultiClassTM(**kw, seed=7)
        tm.fit(X, y)
        sizes = (3000, 700)
    elif case == "several_patches":  # config 3 geometry, 300 clauses
        X, y, Xt, _, kw = workloads.make(3, 60, 300)
        kw["number_of_clauses_per_class"] = 300
        tm = MultiClassTM(**kw, seed=7)
        tm.fit(X, y)
        sizes = (300, 100)
    elif case == "narrow_one_patch_passes":  # 7-word clauses, 2000 clauses: three passes
        kw = dict(number_of_clauses_per_class=2000, T=50, s=5.0, dim=(100, 1, 1), n_classes=10, seed=7)
        tm = MultiClassTM(**kw)
        random_state(tm, rng, 4.0 / tm.number_of_literals)
        Xt = (rng.random((45000, 100)) < 0.5).astype(np.uint32)
        sizes = (45000, 5000)
    else:  # 20 classes: the plain scorer
        kw = dict(number_of_clauses_per_class=300, T=50, s=5.0, dim=(40, 1, 1), n_classes=20, seed=7)
        tm = MultiClassTM(**kw)
        random_state(tm, rng, 3.0 / tm.number_of_literals)
        Xt = (rng.random((500, 40)) < 0.5).astype(np.uint32)
        sizes = (500, 120)
    encXt = tm.encode(Xt)
    okw = dict(kw)
    okw.pop("seed", None)
    oracle = orc.OracleTM(okw.pop("number_of_clauses_per_class"), okw.pop("T"), okw.pop("s"), okw.pop("dim"),
                          okw.pop("n_classes"), **okw)
    oracle.load_state(tm.get_ta_state(), tm.get_weights(), tm.get_patch_weights(), tm.stats()["step"])
    for n in sizes:
        data = tm.device_data(encXt[:n], is_X_encoded=True)
        ref, got = score_both(tm, data, tm.number_of_outputs)
        data.release()
        np.testing.assert_array_equal(got, ref, err_msg=f"{case} n={n}")
        assert np.any(ref != 0), "a meaningful comparison needs non-zero class sums"
        np.testing.assert_array_equal(got, oracle.score(encXt[:n]), err_msg=f"{case} n={n}: oracle")
    tm.release()


def test_noalloc_rejects_models_beyond_its_scratch():
    """Literal lists of 66000 wide one-patch clauses (34 MB) exceed the 32 MiB scratch: a clear
    error, no kernel launched."""
    tm = MultiClassTM(number_of_clauses_per_class=66000, T=50, s=5.0, dim=(600, 1, 1), n_classes=2, seed=1)
    X = np.zeros((4, 600), dtype=np.uint32)
    data = tm.device_data(tm.encode(X), is_X_encoded=True)
    d_out = ctypes.c_void_p(0)
    assert _hip.hipMalloc(ctypes.byref(d_out), 4 * 2 * 4) == 0
    try:
        with pytest.raises(ValueError, match="too large for the allocation-free scorer"):
            check(lib.ytm_score_dataset_noalloc(tm._handle, data.handle, d_out))
    finally:
        _hip.hipFree(d_out)
    data.release()
    tm.release()
