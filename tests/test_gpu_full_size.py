"""HIP path against the C oracle at the BASELINE sizes, bit for bit.

Training parity at the real model sizes of all five configurations (full clause counts,
literal widths and patch counts), and inference over test sets at those sizes:
  * config 2: one full 60000-sample epoch (TA states, weights, patch weights, update
    count), then class sums and predictions on all 10000 test samples;
  * config 1: all 10 epochs on the full 5000-sample training set, then the 5000 test samples;
  * configs 3 / 4 / 5 at full clause count (8000 / 20000 / 10000): trained past the
    all-empty-clause regime, then class sums and clause outputs on 200 test samples.
    Configs 3 and 4 have more than 4096 clauses, so their scores and clause outputs go
    through the several-patch kernels' clause-chunk loop;
  * a config-3 geometry scored on 70000 samples, more blocks than one launch holds
    (the grid-stride loop past the 65536-block grid).
Reference semantics: src/cutm/base.py:266-420,465-542; src/cutm/cuda/kernel.cu:255-394.
"""
import os

import numpy as np
import pytest

import workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ytm_amd = pytest.importorskip("ytm_amd")
from ytm_amd import MultiClassTM  # noqa: E402

orc.set_threads(min(16, os.cpu_count() or 1))


@pytest.fixture(autouse=True)
def _specialised_kernels_required(monkeypatch):
    monkeypatch.setenv("YTM_JIT", "2")


def make_pair(cfg, n_train, n_test, **opts):
    X, y, Xt, yt, kw = workloads.make(cfg, n_train, n_test)
    kw.update(opts)
    kw["seed"] = workloads.MODEL_SEED
    print(f"[full] cfg={cfg} n_train={n_train} n_test={n_test} kw={kw}", flush=True)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(kw.pop("number_of_clauses_per_class"), kw.pop("T"), kw.pop("s"), kw.pop("dim"),
                       kw.pop("n_classes"), **kw)
    return tm, ref, X, y, Xt, yt


def assert_state_equal(tm, ref, where):
    np.testing.assert_array_equal(tm.get_ta_state().reshape(ref.ta.shape), ref.ta, err_msg=f"TA {where}")
    np.testing.assert_array_equal(tm.get_weights().reshape(ref.w.shape), ref.w, err_msg=f"weights {where}")
    np.testing.assert_array_equal(tm.get_patch_weights().reshape(ref.pw.shape), ref.pw, err_msg=f"pw {where}")


def train_both(tm, ref, encX, y, epochs, where):
    encY = ref.encode_y_multiclass(y)
    for epoch in range(epochs):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        print(f"[full] {where} epoch {epoch}: updates {upd} ({upd / len(y):.1f}/sample)", flush=True)
        assert tm.stats()["last_fit_updates"] == upd, f"update count {where} epoch {epoch}"
    assert_state_equal(tm, ref, where)


def check_scores(tm, ref, encXt, where):
    preds, cs = tm.predict(encXt, is_X_encoded=True)
    ref_cs = ref.score(encXt)
    np.testing.assert_array_equal(cs, ref_cs, err_msg=f"class sums {where}")
    np.testing.assert_array_equal(preds, np.argmax(ref_cs, axis=1), err_msg=f"predictions {where}")
    return preds


def test_config2_full_epoch_and_test_set():
    tm, ref, X, y, Xt, yt = make_pair(2, None, None)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX[:2000], ref.encode(X[:2000]))
    assert encX.shape == (60000, 1, 49)
    train_both(tm, ref, encX, y, 1, "config 2 full epoch")
    ta = tm.get_ta_state()
    assert ta.max() <= 256 + 10
    encXt = tm.encode(Xt)
    preds = check_scores(tm, ref, encXt, "config 2, 10000 test samples")
    print(f"[full] config 2 test accuracy after one epoch: {(preds == yt).mean():.4f}", flush=True)
    np.testing.assert_array_equal(tm.transform(encXt[:500], is_X_encoded=True), ref.transform(encXt[:500]))


def test_config1_ten_epochs():
    tm, ref, X, y, Xt, yt = make_pair(1, None, None)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX, ref.encode(X))
    train_both(tm, ref, encX, y, workloads.CONFIGS[1]["epochs"], "config 1, 10 epochs")
    preds = check_scores(tm, ref, tm.encode(Xt), "config 1, 5000 test samples")
    print(f"[full] config 1 test accuracy: {(preds == yt).mean():.4f}", flush=True)


@pytest.mark.parametrize("cfg,n_train", [(3, 300), (4, 40), (5, 100)])
def test_full_clause_count(cfg, n_train):
    """Full clause counts; trained long enough that the clauses are no longer all empty, so
    that the scores and clause outputs depend on included literals."""
    tm, ref, X, y, Xt, yt = make_pair(cfg, n_train, 200)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX[:8], ref.encode(X[:8]))
    train_both(tm, ref, encX, y, 1, f"config {cfg} full clause count")
    n_inc = (tm.get_ta_state() > tm.number_of_ta_states // 2).sum(axis=-1)
    assert (n_inc > 0).mean() > 0.5, "most clauses should include literals by now"
    encXt = tm.encode(Xt)
    np.testing.assert_array_equal(encXt, ref.encode(Xt))
    check_scores(tm, ref, encXt, f"config {cfg}, 200 test samples")
    np.testing.assert_array_equal(tm.transform(encXt, is_X_encoded=True), ref.transform(encXt),
                                  err_msg=f"transform config {cfg}")
    pw = tm.transform_patchwise(encXt[:4], is_X_encoded=True, packed=True)
    ref_pw = ref.transform(encXt[:4], patchwise=True)
    P = ref_pw.shape[2]
    bits = np.unpackbits(np.ascontiguousarray(pw).view(np.uint8), axis=-1, bitorder="little")
    np.testing.assert_array_equal(bits[..., :P], ref_pw, err_msg=f"packed transform_patchwise config {cfg}")


def test_score_beyond_one_launch_grid(monkeypatch):
    """Config-3 geometry (several patches) with 16 clauses scored on 70000 samples: one
    block per sample, so the launch is clamped to 65536 blocks and the blocks loop."""
    X, y, Xt, yt, kw = workloads.make(3, 70000, 0)
    kw.update(number_of_clauses_per_class=16, seed=3)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(16, kw["T"], kw["s"], kw["dim"], kw["n_classes"], patch_dim=kw["patch_dim"], seed=3)
    rng = np.random.default_rng(5)
    C, L, K = tm.number_of_clauses, tm.number_of_literals, 10
    # clauses of 1-3 positive pixel literals, so that they fire on some samples only
    ta = np.full((C, L), 100, dtype=np.uint32)
    for c in range(1, C):
        ta[c, rng.choice(L // 2, size=1 + c % 3, replace=False)] = 200
    w = rng.integers(-20, 21, (C, K)).astype(np.float32)
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w,
                                  "patch_weights": np.zeros((C, tm.number_of_patches), np.int32),
                                  "min_y": None, "max_y": None}})
    ref.ta[...] = ta
    ref.w[...] = w
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX[-500:], ref.encode(X[-500:]))
    cs = tm.score(encX, is_X_encoded=True)
    np.testing.assert_array_equal(cs, ref.score(encX))
    monkeypatch.setenv("YTM_TRANSFORM_CHUNK", "70000")  # one transform pass over all samples
    np.testing.assert_array_equal(tm.transform(encX, is_X_encoded=True), ref.transform(encX))
