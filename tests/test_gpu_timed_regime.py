"""HIP path against the C oracle in the regime the benchmark times, at full size.

bench.py times config 2's epochs 6-25 (after 5 untimed ones) and configs 3-5's epochs 2-3
(after one).  By then most samples need no feedback (config 2: about 2% of them), the
streaming kernel runs long repaired streams, and the several-patch kernels skip the
feedback and the firing-patch scan of most samples.  Each test here trains the full-size
model on the GPU alone up to that point, loads the GPU's state (TA states, weights, patch
weights, and the step of the random stream) into the oracle, then runs the same window on
both and compares the states, the update counts, the feedback-sample counts and the class
sums of at least 2000 test samples, bit for bit:
  * config 2: epochs 1-3 from the start, then epoch 6 after 5 GPU epochs and epoch 25
    after 24 (the first and last timed epochs);
  * config 3: 2000 samples of epoch 3 after 2 GPU epochs;
  * config 4: 500 samples of epoch 3 after 2 GPU epochs;
  * config 5: 200 samples of epoch 3 after 2 GPU epochs.
Reference semantics: src/cutm/base.py:266-359 (the per-sample loop),
src/cutm/cuda/kernel.cu:255-316,531-613 (evaluation, selection, feedback), :319-343
(inference).
"""
import os
import time

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


def log(msg):
    print(f"[timed] {msg}", flush=True)


def encoded_workload(tm, cfg, n_test):
    """Encoded training set (full size), its labels, and the first n_test encoded test
    samples with their labels."""
    c = workloads.CONFIGS[cfg]
    if cfg == 4:  # the values of workloads.make(4), generated and encoded in chunks
        gen = workloads.CifarStream(c["n_train"], c["n_test"])
        encX = np.empty((c["n_train"], tm.number_of_patches, tm.number_of_literal_chunks), dtype=np.uint32)
        for s in range(0, c["n_train"], 2048):
            e = min(c["n_train"], s + 2048)
            encX[s:e] = tm.encode(gen.train_rows(s, e))
        encXt = tm.encode(gen.test_rows(0, n_test))
        return encX, gen.y, encXt, gen.yt[:n_test]
    X, y, Xt, yt, _ = workloads.make(cfg, None, n_test)
    return tm.encode(X), y, tm.encode(Xt), yt


def oracle_for(kw):
    kw = dict(kw)
    return orc.OracleTM(kw.pop("number_of_clauses_per_class"), kw.pop("T"), kw.pop("s"), kw.pop("dim"),
                        kw.pop("n_classes"), **kw)


def gpu_epochs(tm, data, n, where):
    for _ in range(n):
        tm.fit_device(data)
        st = tm.stats()
        log(f"{where} GPU epoch to step {st['step']}: updates {st['last_fit_updates']} feedback samples "
            f"{st['last_fit_feedback_samples']} kernel {st['train_kind']} stream {st['last_fit_stream']}")


def continue_both(tm, ref, data, encX, encY, first, count, where):
    """Loads the GPU model's state into the oracle, runs samples [first, first+count) on both,
    and compares everything the window changes."""
    st = tm.stats()
    ref.load_state(tm.get_ta_state(), tm.get_weights(), tm.get_patch_weights(), st["step"])
    t = time.perf_counter()
    tm.fit_device(data, first=first, count=count)
    st = tm.stats()
    upd = ref.fit_encoded(encX[first:first + count], encY[first:first + count])
    log(f"{where}: samples [{first}, {first + count}) at step {st['step'] - count}: updates {upd}, feedback "
        f"samples {ref.last_feedback_samples}, kernel {st['train_kind']} stream {st['last_fit_stream']} "
        f"(oracle + GPU {time.perf_counter() - t:.1f}s)")
    assert st["last_fit_updates"] == upd, f"update count {where}"
    assert st["last_fit_feedback_samples"] == ref.last_feedback_samples, f"feedback samples {where}"
    np.testing.assert_array_equal(tm.get_ta_state().reshape(ref.ta.shape), ref.ta, err_msg=f"TA {where}")
    np.testing.assert_array_equal(tm.get_weights().reshape(ref.w.shape), ref.w, err_msg=f"weights {where}")
    np.testing.assert_array_equal(tm.get_patch_weights().reshape(ref.pw.shape), ref.pw, err_msg=f"pw {where}")
    return st


def check_scores(tm, ref, encXt, where):
    cs = tm.score(encXt, is_X_encoded=True)
    np.testing.assert_array_equal(cs, ref.score(encXt), err_msg=f"class sums {where}")


def test_config2_first_three_epochs():
    kw = dict(workloads.CONFIGS[2]["model"], seed=workloads.MODEL_SEED)
    tm, ref = MultiClassTM(**kw), oracle_for(kw)
    encX, y, encXt, yt = encoded_workload(tm, 2, 2000)
    data = tm.device_data(encX, y, is_X_encoded=True)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(3):
        continue_both(tm, ref, data, encX, encY, 0, encX.shape[0], f"config 2 epoch {epoch + 1}")
    check_scores(tm, ref, encXt, "config 2 after 3 epochs, 2000 test samples")
    data.release()


def test_config2_timed_epochs():
    """Epoch 6 after 5 GPU epochs and epoch 25 after 24: the first and the last epoch that
    bench.py times (streaming kernel, feedback at about 2% of the samples)."""
    kw = dict(workloads.CONFIGS[2]["model"], seed=workloads.MODEL_SEED)
    tm, ref = MultiClassTM(**kw), oracle_for(kw)
    encX, y, encXt, yt = encoded_workload(tm, 2, 10000)
    data = tm.device_data(encX, y, is_X_encoded=True)
    encY = ref.encode_y_multiclass(y)
    N = encX.shape[0]
    gpu_epochs(tm, data, 5, "config 2")
    st = continue_both(tm, ref, data, encX, encY, 0, N, "config 2 epoch 6")
    assert st["last_fit_stream"] == 1 and st["last_fit_feedback_samples"] < N // 10
    gpu_epochs(tm, data, 18, "config 2")
    st = continue_both(tm, ref, data, encX, encY, 0, N, "config 2 epoch 25")
    assert st["last_fit_stream"] == 1
    check_scores(tm, ref, encXt, "config 2 after 25 epochs, 10000 test samples")
    data.release()


@pytest.mark.parametrize("cfg,window", [(3, 2000), (4, 500), (5, 200)])
def test_several_patch_and_text_timed_epoch(cfg, window):
    """Two GPU epochs, then the first `window` samples of epoch 3 on both: the feedback skip
    (no class can update) and, with several patches, the skipped firing-patch scan of
    clauses that fire on no patch."""
    kw = dict(workloads.CONFIGS[cfg]["model"], seed=workloads.MODEL_SEED)
    tm, ref = MultiClassTM(**kw), oracle_for(kw)
    encX, y, encXt, yt = encoded_workload(tm, cfg, 2000)
    data = tm.device_data(encX, y, is_X_encoded=True)
    encY = ref.encode_y_multiclass(y)
    gpu_epochs(tm, data, 2, f"config {cfg}")
    st = continue_both(tm, ref, data, encX, encY, 0, window, f"config {cfg} epoch 3")
    assert st["last_fit_feedback_samples"] < window, "the window should hold samples without feedback"
    check_scores(tm, ref, encXt, f"config {cfg} after 2 epochs + {window} samples, 2000 test samples")
    data.release()
