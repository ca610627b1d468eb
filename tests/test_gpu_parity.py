"""HIP path (libytm.so on the GPU) against the C oracle, bit for bit.

Parity bar: integer/bit work is bit-exact (encoded X, clause outputs, TA states, patch
weights, update counts); class sums and weights are integer-valued floats and must be
equal exactly as well.  Sizes are chosen so the oracle finishes in seconds; the full
configurations are covered by size-independent properties at the end.
"""
import os
import pickle

import numpy as np
import pytest

import workloads
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ytm_amd = pytest.importorskip("ytm_amd")
from ytm_amd import MultiClassTM, MultiOutputTM  # noqa: E402
from ytm_amd._lib import YtmError  # noqa: E402

orc.set_threads(min(16, os.cpu_count() or 1))

@pytest.fixture(autouse=True)
def _specialised_kernels_required(monkeypatch):
    """Training runs the kernels compiled per model (hipRTC); a failed compile is an error
    here rather than a silent switch to the built-in kernels (tested on their own below)."""
    monkeypatch.setenv("YTM_JIT", "2")


def pair(cfg, n_train, n_test=0, clauses=None, seed=workloads.MODEL_SEED, **opts):
    X, y, Xt, yt, kw = workloads.make(cfg, n_train, n_test)
    if clauses is not None:
        kw["number_of_clauses_per_class"] = clauses
    kw.update(opts)
    kw["seed"] = seed
    print(f"[pair] cfg={cfg} n_train={n_train} kw={kw}", flush=True)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(kw.pop("number_of_clauses_per_class"), kw.pop("T"), kw.pop("s"), kw.pop("dim"),
                       kw.pop("n_classes"), **kw)
    return tm, ref, X, y, Xt, yt


def assert_state_equal(tm, ref, where=""):
    np.testing.assert_array_equal(tm.get_ta_state().reshape(ref.ta.shape), ref.ta, err_msg=f"TA {where}")
    np.testing.assert_array_equal(tm.get_weights().reshape(ref.w.shape), ref.w, err_msg=f"weights {where}")
    np.testing.assert_array_equal(tm.get_patch_weights().reshape(ref.pw.shape), ref.pw, err_msg=f"pw {where}")


# ------------------------------------------------------------------ encode / init
@pytest.mark.parametrize("cfg,n", [(1, 64), (2, 32), (3, 8), (4, 4), (5, 16)])
def test_encode(cfg, n):
    tm, ref, X, *_ = pair(cfg, n)
    np.testing.assert_array_equal(tm.encode(X), ref.encode(X))


@pytest.mark.parametrize("dim,patch_dim", [((7, 6, 2), (3, 2)), ((12, 12, 3), (4, 5)), ((5, 9, 1), (5, 2)),
                                           ((33, 4, 1), (33, 2)), ((5000, 1, 1), (5000, 1)), ((70, 70, 1), (70, 70))])
@pytest.mark.parametrize("encode_loc,append_negated", [(True, True), (False, True), (True, False), (False, False)])
def test_encode_several_patch_variants(dim, patch_dim, encode_loc, append_negated):
    """The several-patch encoder (a block per sample, its pixel bits staged in LDS, a word's
    pixel literals taken as bit ranges of patch rows) against the oracle with and without
    position thermometers and appended negations, on patch shapes whose words hold ranges
    across rows, patches and the negated half, and a patch row longer than a word; also one
    patch of 313 and 307 words, which takes the same encoder."""
    kw = dict(patch_dim=patch_dim, encode_loc=encode_loc, append_negated=append_negated, seed=3)
    tm = MultiClassTM(10, 15, 3.9, dim=dim, n_classes=2, **kw)
    ref = orc.OracleTM(10, 15, 3.9, dim, 2, **kw)
    X = (np.random.default_rng(9).random((37,) + dim) < 0.4).astype(np.uint32).reshape(37, -1)
    np.testing.assert_array_equal(tm.encode(X), ref.encode(X))


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_initial_state(cfg):
    tm, ref, *_ = pair(cfg, 1)
    assert_state_equal(tm, ref, "init")
    assert np.all(tm.get_literals() == 0)
    assert np.all(tm.get_bias_weights() == 0)


# ------------------------------------------------------------------ training
@pytest.mark.parametrize(
    "cfg,n,clauses,epochs",
    [(1, 5000, None, 3), (2, 300, None, 2), (3, 40, None, 1), (3, 200, 200, 2), (4, 3, None, 1),
     (4, 40, 500, 1), (5, 4, None, 1), (5, 60, 300, 2)],
)
def test_fit_counter_stream(cfg, n, clauses, epochs):
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(epochs):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        assert tm.stats()["last_fit_updates"] == upd, f"update count epoch {epoch}"
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("cfg,n,clauses", [(1, 3000, None), (2, 200, None), (5, 30, 200), (3, 40, 100), (4, 6, 60)])
def test_fit_global_state_kernel(monkeypatch, cfg, n, clauses):
    """Every configuration also through the kernels that keep clause state in global
    memory (the default keeps it resident in LDS when it fits)."""
    monkeypatch.setenv("YTM_TRAIN_GLOBAL", "1")
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        assert tm.stats()["train_kind"] == (1 if tm.number_of_patches == 1 else 2)
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("cfg,n,clauses,global_state,inject",
                         [(1, 2000, None, False, False), (1, 1000, None, True, False), (2, 150, None, False, False),
                          (2, 100, None, True, False), (3, 40, 100, False, False), (3, 30, 100, True, False),
                          (4, 6, 60, False, False), (5, 30, 200, False, False), (1, 40, None, False, True),
                          (3, 4, 12, False, True)])
def test_fit_builtin_kernels(monkeypatch, cfg, n, clauses, global_state, inject):
    """The built-in training kernels (geometry read from the kernel arguments) give the
    same results as the per-model compiled ones: both against the oracle."""
    monkeypatch.setenv("YTM_JIT", "0")
    if global_state:
        monkeypatch.setenv("YTM_TRAIN_GLOBAL", "1")
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    rng = np.random.default_rng(cfg)
    for epoch in range(2):
        inj = rng.random(tm.random_stream_size(n)).astype(np.float32) if inject else None
        tm.fit(encX, y, is_X_encoded=True, random_stream=inj)
        upd = ref.fit_encoded(encX, encY, inject=inj)
        st = tm.stats()
        assert st["train_specialised"] == 0
        if global_state:
            assert st["train_kind"] == (2 if tm.number_of_patches > 1 else 1)
        assert st["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("cfg,n,clauses,epochs", [(1, 3000, None, 2), (2, 300, None, 2), (2, 200, 60, 3)])
def test_fit_resident_kernel_counter_stream(monkeypatch, cfg, n, clauses, epochs):
    """One-patch models on the resident kernel (the streaming kernel switched off)."""
    monkeypatch.setenv("YTM_TRAIN_STREAM", "0")
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(epochs):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        assert tm.stats()["train_kind"] == 0 and tm.stats()["last_fit_stream"] == 0
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")


def test_stream_kernel_choice_follows_feedback():
    """A new model updates at nearly every sample, so one-patch models start on the resident
    kernel and stay there while the feedback share is at half of the samples or more (config
    1, noisy XOR: every epoch); the counts of samples with feedback agree between the
    kernels, and every fit matches the oracle."""
    tm, ref, X, y, *_ = pair(1, 3000)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    kinds = []
    for epoch in range(3):
        upd = ref.fit_encoded(encX, encY)
        tm.fit(encX, y, is_X_encoded=True)
        st = tm.stats()
        kinds.append(st["train_kind"])
        assert st["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")
        assert st["last_fit_feedback_samples"] > 1500  # noisy XOR: feedback at nearly every sample
    assert kinds == [0, 0, 0]


def test_first_epoch_in_segments():
    """The first fits of a new config-2 model go in segments of 4096 samples on the resident
    kernel while the feedback share stays at half or more, then on the streaming kernel for
    the rest (config 2 on 12000 samples: feedback at 82% of the first epoch's samples, 45%
    of the second's); once the share is low a fit streams in one launch.  Update and
    feedback counts add up over the segments, and every fit matches the oracle."""
    tm, ref, X, y, *_ = pair(2, 12000)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(4):
        upd = ref.fit_encoded(encX, encY)
        tm.fit(encX, y, is_X_encoded=True)
        st = tm.stats()
        print(f"[segments] epoch {epoch}: kind {st['train_kind']} launches {st['last_fit_launches']} "
              f"feedback samples {st['last_fit_feedback_samples']} updates {upd}", flush=True)
        assert st["last_fit_updates"] == upd, f"update count epoch {epoch}"
        assert st["last_fit_feedback_samples"] == ref.last_feedback_samples
        assert st["last_fit_samples"] == 12000
        assert_state_equal(tm, ref, f"epoch {epoch}")
        if epoch == 0:
            assert st["last_fit_launches"] >= 2
    assert st["train_kind"] == 3 and st["last_fit_launches"] == 1


@pytest.mark.parametrize("wgs,threads,gens", [("", "", ""), ("7", "", ""), ("31", "512", ""), ("64", "256", ""),
                                              ("", "", "1"), ("7", "", "3")])
def test_fit_stream_launch_shapes(monkeypatch, wgs, threads, gens):
    """The streaming kernel (one patch, counter stream) against the oracle over several
    epochs, as training moves from feedback on most samples to feedback on few, for several
    grids (50 clauses per workgroup down to 3) and workgroup sizes.  A stream normally goes
    on past each stop (the rows published past it get the updated clauses' vote
    differences); YTM_TRAIN_STREAM_GENS makes it start a fresh one on fresh rows every
    1 or 3 stops instead."""
    monkeypatch.setenv("YTM_TRAIN_WGS", wgs)
    monkeypatch.setenv("YTM_TRAIN_THREADS", threads)
    monkeypatch.setenv("YTM_TRAIN_STREAM_GENS", gens)
    monkeypatch.setenv("YTM_TRAIN_STREAM", "1")  # also where the last fit had feedback at most samples
    tm, ref, X, y, *_ = pair(2, 2000, clauses=200)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(4):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        st = tm.stats()
        assert st["last_fit_stream"] == 1 and st["train_kind"] == 3
        assert st["last_fit_updates"] == upd, f"update count epoch {epoch}"
        assert 0 < st["last_fit_feedback_samples"] <= 2000
        assert st["last_fit_evaluations"] >= 2000
        print(f"[stream] wgs={wgs or 'default'} epoch {epoch}: feedback samples {st['last_fit_feedback_samples']}, "
              f"evaluations {st['last_fit_evaluations']}, updates {upd}", flush=True)
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("classes,wlim", [(10, 50), (10, 511), (10, 512), (3, 300), (3, 3000)])
def test_stream_votes_with_large_weights(monkeypatch, classes, wlim):
    """The streaming kernel sums two classes' votes in one 32-bit reduction while every own
    clause's |weight| is below 512, and one class at a time otherwise (an odd class count
    leaves one class alone either way).  Weights drawn from [-wlim, wlim] put the workgroups
    on either side of that bound; both against the oracle."""
    monkeypatch.setenv("YTM_TRAIN_STREAM", "1")
    kw = dict(number_of_clauses_per_class=120, T=400, s=4.0, dim=(40, 1, 1), n_classes=classes, seed=13)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(120, 400, 4.0, (40, 1, 1), classes, seed=13)
    rng = np.random.default_rng(wlim)
    X = (rng.random((600, 40)) < 0.5).astype(np.uint32)
    y = rng.integers(0, classes, size=600).astype(np.uint32)
    ta = tm.get_ta_state().reshape(ref.ta.shape)
    w = rng.integers(-wlim, wlim + 1, ref.w.shape).astype(np.float32)
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w,
                                  "patch_weights": np.zeros(ref.pw.shape, dtype=np.int32),
                                  "min_y": None, "max_y": None}})
    ref.w[...] = w
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, encY)
        assert tm.stats()["train_kind"] == 3
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("env", [dict(YTM_TRAIN_STREAM="1"), dict(YTM_TRAIN_STREAM="0"),
                                 dict(YTM_TRAIN_STREAM="0", YTM_TRAIN_GLOBAL="1")])
def test_rank1_draw_of_exactly_one(monkeypatch, env):
    """With one patch a firing clause is selected unless its reservoir draw is exactly 1.0
    (u < 1.0f / 1, kernel.cu:295-301), which happens once in 2^24 draws of the counter stream.
    Seed 6589 has that draw at step 58 for clause 28, among the first steps of a fresh model:
    the streaming, resident and global one-patch kernels against the oracle."""
    ctr_word = orc.philox4x32_10([58, 28, 1 << 28, 0], [6589, 0])[0]
    assert (int(ctr_word) >> 8) == 0xFFFFFF  # site (t=58, c=28, SEL, 0), word 0: u = 1.0
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    kw = dict(number_of_clauses_per_class=64, T=10, s=3.9, dim=(16, 1, 1), n_classes=2, seed=6589)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(64, 10, 3.9, (16, 1, 1), 2, seed=6589)
    rng = np.random.default_rng(1)
    X = (rng.random((100, 16)) < 0.5).astype(np.uint32)
    y = rng.integers(0, 2, size=100).astype(np.uint32)
    encX = tm.encode(X)
    # clause 28 fires on sample 58 after the first 58 steps: the rejected draw decides its selection
    pre = orc.OracleTM(64, 10, 3.9, (16, 1, 1), 2, seed=6589)
    pre.fit_encoded(encX[:58], pre.encode_y_multiclass(y[:58]))
    inc = pre.ta.reshape(64, -1)[28] > tm.number_of_ta_states // 2
    bits = np.unpackbits(encX[58].reshape(-1).view(np.uint8), bitorder="little")[:inc.size]
    assert np.all(bits[inc] == 1)
    tm.fit(encX, y, is_X_encoded=True)
    upd = ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    want = 3 if env["YTM_TRAIN_STREAM"] == "1" else (1 if "YTM_TRAIN_GLOBAL" in env else 0)
    assert tm.stats()["train_kind"] == want
    assert tm.stats()["last_fit_updates"] == upd
    assert_state_equal(tm, ref)


def test_specialised_kernel_is_used():
    tm, ref, X, y, *_ = pair(2, 20)
    tm.fit(tm.encode(X), y, is_X_encoded=True)
    assert tm.stats()["train_specialised"] == 1


@pytest.mark.parametrize("cfg,n,clauses", [(1, 60, None), (2, 6, 40), (3, 5, 12), (4, 2, 6), (5, 3, 4)])
def test_fit_injected_stream(cfg, n, clauses):
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    rng = np.random.default_rng(cfg)
    s_inv = np.float32(orc.s_inv_of(workloads.CONFIGS[cfg]["model"]["s"]))
    for epoch in range(2):
        inj = rng.random(tm.random_stream_size(n)).astype(np.float32)
        inj[::13] = 1.0       # reservoir rejects u = 1.0
        inj[7::29] = s_inv    # literal draw exactly at S_INV is accepted
        tm.fit(encX, y, is_X_encoded=True, random_stream=inj)
        upd = ref.fit_encoded(encX, encY, inject=inj)
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")


@pytest.mark.parametrize("T", [3, 4, 16777215, 16777216])
def test_update_test_at_its_boundaries(T):
    """Update draws injected at the probabilities (y - v) / (2y) that clipped class sums
    v in [-T, T] give (kernel.cu:508-529), rounded to float, and at the floats either side.
    The GPU's feedback decisions for a few clauses per workgroup test u <= prob without
    the division, and clip the integer sum, for integral T < 2^24; 2^24 takes the division.
    The oracle divides (double, IEEE), so every equality and rounding case is checked."""
    kw = dict(number_of_clauses_per_class=8, T=T, s=3.0, dim=(16, 1, 1), n_classes=3, seed=11)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(8, T, 3.0, (16, 1, 1), 3, seed=11)
    n = 60
    rng = np.random.default_rng(T % 1009)
    X = (rng.random((n, 16)) < 0.5).astype(np.uint32)
    y = rng.integers(0, 3, size=n).astype(np.uint32)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    C, K, P, L = tm.number_of_clauses, 3, tm.number_of_patches, tm.number_of_literals
    vs = np.arange(-min(T, 40), min(T, 40) + 1, dtype=np.float64)
    vs = np.concatenate([vs, [-T, T]])
    q = np.concatenate([(T - vs) / (2.0 * T), (-T - vs) / (-2.0 * T)])
    f = q.astype(np.float32)
    cand = np.unique(np.concatenate([f, np.nextafter(f, np.float32(2)), np.nextafter(f, np.float32(-1))]))
    cand = cand[(cand > 0) & (cand <= 1)]
    block = C * P + 2 * C * K + C * K * L
    lo, hi = C * P + C * K, C * P + 2 * C * K  # the update draws of a sample block
    for epoch in range(3):
        inj = rng.random(tm.random_stream_size(n)).astype(np.float32).reshape(n, block)
        inj[:, lo:hi] = rng.choice(cand, size=(n, hi - lo))
        inj = inj.ravel()
        tm.fit(encX, y, is_X_encoded=True, random_stream=inj)
        upd = ref.fit_encoded(encX, encY, inject=inj)
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"T={T} epoch {epoch}")


@pytest.mark.parametrize(
    "opts",
    [dict(coalesced=False), dict(negative_polarity=False, init_neg_weights=False), dict(max_included_literals=4),
     dict(append_negated=False), dict(number_of_ta_states=16), dict(q=3), dict(q=0.5)],
)
def test_fit_variant_flags(opts):
    tm, ref, X, y, *_ = pair(2, 200, clauses=60, **opts)
    encX = tm.encode(X)
    for _ in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    assert_state_equal(tm, ref, str(opts))


@pytest.mark.parametrize("case", [
    dict(dim=(16, 1, 1), n_classes=64, clauses=64, n=160),                           # 64 classes: a lane per class
    dict(dim=(20, 1, 1), n_classes=3, clauses=40, n=120, number_of_ta_states=65535),  # 16 state bit-planes
    dict(dim=(20, 1, 1), n_classes=3, clauses=40, n=120, number_of_ta_states=(1 << 20) + 3),  # 21 bit-planes
    dict(dim=(20, 1, 1), n_classes=3, clauses=40, n=120, number_of_ta_states=2**31 - 1),  # 31: the int32 maximum
    dict(dim=(66, 66, 1), patch_dim=(3, 3), n_classes=2, clauses=16, n=3),            # 4096 patches (no literal-major copy)
    # beyond the persistent kernels: a launch per sample, decisions 64 classes at a time
    dict(dim=(16, 1, 1), n_classes=65, clauses=40, n=200),
    dict(dim=(12, 1, 1), n_classes=150, clauses=30, n=300),
    dict(dim=(8, 8, 1), patch_dim=(3, 3), n_classes=70, clauses=20, n=40),
    dict(dim=(16, 1, 1), n_classes=70, clauses=2, n=200, coalesced=False),
    # more patches than 64 chunks of 64: the reservoir's patch found in a second pass
    dict(dim=(70, 70, 1), patch_dim=(3, 3), n_classes=2, clauses=12, n=3),
    dict(dim=(130, 130, 1), patch_dim=(2, 2), n_classes=3, clauses=4, n=2),
])
def test_supported_limits(case):
    """Training, scores and clause outputs at the largest sizes the persistent kernels take
    and beyond them: more than 64 classes (one launch per sample) and more than 4096 patches."""
    case = dict(case)
    n, clauses = case.pop("n"), case.pop("clauses")
    kw = dict(number_of_clauses_per_class=clauses, T=20, s=3.0, seed=5, **case)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(clauses, 20, 3.0, kw["dim"], kw["n_classes"],
                       **{k: v for k, v in kw.items() if k in ("patch_dim", "number_of_ta_states", "seed", "coalesced")})
    rng = np.random.default_rng(17)
    X = (rng.random((n, int(np.prod(kw["dim"])))) < 0.5).astype(np.uint32)
    y = rng.integers(0, kw["n_classes"], size=n).astype(np.uint32)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX, ref.encode(X))
    for epoch in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, ref.encode_y_multiclass(y))
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")
        if kw["n_classes"] > 64:
            assert tm.stats()["train_kind"] == 4
    np.testing.assert_array_equal(tm.score(encX, is_X_encoded=True), ref.score(encX))
    np.testing.assert_array_equal(tm.transform(encX, is_X_encoded=True), ref.transform(encX))
    ref_pw = ref.transform(encX[:2], patchwise=True)
    np.testing.assert_array_equal(tm.transform_patchwise(encX[:2], is_X_encoded=True), ref_pw)
    assert_packed_equal(tm.transform_patchwise(encX[:2], is_X_encoded=True, packed=True), ref_pw)


@pytest.mark.parametrize("case", [
    dict(dim=(12, 1, 1), n_classes=130, clauses=24, n=120),
    dict(dim=(8, 8, 1), patch_dim=(3, 3), n_classes=66, clauses=16, n=30),
])
def test_many_classes_injected_and_multioutput(case):
    """More than 64 classes on the per-sample path: injected draws (Q-skip, update and
    literal draws indexed by class past 64, reservoir u = 1.0), then MultiOutputTM with 70
    outputs, against the oracle."""
    case = dict(case)
    n, clauses = case.pop("n"), case.pop("clauses")
    kw = dict(number_of_clauses_per_class=clauses, T=15, s=2.5, seed=9, **case)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(clauses, 15, 2.5, kw["dim"], kw["n_classes"],
                       **{k: v for k, v in kw.items() if k in ("patch_dim", "seed")})
    rng = np.random.default_rng(31)
    X = (rng.random((n, int(np.prod(kw["dim"])))) < 0.5).astype(np.uint32)
    y = rng.integers(0, kw["n_classes"], size=n).astype(np.uint32)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    for epoch in range(2):
        inj = rng.random(tm.random_stream_size(n)).astype(np.float32)
        inj[::13] = 1.0
        tm.fit(encX, y, is_X_encoded=True, random_stream=inj)
        upd = ref.fit_encoded(encX, encY, inject=inj)
        assert tm.stats()["train_kind"] == 4
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"injected epoch {epoch}")
    np.testing.assert_array_equal(tm.score(encX, is_X_encoded=True), ref.score(encX))
    # multi-output: 70 independent +-T targets
    from ytm_amd import MultiOutputTM
    mo = MultiOutputTM(**dict(kw, n_classes=70))
    refo = orc.OracleTM(clauses, 15, 2.5, kw["dim"], 70, **{k: v for k, v in kw.items() if k in ("patch_dim", "seed")})
    Y = (rng.random((n, 70)) < 0.3).astype(np.uint32)
    mo.fit(encX, Y, is_X_encoded=True)
    upd = refo.fit_encoded(encX, np.where(Y == 1, 15, -15).astype(np.int32))
    assert mo.stats()["last_fit_updates"] == upd
    assert_state_equal(mo, refo, "multi-output")
    np.testing.assert_array_equal(mo.score(encX, is_X_encoded=True), refo.score(encX))


def test_scoring_lists_follow_the_state():
    """One-patch scoring keeps its literal lists between calls while the TA states are
    unchanged: scores after a second call, after more training and after ytm_set_ta_state
    (load_state_dict) all equal the oracle's."""
    tm, ref, X, y, Xt, yt = pair(2, 300, 200, clauses=120)
    encX, encXt = tm.encode(X), tm.encode(Xt)
    encY = ref.encode_y_multiclass(y)
    data = tm.device_data(encXt, is_X_encoded=True)
    tm.fit(encX[:200], y[:200], is_X_encoded=True)
    ref.fit_encoded(encX[:200], encY[:200])
    for where in ("first", "again"):
        np.testing.assert_array_equal(tm.score_device(data), ref.score(encXt), err_msg=where)
    tm.fit(encX[200:], y[200:], is_X_encoded=True)
    ref.fit_encoded(encX[200:], encY[200:])
    np.testing.assert_array_equal(tm.score_device(data), ref.score(encXt), err_msg="after training")
    rng = np.random.default_rng(8)
    ta = np.where(rng.random(ref.ta.shape) < 0.02, 200, 60).astype(np.uint32)
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": tm.get_weights(),
                                  "patch_weights": tm.get_patch_weights(), "min_y": None, "max_y": None}})
    ref.load_state(ta, ref.w, ref.pw, ref.step)
    np.testing.assert_array_equal(tm.score_device(data), ref.score(encXt), err_msg="after set_ta_state")
    data.release()


@pytest.mark.parametrize("wmax", [2048, 2049, 100000])
def test_wide_scoring_weight_range(wmax):
    """One-patch wide scoring with 4 or more classes sums the votes of a wave's 64 clauses
    on the matrix cores while every weight of those clauses is at most 2048 in magnitude
    (f16 holds it exactly) and adds them one by one otherwise: random states with weights
    up to +-2048 (both bounds present), one weight of 2049 in the second wave's clauses,
    and weights up to +-100000, against the oracle."""
    print(f"[wide weights] wmax {wmax}", flush=True)
    rng = np.random.default_rng(31)
    kw = dict(number_of_clauses_per_class=300, T=50, s=5.0, dim=(28, 28, 1), n_classes=10)
    tm = MultiClassTM(**kw, seed=7)
    C, L, K = tm.number_of_clauses, tm.number_of_literals, tm.number_of_outputs
    ta = np.where(rng.random((C, L)) < 3.0 / L, 200, 60).astype(np.uint32)
    lim = min(wmax, 2048) if wmax != 100000 else wmax
    w = rng.integers(-lim, lim + 1, (C, K)).astype(np.float32)
    w[0, :], w[1, :] = 2048.0, -2048.0
    if wmax == 2049:
        w[100, 3] = 2049.0
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w,
                                  "patch_weights": np.zeros((C, 1), np.int32), "min_y": None, "max_y": None}})
    Xt = (rng.random((700, 28 * 28)) < 0.5).astype(np.uint32)
    encXt = tm.encode(Xt)
    oracle = orc.OracleTM(300, 50, 5.0, (28, 28, 1), 10)
    oracle.load_state(tm.get_ta_state(), tm.get_weights(), tm.get_patch_weights(), tm.stats()["step"])
    want = oracle.score(encXt)
    assert np.count_nonzero(want) > want.size // 2, "a meaningful comparison needs firing clauses"
    np.testing.assert_array_equal(tm.score(encXt, is_X_encoded=True), want)
    tm.release()


def test_fit_conv_lists_of_literal_indices():
    """Literal lists hold byte offsets into the literal-major sample only while those fit 16
    bits; with 696 literals over 29 patch words ((L-1) * 4 * 29 > 65535) they hold literal
    indices.  Training, scores and clause outputs against the oracle on that geometry."""
    kw = dict(number_of_clauses_per_class=24, T=20, s=3.0, dim=(32, 32, 32), patch_dim=(3, 3), n_classes=2, seed=3)
    tm = MultiClassTM(**kw)
    assert (tm.number_of_literals - 1) * 4 * 29 > 0xFFFF
    ref = orc.OracleTM(24, 20, 3.0, (32, 32, 32), 2, patch_dim=(3, 3), seed=3)
    rng = np.random.default_rng(23)
    X = (rng.random((12, 32 * 32 * 32)) < 0.5).astype(np.uint32)
    y = rng.integers(0, 2, size=12).astype(np.uint32)
    encX = tm.encode(X)
    for epoch in range(3):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, ref.encode_y_multiclass(y))
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")
    np.testing.assert_array_equal(tm.score(encX, is_X_encoded=True), ref.score(encX))
    np.testing.assert_array_equal(tm.transform(encX, is_X_encoded=True), ref.transform(encX))


def test_fit_conv_variant_no_loc():
    tm, ref, X, y, *_ = pair(3, 30, clauses=50, encode_loc=False)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX, ref.encode(X))
    tm.fit(encX, y, is_X_encoded=True)
    ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    assert_state_equal(tm, ref)


@pytest.mark.parametrize("halves_env", ["", "0"])
def test_encoded_samples_without_complement_halves(monkeypatch, halves_env):
    """Samples encoded elsewhere (fit(is_X_encoded=True)) need not hold the negated literals as
    the complements of the others.  Where they do, the several-patch training kernels stage
    only the first half of a sample's literal-major copy and complement it; where they do
    not (bits flipped here), the whole copy.  Both against the oracle; YTM_TRAIN_XT_HALVES=0
    stages the whole copy either way."""
    monkeypatch.setenv("YTM_TRAIN_GLOBAL", "1")
    monkeypatch.setenv("YTM_TRAIN_XT_HALVES", halves_env)
    tm, ref, X, y, *_ = pair(4, 8, clauses=40)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    L = tm.number_of_literals
    rng = np.random.default_rng(3)
    odd = encX.copy()
    for e in range(0, len(odd), 2):  # every other sample: a few literals of a few patches flipped
        for _ in range(5):
            p, l = rng.integers(tm.number_of_patches), rng.integers(L)
            odd[e, p, l // 32] ^= np.uint32(1 << (l % 32))
    for data in (encX, odd):
        tm.fit(data, y, is_X_encoded=True)
        upd = ref.fit_encoded(data, encY)
        assert tm.stats()["train_kind"] == 2
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref)


@pytest.mark.parametrize("cfg,n,clauses,opts", [
    (2, 150, 30, dict()),                                          # one patch
    (3, 30, 20, dict()),                                           # several patches
    (5, 60, 40, dict(negative_polarity=False, init_neg_weights=False)),
    (1, 400, None, dict(max_included_literals=3, q=2)),
])
def test_fit_clause_banks(cfg, n, clauses, opts):
    """Clause banks (coalesced=False, kernel.cu:59-67,306-312,563-565): each clause votes for
    and learns only its bank's class.  Counter stream, injected draws and a clause drop mask,
    then scores and clause outputs of the trained model, against the oracle."""
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses, coalesced=False, **opts)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    tm.fit(encX, y, is_X_encoded=True)
    upd = ref.fit_encoded(encX, encY)
    assert tm.stats()["train_kind"] == 4
    assert tm.stats()["last_fit_updates"] == upd
    assert_state_equal(tm, ref, "counter stream")
    rng = np.random.default_rng(cfg + 100)
    inj = rng.random(tm.random_stream_size(n)).astype(np.float32)
    inj[::13] = 1.0
    tm.fit(encX, y, is_X_encoded=True, random_stream=inj)
    upd = ref.fit_encoded(encX, encY, inject=inj)
    assert tm.stats()["last_fit_updates"] == upd
    assert_state_equal(tm, ref, "injected")
    drop_rng = np.random.default_rng(workloads.MODEL_SEED)  # the model's numpy rng (base.py:123,289)
    tm.fit(encX, y, is_X_encoded=True, clause_drop_p=0.25)
    drop = (drop_rng.random(ref.C) <= 0.25).astype(np.uint32)
    upd = ref.fit_encoded(encX, encY, drop=drop)
    assert tm.stats()["last_fit_updates"] == upd
    assert_state_equal(tm, ref, "clause drop")
    w = tm.get_weights().reshape(ref.w.shape)
    bank = np.arange(ref.C) // (ref.C // w.shape[1])
    off_bank = np.ones_like(w, dtype=bool)
    off_bank[np.arange(ref.C), bank] = False
    assert np.all(w[off_bank] == 0)  # weights outside the own bank stay 0
    np.testing.assert_array_equal(tm.score(encX, is_X_encoded=True), ref.score(encX))
    np.testing.assert_array_equal(tm.transform(encX, is_X_encoded=True), ref.transform(encX))


def test_clause_drop():
    tm, ref, X, y, *_ = pair(2, 150, clauses=80)
    encX = tm.encode(X)
    drop_rng = np.random.default_rng(workloads.MODEL_SEED)  # the model's numpy rng (base.py:123,289)
    for _ in range(2):
        tm.fit(encX, y, is_X_encoded=True, clause_drop_p=0.3)
        drop = (drop_rng.random(ref.C) <= 0.3).astype(np.uint32)
        ref.fit_encoded(encX, ref.encode_y_multiclass(y), drop=drop)
    assert_state_equal(tm, ref)


@pytest.mark.parametrize("cfg,n,clauses,global_state", [(3, 120, 100, False), (3, 60, 100, True), (4, 12, 60, False)])
def test_clause_drop_several_patches(monkeypatch, cfg, n, clauses, global_state):
    """A clause drop mask on models with several patches (resident and global kernels): a
    dropped clause fires on no patch, so its reservoir step takes the no-firing exit, and
    neither votes nor learns."""
    if global_state:
        monkeypatch.setenv("YTM_TRAIN_GLOBAL", "1")
    tm, ref, X, y, *_ = pair(cfg, n, clauses=clauses)
    encX = tm.encode(X)
    encY = ref.encode_y_multiclass(y)
    drop_rng = np.random.default_rng(workloads.MODEL_SEED)  # the model's numpy rng (base.py:123,289)
    for epoch in range(2):
        tm.fit(encX, y, is_X_encoded=True, clause_drop_p=0.3)
        drop = (drop_rng.random(ref.C) <= 0.3).astype(np.uint32)
        upd = ref.fit_encoded(encX, encY, drop=drop)
        assert tm.stats()["last_fit_updates"] == upd, f"update count epoch {epoch}"
        assert_state_equal(tm, ref, f"clause drop, epoch {epoch}")


def test_launch_shape_independence(monkeypatch):
    """The same seed gives the same model whatever the persistent grid / copy grouping."""
    states = []
    for wgs, group in [("", ""), ("3", "1"), ("17", "4"), ("256", "64")]:
        monkeypatch.setenv("YTM_TRAIN_WGS", wgs)
        monkeypatch.setenv("YTM_TRAIN_GROUP", group)
        tm, _, X, y, *_ = pair(3, 60, clauses=100)
        tm.fit(tm.encode(X), y, is_X_encoded=True)
        states.append((tm.get_ta_state(), tm.get_weights(), tm.get_patch_weights()))
    for s in states[1:]:
        for a, b in zip(states[0], s):
            np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("cfg,clauses", [(2, 100), (3, 30)])  # streaming kernel; resident conv kernel
def test_timeout_leaves_model_refusing_until_reloaded(monkeypatch, cfg, clauses):
    """A class-sum wait that expires (forced from the host: YTM_TRAIN_TEST_TIMEOUT makes every
    wait miss its sums and expire at once, and every workgroup exits normally) returns
    YTM_ETIMEOUT; the model then refuses fit and score until a whole state is loaded again,
    and trains on from there like the oracle does."""
    tm, ref, X, y, Xt, yt = pair(cfg, 60, 20, clauses=clauses)
    encX = tm.encode(X)
    tm.fit(encX, y, is_X_encoded=True)
    ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    state = tm.get_state_dict()
    monkeypatch.setenv("YTM_TRAIN_TEST_TIMEOUT", "1")
    with pytest.raises(YtmError, match="bounded wait"):
        tm.fit(encX, y, is_X_encoded=True)
    monkeypatch.delenv("YTM_TRAIN_TEST_TIMEOUT")
    with pytest.raises(ValueError, match="timed out"):
        tm.fit(encX, y, is_X_encoded=True)
    with pytest.raises(ValueError, match="timed out"):
        tm.score(tm.encode(Xt), is_X_encoded=True)
    tm.load_state_dict({"state": state})
    # the failed launch advanced neither the model's step nor the oracle's: both go on alike
    assert tm.stats()["step"] == ref.step
    tm.fit(encX, y, is_X_encoded=True)
    assert tm.stats()["last_fit_updates"] == ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    assert_state_equal(tm, ref, "after reloading")
    np.testing.assert_array_equal(tm.score(tm.encode(Xt), is_X_encoded=True), ref.score(ref.encode(Xt)))


# ------------------------------------------------------------------ inference
@pytest.mark.parametrize("cfg,n_train,n_test,clauses", [(1, 2000, 500, None), (2, 300, 300, None),
                                                        (3, 60, 40, 300), (4, 10, 8, 400), (5, 40, 60, 300)])
def test_score_transform(cfg, n_train, n_test, clauses):
    tm, ref, X, y, Xt, yt = pair(cfg, n_train, n_test, clauses=clauses)
    encX = tm.encode(X)
    tm.fit(encX, y, is_X_encoded=True)
    ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    encXt = tm.encode(Xt)
    preds, cs = tm.predict(encXt, is_X_encoded=True)
    ref_cs = ref.score(encXt)
    np.testing.assert_array_equal(cs, ref_cs)
    np.testing.assert_array_equal(preds, np.argmax(ref_cs, axis=1))
    np.testing.assert_array_equal(tm.transform(encXt, is_X_encoded=True), ref.transform(encXt))
    n_pw = min(n_test, 12)
    ref_pw = ref.transform(encXt[:n_pw], patchwise=True)
    np.testing.assert_array_equal(tm.transform_patchwise(encXt[:n_pw], is_X_encoded=True), ref_pw)
    assert_packed_equal(tm.transform_patchwise(encXt[:n_pw], is_X_encoded=True, packed=True), ref_pw)


def assert_packed_equal(packed, ref_pw):
    """packed: uint32 (N, C, ceil(P/32)), bit b of word j = patch 32j + b, zero beyond P."""
    P = ref_pw.shape[2]
    assert packed.dtype == np.uint32 and packed.shape == ref_pw.shape[:2] + ((P + 31) // 32,)
    bits = np.unpackbits(np.ascontiguousarray(packed).view(np.uint8), axis=-1, bitorder="little")
    np.testing.assert_array_equal(bits[..., :P], ref_pw)
    assert not bits[..., P:].any()


def random_state(tm, ref, rng, include_p):
    """Random TA states (each literal included with probability include_p[c] per clause)
    and random integer weights, loaded into both models."""
    C, L, K = tm.number_of_clauses, tm.number_of_literals, ref.w.shape[1]
    half = tm.number_of_ta_states // 2
    inc = rng.random((C, L)) < np.asarray(include_p)[:, None]
    ta = np.where(inc, rng.integers(half + 1, 2 * half + 1, (C, L)), rng.integers(0, half + 1, (C, L)))
    ta = ta.astype(np.uint32)
    w = rng.integers(-50, 51, (C, K)).astype(np.float32)
    pw = np.zeros((C, tm.number_of_patches), dtype=np.int32)
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w, "patch_weights": pw,
                                  "min_y": None, "max_y": None}})
    ref.ta[...] = ta.reshape(ref.ta.shape)
    ref.w[...] = w.reshape(ref.w.shape)


@pytest.mark.parametrize("dim,patch_dim,classes,clauses", [
    ((100, 1, 1), None, 3, 300),     # one patch, 7 words
    ((30, 1, 1), None, 20, 200),     # one patch, more classes than the tiled scorer holds
    ((1500, 1, 1), None, 2, 150),    # one patch, 94 words
    ((12, 12, 2), (4, 4), 4, 300),   # several patches, literal lists
    ((16, 16, 16), (3, 3), 3, 120),  # several patches, 340 literals: some clauses beyond the list capacity
    ((32, 32, 32), (3, 3), 2, 40),   # 696 literals x 29 patch words: list entries are literal indices
])
def test_inference_random_state(dim, patch_dim, classes, clauses):
    """Class sums and clause outputs on random states: every inference kernel variant
    (tiles, lists, the include-mask fallback) against the oracle."""
    kw = dict(number_of_clauses_per_class=clauses, T=50, s=5.0, dim=dim, n_classes=classes, seed=7)
    if patch_dim is not None:
        kw["patch_dim"] = patch_dim
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(clauses, 50, 5.0, dim, classes, **({"patch_dim": patch_dim} if patch_dim else {}), seed=7)
    rng = np.random.default_rng(11)
    L = tm.number_of_literals
    # mostly narrow clauses (these fire), some empty ones, some with over 256 literals
    include_p = np.where(rng.random(tm.number_of_clauses) < 0.1, 0.0, 3.0 / L)
    include_p[rng.random(tm.number_of_clauses) < 0.05] = min(1.0, 300.0 / L)
    random_state(tm, ref, rng, include_p)
    X = (rng.random((70,) + tuple(dim)) < 0.5).astype(np.uint32).reshape(70, -1)
    encX = tm.encode(X)
    np.testing.assert_array_equal(encX, ref.encode(X))
    np.testing.assert_array_equal(tm.score(encX, is_X_encoded=True), ref.score(encX))
    np.testing.assert_array_equal(tm.transform(encX, is_X_encoded=True), ref.transform(encX))
    ref_pw = ref.transform(encX[:9], patchwise=True)
    np.testing.assert_array_equal(tm.transform_patchwise(encX[:9], is_X_encoded=True), ref_pw)
    assert_packed_equal(tm.transform_patchwise(encX[:9], is_X_encoded=True, packed=True), ref_pw)


def test_score_whole_sample_blocks(monkeypatch):
    """A literal-major copy above 32 KB (1024-thread scoring blocks) and more than 4096
    clauses: blocks over every clause of a sample (taken from YTM_SCORE_WHOLE_MIN samples
    on) give the class sums of blocks over chunks of 4096 clauses, and the oracle's."""
    dim, patch_dim, classes, clauses = (32, 32, 10), (3, 3), 3, 4300
    kw = dict(number_of_clauses_per_class=clauses, T=50, s=5.0, dim=dim, n_classes=classes, seed=7,
              patch_dim=patch_dim)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(clauses, 50, 5.0, dim, classes, patch_dim=patch_dim, seed=7)
    L, P = tm.number_of_literals, tm.number_of_patches
    assert L * ((P + 31) // 32) * 4 > 32 * 1024 and tm.number_of_clauses > 4096
    rng = np.random.default_rng(17)
    include_p = np.where(rng.random(tm.number_of_clauses) < 0.1, 0.0, 3.0 / L)
    random_state(tm, ref, rng, include_p)
    X = (rng.random((20,) + dim) < 0.5).astype(np.uint32).reshape(20, -1)
    encX = tm.encode(X)
    monkeypatch.setenv("YTM_SCORE_WHOLE_MIN", "1")
    whole = tm.score(encX, is_X_encoded=True)
    monkeypatch.setenv("YTM_SCORE_WHOLE_MIN", "1000000")
    chunked = tm.score(encX, is_X_encoded=True)
    np.testing.assert_array_equal(whole, chunked)
    np.testing.assert_array_equal(whole[:3], ref.score(encX[:3]))


@pytest.mark.parametrize("global_state", [False, True])
def test_fit_random_state_wide_one_patch(monkeypatch, global_state):
    """Training from a random state of a one-patch model with 94-word clauses, some of which
    include ~300 literals, on the resident and the global kernel."""
    if global_state:
        monkeypatch.setenv("YTM_TRAIN_GLOBAL", "1")
    dim, classes, clauses = (1500, 1, 1), 2, 60
    kw = dict(number_of_clauses_per_class=clauses, T=50, s=5.0, dim=dim, n_classes=classes, seed=7)
    tm = MultiClassTM(**kw)
    ref = orc.OracleTM(clauses, 50, 5.0, dim, classes, seed=7)
    rng = np.random.default_rng(13)
    L = tm.number_of_literals
    include_p = np.where(rng.random(tm.number_of_clauses) < 0.1, 0.0, 4.0 / L)
    include_p[rng.random(tm.number_of_clauses) < 0.1] = 300.0 / L
    random_state(tm, ref, rng, include_p)
    X = (rng.random((80, 1500)) < 0.9).astype(np.uint32)  # dense, so that wide clauses can fire
    y = rng.integers(0, classes, size=80).astype(np.uint32)
    encX = tm.encode(X)
    for epoch in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, ref.encode_y_multiclass(y))
        assert tm.stats()["last_fit_updates"] == upd
        assert_state_equal(tm, ref, f"epoch {epoch}")
    if global_state:
        assert tm.stats()["train_kind"] == 1


@pytest.mark.parametrize("cfg", [3, 5])  # several patches; one patch with 625-word clauses
def test_transform_in_chunks(monkeypatch, cfg):
    """Samples go through transform in chunks (forced small here): ragged last chunk, the
    literal lists built once and reused."""
    tm, ref, X, y, Xt, yt = pair(cfg, 30, 23, clauses=60)
    encX = tm.encode(X)
    tm.fit(encX, y, is_X_encoded=True)
    ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    encXt = tm.encode(Xt)
    monkeypatch.setenv("YTM_TRANSFORM_CHUNK", "5")
    np.testing.assert_array_equal(tm.transform(encXt, is_X_encoded=True), ref.transform(encXt))
    ref_pw = ref.transform(encXt, patchwise=True)
    np.testing.assert_array_equal(tm.transform_patchwise(encXt, is_X_encoded=True), ref_pw)
    assert_packed_equal(tm.transform_patchwise(encXt, is_X_encoded=True, packed=True), ref_pw)


def test_score_edge_cases():
    tm, ref, X, y, Xt, yt = pair(3, 30, 20, clauses=40)
    # empty input
    empty = np.zeros((0, tm.number_of_patches, tm.number_of_literal_chunks), dtype=np.uint32)
    assert tm.score(empty, is_X_encoded=True).shape == (0, 10)
    assert tm.transform(empty, is_X_encoded=True).shape == (0, tm.number_of_clauses)
    # fresh model: every clause empty -> class sums are the (zero) bias, transform all ones
    encXt = tm.encode(Xt)
    np.testing.assert_array_equal(tm.score(encXt, is_X_encoded=True), np.zeros((20, 10), dtype=np.float32))
    assert np.all(tm.transform(encXt, is_X_encoded=True) == 1)
    # ragged tail: a batch that is not a multiple of any launch tile
    tm.fit(tm.encode(X), y, is_X_encoded=True)
    ref.fit_encoded(ref.encode(X), ref.encode_y_multiclass(y))
    np.testing.assert_array_equal(tm.score(encXt[:7], is_X_encoded=True), ref.score(encXt[:7]))


def test_one_patch_edge_batches():
    """One patch (the sample-tiled kernels, 64 samples per wave, 256 per block): an empty fit,
    a one-sample fit, and scores / clause outputs for batch sizes on either side of the tile
    edges, where the lanes past the last sample read a clamped sample and discard it."""
    tm, ref, X, y, Xt, yt = pair(2, 40, 300, clauses=30)
    encX, encXt = tm.encode(X), tm.encode(Xt)
    empty = np.zeros((0,) + encX.shape[1:], dtype=np.uint32)
    tm.fit(empty, np.zeros(0, dtype=np.uint32), is_X_encoded=True)
    assert tm.stats()["last_fit_samples"] == 0
    assert_state_equal(tm, ref, "after an empty fit")
    tm.fit(encX[:1], y[:1], is_X_encoded=True)
    ref.fit_encoded(encX[:1], ref.encode_y_multiclass(y[:1]))
    tm.fit(encX, y, is_X_encoded=True)
    ref.fit_encoded(encX, ref.encode_y_multiclass(y))
    assert_state_equal(tm, ref, "after one sample and one epoch")
    assert tm.score(empty, is_X_encoded=True).shape == (0, 10)
    for n in (1, 63, 65, 255, 257, 300):
        np.testing.assert_array_equal(tm.score(encXt[:n], is_X_encoded=True), ref.score(encXt[:n]), err_msg=f"n={n}")
        np.testing.assert_array_equal(tm.transform(encXt[:n], is_X_encoded=True), ref.transform(encXt[:n]),
                                      err_msg=f"n={n}")


# ------------------------------------------------------------------ API surface
def test_api_shapes_dtypes_errors():
    tm, *_ = pair(3, 4, clauses=50)
    X, y, Xt, yt, _ = workloads.make(3, 20, 10)
    tm.fit(X, y)  # raw X path (encodes internally)
    preds, cs = tm.predict(Xt)
    assert preds.shape == (10,) and cs.shape == (10, 10) and cs.dtype == np.float32
    assert tm.get_ta_state().shape == (50, 272) and tm.get_ta_state().dtype == np.uint32
    assert tm.get_weights().shape == (50, 10) and tm.get_weights().dtype == np.float32
    assert tm.get_patch_weights().shape == (50, 361) and tm.get_patch_weights().dtype == np.int32
    assert tm.get_patch_weights().sum() > 0
    with pytest.raises(AssertionError):
        tm.encode(X.astype(np.int64))
    with pytest.raises(AssertionError):
        tm.fit(X, y.reshape(-1, 1))
    with pytest.raises(OverflowError):
        tm.transform_patchwise(_big_view(tm), is_X_encoded=True)


def _big_view(tm):
    # A zero-stride view with more samples than transform_patchwise accepts (no memory used).
    n = np.iinfo(np.uint32).max // (tm.number_of_clauses * tm.number_of_patches) + 1
    base = np.zeros((1, tm.number_of_patches, tm.number_of_literal_chunks), dtype=np.uint32)
    return np.broadcast_to(base, (n,) + base.shape[1:])


@pytest.mark.parametrize("cfg,clauses,opts,want", [
    (2, 300, {}, ([3, 0],)),               # one patch: streaming, then resident
    (4, 40, {}, ([0], [2])),               # several patches: resident or global, as the LDS allows
    (2, 30, dict(coalesced=False), ([],)),  # clause banks: built-in kernels only
])
def test_load_kernels(cfg, clauses, opts, want):
    """load_kernels() loads the training kernels a model's fits choose between; fits after it
    take those kinds and still match the oracle."""
    tm, ref, X, y, *_ = pair(cfg, 30, clauses=clauses, **opts)
    kinds = tm.load_kernels()
    assert kinds in want
    encX = tm.encode(X)
    for _ in range(2):
        tm.fit(encX, y, is_X_encoded=True)
        upd = ref.fit_encoded(encX, ref.encode_y_multiclass(y))
        assert tm.stats()["last_fit_updates"] == upd
        assert tm.stats()["train_kind"] in (kinds or [4])
    assert_state_equal(tm, ref)


def test_non_coalesced_shapes():
    X, y, *_ , kw = workloads.make(2, 50, 1)
    kw.update(number_of_clauses_per_class=6, coalesced=False, seed=3)
    tm = MultiClassTM(**kw)
    tm.fit(X, y)
    assert tm.get_ta_state().shape == (10, 6, 1568)
    assert tm.get_weights().shape == (10, 6, 10)
    w = tm.get_weights()
    for bank in range(10):  # weights outside the own bank stay 0
        assert np.all(np.delete(w[bank], bank, axis=1) == 0)


def test_pickle_roundtrip():
    tm, ref, X, y, Xt, yt = pair(2, 200, 50, clauses=50)
    tm.fit(X, y)
    blob = pickle.dumps(tm)
    tm2 = pickle.loads(blob)
    state = tm.__getstate__()
    assert set(state) == {"args", "state"}
    assert set(state["state"]) == {"ta_state", "clause_weights", "patch_weights", "min_y", "max_y"}
    assert state["state"]["ta_state"].dtype == np.uint32 and state["state"]["ta_state"].ndim == 1
    np.testing.assert_array_equal(tm2.get_ta_state(), tm.get_ta_state())
    np.testing.assert_array_equal(tm2.get_weights(), tm.get_weights())
    np.testing.assert_array_equal(tm2.predict(Xt)[1], tm.predict(Xt)[1])


def test_lzma_checkpoint_continue_training(tmp_path):
    """A model saved the way the reference's examples save one (an LZMA-compressed pickle,
    test/cutm/pneumonia_mnist/pneumonia_mnist.py:119-120), loaded and trained further,
    matches the oracle restarted from the same state (unpickling re-runs __init__, which
    restarts the random stream, base.py:555-558)."""
    import lzma

    tm, ref, X, y, Xt, yt = pair(3, 30, 10, clauses=20)
    encX = tm.encode(X)
    tm.fit(encX, y, is_X_encoded=True)
    path = tmp_path / "model.tm"
    with lzma.LZMAFile(path, "wb") as f:
        pickle.dump(tm, f)
    with lzma.LZMAFile(path, "rb") as f:
        tm2 = pickle.load(f)  # written by this test
    kw = dict(workloads.CONFIGS[3]["model"], number_of_clauses_per_class=20, seed=workloads.MODEL_SEED)
    ref2 = orc.OracleTM(kw.pop("number_of_clauses_per_class"), kw.pop("T"), kw.pop("s"), kw.pop("dim"),
                        kw.pop("n_classes"), **kw)
    ref2.ta[:] = tm.get_ta_state().reshape(ref2.ta.shape)
    ref2.w[:] = tm.get_weights().reshape(ref2.w.shape)
    ref2.pw[:] = tm.get_patch_weights().reshape(ref2.pw.shape)
    for _ in range(2):
        tm2.fit(encX, y, is_X_encoded=True)
        assert tm2.stats()["last_fit_updates"] == ref2.fit_encoded(encX, ref2.encode_y_multiclass(y))
    assert_state_equal(tm2, ref2, "after the checkpoint")


def test_multioutput():
    X, y, Xt, yt, kw = workloads.make(2, 150, 40)
    Y = np.stack([(y == k).astype(np.uint32) for k in range(10)], axis=1)
    kw.update(number_of_clauses_per_class=60, seed=5)
    tm = MultiOutputTM(**kw)
    ref = orc.OracleTM(60, kw["T"], kw["s"], kw["dim"], 10, seed=5)
    tm.fit(X, Y)
    ref.fit_encoded(ref.encode(X), np.where(Y == 1, kw["T"], -kw["T"]).astype(np.int32))
    assert_state_equal(tm, ref)
    preds, cs = tm.predict(Xt)
    np.testing.assert_array_equal(cs, ref.score(ref.encode(Xt)))
    np.testing.assert_array_equal(preds, (cs >= 0).astype(np.uint32))


# ------------------------------------------------------------------ full-size properties
def test_full_config2_epoch_properties():
    """Config 2 at its real size: one epoch in one call equals the same epoch in two calls
    (step continuity across launches), the same seed reproduces it, and the states obey
    0 <= s <= max(256, 128 + K)."""
    X, y, Xt, yt, kw = workloads.make(2)
    kw["seed"] = workloads.MODEL_SEED
    a = MultiClassTM(**kw)
    b = MultiClassTM(**kw)
    encX = a.encode(X)
    a.fit(encX, y, is_X_encoded=True)
    b.fit(encX[:25000], y[:25000], is_X_encoded=True)
    b.fit(encX[25000:], y[25000:], is_X_encoded=True)
    ta = a.get_ta_state()
    np.testing.assert_array_equal(ta, b.get_ta_state())
    np.testing.assert_array_equal(a.get_weights(), b.get_weights())
    assert ta.max() <= 256
    acc = (a.predict(Xt)[0] == yt).mean()
    print(f"config 2 after 1 epoch: test accuracy {acc:.4f}")
    assert acc > 0.5
