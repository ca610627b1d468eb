"""The C oracle against the independent pure-Python restatement (tests/pyref.py) on
small shapes: encode, inference, transform and training (counter and injected streams),
across the variant flags of src/cutm/base.py:16-29."""
import numpy as np
import pytest

import pyref

CASES = {
    # name: (clauses_per_class, K, T, s, dim, patch_dim, extra opts)
    "vanilla": (4, 2, 6, 3.9, (7, 1, 1), (7, 1), {}),
    "vanilla_int_s": (3, 3, 5, 2, (10, 1, 1), (10, 1), {}),
    "conv": (4, 3, 8, 2.5, (5, 4, 1), (2, 3), {}),
    "conv_channels": (3, 2, 7, 4.0, (4, 4, 2), (2, 2), {}),
    "banks": (2, 3, 5, 3.0, (6, 1, 1), (6, 1), {"coalesced": False}),
    "pos_polarity": (3, 2, 5, 2.0, (6, 1, 1), (6, 1), {"negative_polarity": False, "init_neg_weights": False}),
    "maxinc": (3, 2, 6, 2.0, (5, 3, 1), (3, 2), {"max_included_literals": 3}),
    "no_negated": (3, 2, 5, 3.0, (6, 1, 1), (6, 1), {"append_negated": False}),
    "no_loc": (3, 2, 6, 3.0, (5, 5, 1), (3, 3), {"encode_loc": False}),
    "small_states": (3, 4, 6, 2.0, (6, 1, 1), (6, 1), {"number_of_ta_states": 8}),
    "q_int": (3, 4, 6, 2.0, (6, 1, 1), (6, 1), {"q": 2}),
}


def build(oracle_mod, name, seed=11):
    cpc, K, T, s, dim, pdim, opts = CASES[name]
    om = oracle_mod.OracleTM(cpc, T, s, dim, K, patch_dim=pdim, seed=seed, **opts)
    q = min(opts.get("q", 1.0), float(K))
    pm = pyref.PyTM(om.C, K, T, oracle_mod.s_inv_of(s), oracle_mod.q_prob_of(q, K), dim, pdim,
                    n_states=opts.get("number_of_ta_states", 256), maxinc=opts.get("max_included_literals"),
                    append_negated=opts.get("append_negated", True), encode_loc=opts.get("encode_loc", True),
                    coalesced=opts.get("coalesced", True), negative_polarity=opts.get("negative_polarity", True),
                    init_neg_weights=opts.get("init_neg_weights", True), seed=seed)
    return om, pm


def data(om, N, seed, density=0.5):
    rng = np.random.default_rng(seed)
    F = om.p.dim0 * om.p.dim1 * om.p.dim2
    X = (rng.random((N, F)) < density).astype(np.uint32) * rng.integers(1, 5, (N, F)).astype(np.uint32)
    y = rng.integers(0, om.K, N)
    return X, y


@pytest.mark.parametrize("name", sorted(CASES))
def test_encode(oracle_mod, name):
    om, pm = build(oracle_mod, name)
    X, _ = data(om, 6, 1)
    np.testing.assert_array_equal(om.encode(X), pm.encode(X))


@pytest.mark.parametrize("name", sorted(CASES))
def test_initial_weights(oracle_mod, name):
    om, pm = build(oracle_mod, name)
    np.testing.assert_array_equal(om.w, pm.w_array())


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("mode", ["counter", "inject"])
def test_fit_score_transform(oracle_mod, name, mode):
    om, pm = build(oracle_mod, name)
    X, y = data(om, 12, 2)
    encX = om.encode(X)
    encY = om.encode_y_multiclass(y)
    rng = np.random.default_rng(3)
    drop = (rng.random(om.C) < 0.25).astype(np.uint32) if name in ("vanilla", "conv") else None
    for epoch in range(3):
        inj = None
        if mode == "inject":
            block = om.C * om.P + 2 * om.C * om.K + om.C * om.K * om.L
            inj = rng.random(len(encX) * block).astype(np.float32)
            # exercise the comparison edges: exact 1.0 (reservoir rejects), exact S_INV
            inj[:: 17] = 1.0
            inj[5:: 23] = np.float32(oracle_mod.s_inv_of(CASES[name][3]))
        u1 = om.fit_encoded(encX, encY, drop=drop, inject=inj)
        u2 = pm.fit(encX, encY, drop=drop, inject=inj)
        assert u1 == u2
        np.testing.assert_array_equal(om.ta, pm.ta_array(), err_msg=f"epoch {epoch}")
        np.testing.assert_array_equal(om.w, pm.w_array())
        np.testing.assert_array_equal(om.pw, pm.pw_array())
    np.testing.assert_array_equal(om.score(encX), pm.score(encX))
    np.testing.assert_array_equal(om.transform(encX), pm.transform(encX))
    np.testing.assert_array_equal(om.transform(encX, True), pm.transform(encX, True))
