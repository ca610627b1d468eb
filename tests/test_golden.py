"""The committed golden fixtures (tests/golden/fixtures.json, written by
tests/golden/make_fixtures.py): seeded workload fingerprints and small end-to-end vectors.

CPU: the workload generators and the C oracle still produce them.  GPU: the HIP path
produces the same bytes (encoded samples, TA states, weights, patch weights, class sums,
clause outputs and update counts) without consulting the oracle."""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import workloads

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_fixtures  # noqa: E402

FIX = json.loads((GOLDEN / "fixtures.json").read_text())


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("cfg", sorted(FIX["workloads"]))
def test_workload_fingerprints(cfg):
    X, y, Xt, yt, _ = workloads.make(int(cfg), 64, 64)
    want = FIX["workloads"][cfg]
    assert sha(X.astype(np.uint32)) == want["X64"]
    assert sha(y.astype(np.uint32)) == want["y64"]
    assert sha(Xt.astype(np.uint32)) == want["Xt64"]
    assert sha(yt.astype(np.uint32)) == want["yt64"]


@pytest.mark.parametrize("key", sorted(FIX["cases"]))
def test_oracle_matches_fixtures(key, oracle_mod):
    c = FIX["cases"][key]
    got = make_fixtures.oracle_case(c["config"], c["n_train"], c["n_test"], c["clauses"], c["epochs"])
    for field, value in got.items():
        assert value == c[field], field


@pytest.mark.gpu
@pytest.mark.parametrize("key", sorted(FIX["cases"]))
def test_gpu_matches_fixtures(monkeypatch, key):
    monkeypatch.setenv("YTM_JIT", "2")
    from ytm_amd import MultiClassTM

    c = FIX["cases"][key]
    X, y, Xt, yt, _ = workloads.make(c["config"], c["n_train"], c["n_test"])
    tm = MultiClassTM(**make_fixtures.case_kwargs(c["config"], c["clauses"]))
    encX = tm.encode(X)
    assert sha(encX) == c["encoded_X"]
    updates = []
    for _ in range(c["epochs"]):
        tm.fit(encX, y, is_X_encoded=True)
        updates.append(int(tm.stats()["last_fit_updates"]))
    assert updates == c["updates"]
    assert sha(tm.get_ta_state().reshape(tm.number_of_clauses, -1)) == c["ta_state"]
    assert sha(tm.get_weights().reshape(tm.number_of_clauses, -1)) == c["clause_weights"]
    assert sha(tm.get_patch_weights().reshape(tm.number_of_clauses, -1)) == c["patch_weights"]
    encXt = tm.encode(Xt)
    _, cs = tm.predict(encXt, is_X_encoded=True)
    assert sha(cs.astype(np.float32)) == c["class_sums"]
    assert sha(tm.transform(encXt, is_X_encoded=True).astype(np.uint32)) == c["clause_outputs"]
