"""Writes tests/golden/fixtures.json: fingerprints of the seeded synthetic workloads and
small end-to-end vectors (state after training, class sums, clause outputs) computed by
the C oracle for each benchmark configuration at a reduced size.

    python tests/golden/make_fixtures.py

The fixtures freeze the oracle's behaviour: tests/test_golden.py checks the oracle (CPU)
and the HIP path (GPU) against them.  They are regression vectors of this build's own
restatement; the reference ships no golden vectors for this path.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import workloads  # noqa: E402

OUT = Path(__file__).resolve().parent / "fixtures.json"

# (config, train samples, test samples, clauses per class, epochs)
CASES = [(1, 300, 100, None, 2), (2, 40, 20, 30, 2), (3, 12, 6, 20, 1), (4, 3, 2, 8, 1), (5, 20, 10, 12, 2)]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def case_kwargs(cfg: int, clauses):
    kw = dict(workloads.CONFIGS[cfg]["model"])
    if clauses is not None:
        kw["number_of_clauses_per_class"] = clauses
    kw["seed"] = workloads.MODEL_SEED
    return kw


def oracle_case(cfg, n_train, n_test, clauses, epochs):
    from oracle import oracle as orc

    X, y, Xt, yt, _ = workloads.make(cfg, n_train, n_test)
    kw = case_kwargs(cfg, clauses)
    ref = orc.OracleTM(kw.pop("number_of_clauses_per_class"), kw.pop("T"), kw.pop("s"), kw.pop("dim"),
                       kw.pop("n_classes"), **kw)
    encX = ref.encode(X)
    encY = ref.encode_y_multiclass(y)
    updates = [int(ref.fit_encoded(encX, encY)) for _ in range(epochs)]
    encXt = ref.encode(Xt)
    return {
        "encoded_X": sha(encX),
        "updates": updates,
        "ta_state": sha(ref.ta.astype(np.uint32)),
        "clause_weights": sha(ref.w.astype(np.float32)),
        "patch_weights": sha(ref.pw.astype(np.int32)),
        "class_sums": sha(ref.score(encXt).astype(np.float32)),
        "clause_outputs": sha(ref.transform(encXt).astype(np.uint32)),
    }


def main() -> None:
    from oracle import oracle as orc

    orc.set_threads(8)
    out = {"workloads": {}, "cases": {}}
    for cfg, spec in workloads.CONFIGS.items():
        X, y, Xt, yt, _ = workloads.make(cfg, 64, 64)
        out["workloads"][str(cfg)] = {"X64": sha(X.astype(np.uint32)), "y64": sha(y.astype(np.uint32)),
                                      "Xt64": sha(Xt.astype(np.uint32)), "yt64": sha(yt.astype(np.uint32))}
    for cfg, n_train, n_test, clauses, epochs in CASES:
        key = f"cfg{cfg}"
        out["cases"][key] = {"config": cfg, "n_train": n_train, "n_test": n_test, "clauses": clauses,
                             "epochs": epochs, **oracle_case(cfg, n_train, n_test, clauses, epochs)}
        print(key, out["cases"][key]["updates"], flush=True)
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
