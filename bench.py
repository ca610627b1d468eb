"""Benchmark of the YTM Tsetlin Machine hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2]

A step is one training epoch (one fit() pass over the whole training set, samples in
order, data resident in HBM).  W untimed epochs, then K timed epochs; then inference
over the test set.  Prints ONE JSON line on stdout.  The default workload is
configuration 2 of BASELINE.json (MNIST-shaped, 2000 clauses, 10 classes, 49 words).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# VALU 32-bit lane-ops per second: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz (MI355X).
VALU_PEAK_T = 256 * 4 * 16 * 2.4e9 / 1e12


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def train_bytes_per_launch(tm, samples: int, updates: int) -> float:
    """Algorithmic HBM bytes of training: every TA state read once at 2 B, every weight at
    4 B, per sample; clauses that ran a feedback branch write their TA row and weights
    back; each sample's literals are read once:  B = (N*C + U)(2L + 4K) + N*4*P*W."""
    C, K, L = tm.number_of_clauses, tm.number_of_outputs, tm.number_of_literals
    P, W = tm.number_of_patches, tm.number_of_literal_chunks
    return float((samples * C + updates) * (2 * L + 4 * K) + samples * 4 * P * W)


def infer_word_ands(tm, samples: int) -> float:
    """Inference VALU work: every clause tested on every patch, C*P*W word-ANDs per sample."""
    return float(samples) * tm.number_of_clauses * tm.number_of_patches * tm.number_of_literal_chunks


def infer_bytes(tm, samples: int) -> float:
    return float(samples * (4 * tm.number_of_patches * tm.number_of_literal_chunks + 4 * tm.number_of_outputs))


def load_traffic(config: int):
    """HBM bytes per training-kernel launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (committed summary), or None."""
    path = ROOT / "profiles" / f"train_cfg{config}_traffic.json"
    if not path.exists():
        return None
    try:
        return float(json.loads(path.read_text())["bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def copy_calibration(mib: int) -> None:
    """One device-to-device copy of `mib` MiB (HIP's blit kernel), outside any timed region:
    under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch, against the known
    mib * 1024 KiB, scale the counters read for the training kernel to bytes."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    n = ctypes.c_size_t(mib << 20)
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(ctypes.byref(p), n) != 0:
            raise RuntimeError("hipMalloc failed in the copy calibration")
    try:
        if hip.hipMemset(src, 1, n) or hip.hipMemset(dst, 0, n) or hip.hipDeviceSynchronize():
            raise RuntimeError("hipMemset failed in the copy calibration")
        if hip.hipMemcpy(dst, src, n, 3) or hip.hipDeviceSynchronize():  # 3 = device to device
            raise RuntimeError("hipMemcpy failed in the copy calibration")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    log(f"[bench] copy calibration: {mib} MiB device-to-device")


def cpu_baseline(encX, y, kw, budget_s: float):
    """The C oracle (a CPU restatement of the reference semantics) training on a bounded
    prefix of the same workload, from the same initial state, on this host's cores."""
    from oracle import oracle as orc

    threads = min(16, os.cpu_count() or 1)
    orc.set_threads(threads)
    ref = orc.OracleTM(kw["number_of_clauses_per_class"], kw["T"], kw["s"], kw["dim"], kw["n_classes"],
                       patch_dim=kw.get("patch_dim"), seed=kw["seed"])
    encY = ref.encode_y_multiclass(y)
    # consecutive chunks of the epoch (the oracle's step counter carries across calls, so
    # this is the same computation as one fit over the prefix) until the budget is spent
    t0 = time.perf_counter()
    n, chunk = 0, 32
    while n < encX.shape[0] and time.perf_counter() - t0 < budget_s:
        m = min(chunk, encX.shape[0] - n)
        ref.fit_encoded(encX[n:n + m], encY[n:n + m])
        n += m
        chunk = min(2 * chunk, 2048)
    total = time.perf_counter() - t0
    return {
        "value": n / total,
        "unit": "train samples/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {n} training samples of epoch 1 (fresh model, same seed), "
                  f"{total:.1f} s on {threads} threads; C oracle oracle/ytm_oracle.c",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--n-train", type=int, default=None)
    ap.add_argument("--n-test", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the training path is "
              "single-GPU by design, see DESIGN.md for how it would shard.", file=sys.stderr)
        return 2

    import workloads
    from ytm_amd import MultiClassTM

    if args.copy_calibration:
        copy_calibration(args.copy_calibration)

    cfg = args.config
    t0 = time.perf_counter()
    X, y, Xt, yt, kw = workloads.make(cfg, args.n_train, args.n_test)
    kw["seed"] = workloads.MODEL_SEED
    log(f"[bench] config {cfg} data {X.shape} / {Xt.shape} generated in {time.perf_counter() - t0:.1f}s")
    tm = MultiClassTM(**kw)
    encX = tm.encode(X)
    enc_ms = tm.stats()["last_encode_kernel_ms"]
    encXt = tm.encode(Xt)
    dtrain = tm.device_data(encX, y, is_X_encoded=True)
    dtest = tm.device_data(encXt, is_X_encoded=True)
    N, Nt = encX.shape[0], encXt.shape[0]

    epoch1 = None
    for w in range(args.warmup):
        t = time.perf_counter()
        tm.fit_device(dtrain)
        st = tm.stats()
        log(f"[bench] warmup epoch {w + 1}: {time.perf_counter() - t:.3f}s kernel {st['last_fit_kernel_ms']:.1f}ms "
            f"updates {st['last_fit_updates']}")
        if w == 0:
            epoch1 = N / (st["last_fit_kernel_ms"] / 1e3)

    walls, kern, byts, launches, upd = [], [], [], 0, 0
    for s in range(args.steps):
        t = time.perf_counter()
        tm.fit_device(dtrain)
        walls.append(time.perf_counter() - t)
        st = tm.stats()
        kern.append(st["last_fit_kernel_ms"])
        launches += st["last_fit_launches"]
        upd += st["last_fit_updates"]
        byts.append(train_bytes_per_launch(tm, N, st["last_fit_updates"]))
        log(f"[bench] step {s + 1}: wall {walls[-1]:.3f}s kernel {kern[-1]:.1f}ms updates {st['last_fit_updates']} "
            f"({st['last_fit_updates'] / N:.1f}/sample) workgroups {st['train_workgroups']} "
            f"kind {st['train_kind']} wait {st['last_fit_wait_frac']:.3f} "
            f"feedback samples {st['last_fit_feedback_samples']} evaluations {st['last_fit_evaluations']}")
        if os.environ.get("YTM_TRAIN_PROFILE"):
            names = {0: ("exchange", "barrier", "D1", "barrier", "D2", "D3+re-eval", "barrier", "step1-slowest-wave"),
                     3: ("stream", "drain", "decide", "apply")}.get(
                         st["train_kind"], ("A", "barrier", "exchange", "barrier", "D", "barrier"))
            log("[bench]   phase us/sample (wave 0): "
                + " ".join(f"{n} {v:.2f}" for n, v in zip(names, st["last_fit_phase_us"])))

    # inference over the test set (resident), best of 3 after one warm call
    cs = tm.score_device(dtest)
    inf = []
    for _ in range(3):
        t = time.perf_counter()
        cs = tm.score_device(dtest)
        inf.append((time.perf_counter() - t, tm.stats()["last_score_kernel_ms"]))
    inf_wall, inf_kern = min(inf)
    acc = float((np.argmax(cs, axis=1) == yt).mean())
    log(f"[bench] test accuracy after {args.warmup + args.steps} epochs: {acc:.4f}")

    # PCIe-inclusive rate: one more epoch through fit() from host arrays (upload + train),
    # after the timed region and the inference above
    t = time.perf_counter()
    tm.fit(encX, y, is_X_encoded=True)
    host_wall = time.perf_counter() - t

    total_wall = sum(walls)
    value = N * args.steps / total_wall
    avg_launch_s = sum(kern) / 1e3 / max(1, launches)
    bytes_per_launch = sum(byts) / max(1, launches)
    achieved = bytes_per_launch / avg_launch_s / 1e9
    out = {
        "metric": "train & infer samples/sec on 1 MI355X; % of HBM-bandwidth roofline",
        "value": round(value, 1),
        "unit": "train samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * total_wall / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (seeded generator, workloads.py)",
        "config": {
            "workload": workloads.CONFIGS[cfg]["name"],
            "bench_config": cfg,
            "train_samples": N,
            "test_samples": Nt,
            "clauses": tm.number_of_clauses,
            "classes": tm.number_of_outputs,
            "literals": tm.number_of_literals,
            "literal_words": tm.number_of_literal_chunks,
            "patches": tm.number_of_patches,
            "T": kw["T"],
            "s": kw["s"],
            "step": "one training epoch (fit over all training samples, in order)",
        },
        "infer_samples_per_s": round(Nt / inf_wall, 1),
        "infer_kernel_samples_per_s": round(Nt / (inf_kern / 1e3), 1),
        "train_kernel_samples_per_s": round(N * args.steps / (sum(kern) / 1e3), 1),
        "train_samples_per_s_from_host_buffers": round(N / host_wall, 1),
        "epoch1_train_kernel_samples_per_s": round(epoch1, 1) if epoch1 else None,
        "encode_samples_per_s": round(N / (enc_ms / 1e3), 1) if enc_ms else None,
        "updates_per_sample": round(upd / (N * args.steps), 2),
        "test_accuracy": round(acc, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(cfg),
        },
        "infer_roofline": {
            "bound": "valu",
            "achieved": round(infer_word_ands(tm, Nt) / (inf_kern / 1e3) / 1e12, 3),
            "peak": round(VALU_PEAK_T, 2),
            "unit": "T word-ANDs/s (C*P*W 32-bit lane-ops per sample, no early exit)",
            "frac": round(infer_word_ands(tm, Nt) / (inf_kern / 1e3) / 1e12 / VALU_PEAK_T, 4),
            "hbm_gbs": round(infer_bytes(tm, Nt) / (inf_kern / 1e3) / 1e9, 2),
        },
        "cpu_baseline": None,
    }
    out["train_wait_fraction"] = round(tm.stats()["last_fit_wait_frac"], 4)
    dtrain.release()
    dtest.release()
    tm.release()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(encX, y, kw, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    rc = main()
    if rc:
        sys.exit(rc)
