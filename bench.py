"""Benchmark of the YTM Tsetlin Machine hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-extra] [--no-cpu]

A step is one training epoch (one fit() pass over the whole training set, samples in
order, data resident in HBM).  W untimed epochs, then K timed epochs of the headline
configuration (BASELINE.json's config 2 by default: MNIST-shaped, 2000 clauses, 10 classes,
49 words), then inference over its test set.  The other four configurations follow at their
full sizes under "configs" (config 1: one untimed epoch, then its 10 epochs; configs 3-5: one untimed and two timed
epochs), each with the C oracle's CPU rate beside it.  Prints ONE JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# VALU 32-bit lane-ops per second: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz (MI355X).
VALU_PEAK_T = 256 * 4 * 16 * 2.4e9 / 1e12
# Epochs of the configurations run after the headline one: (untimed, timed).
EXTRA_EPOCHS = {1: (1, 10), 2: (1, 3), 3: (1, 2), 4: (1, 2), 5: (1, 2)}
KIND_NAMES = {0: "resident", 1: "global one-patch", 2: "global several-patch", 3: "streaming"}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def train_bytes(tm, samples: int, updates: int) -> float:
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
        d = json.loads(path.read_text())
        return {"bytes_per_launch": float(d["bytes_per_launch"]), "kernel": d.get("kernel"),
                "hbm_gbs": d.get("hbm_gbs")}
    except (KeyError, ValueError):
        return None


def load_counters(config: int):
    """SQ counters of the training kernel (rocprofv3 --pmc, committed summary): VALU busy,
    instructions per sample, LDS bank conflicts; or None."""
    path = ROOT / "profiles" / f"train_cfg{config}_counters.json"
    if not path.exists():
        return None
    try:
        d = json.loads(path.read_text())
        return {k: d[k] for k in ("kernel", "valu_busy", "valu_insts_per_sample", "salu_per_valu",
                                  "lds_bank_conflict", "wait_frac")}
    except (KeyError, ValueError):
        return None


def cpu_info() -> dict:
    model = platform.processor() or "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


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


def encode_in_chunks(tm, make_chunk, n: int, chunk: int) -> np.ndarray:
    """Encoded samples (n, P, W) on the host, the raw inputs generated and encoded chunk by
    chunk (the full raw array of config 4 is 4.9 GB of uint32)."""
    out = np.empty((n, tm.number_of_patches, tm.number_of_literal_chunks), dtype=np.uint32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        out[s:e] = tm.encode(make_chunk(s, e))
    return out


def cpu_baseline(cfg: int, kw: dict, encX, y, encXt, budget_s: float) -> dict:
    """The C oracle (a CPU restatement of the reference semantics, oracle/ytm_oracle.c)
    training on a prefix of the same workload from the same initial state, then scoring a
    prefix of the test set, on this host's cores (OpenMP)."""
    from oracle import oracle as orc

    info = cpu_info()
    threads = min(16, info["nproc"] or 1)
    orc.set_threads(threads)
    ref = orc.OracleTM(kw["number_of_clauses_per_class"], kw["T"], kw["s"], kw["dim"], kw["n_classes"],
                       patch_dim=kw.get("patch_dim"), seed=kw["seed"])
    encY = ref.encode_y_multiclass(y)
    # consecutive chunks of epoch 1 (the oracle's step counter carries across calls, so this
    # is the same computation as one fit over the prefix) until the budget is spent
    t0 = time.perf_counter()
    n, chunk = 0, 8
    while n < encX.shape[0] and time.perf_counter() - t0 < budget_s:
        m = min(chunk, encX.shape[0] - n)
        ref.fit_encoded(encX[n:n + m], encY[n:n + m])
        n += m
        chunk = min(2 * chunk, 2048)
    train_s = time.perf_counter() - t0
    nt = min(encXt.shape[0], 1000)
    t1 = time.perf_counter()
    ref.score(encXt[:nt])
    infer_s = time.perf_counter() - t1
    return {
        "value": round(n / train_s, 1),
        "unit": "train samples/s",
        "cores": threads,
        "kind": "port",
        "infer_samples_per_s": round(nt / infer_s, 1),
        "nproc": info["nproc"],
        "cpu_model": info["cpu_model"],
        "sample": f"config {cfg}: first {n} training samples of epoch 1 (fresh model, same seed) in {train_s:.1f} s, "
                  f"then {nt} test samples scored, on {threads} OpenMP threads of {info['nproc']}; "
                  f"C oracle oracle/ytm_oracle.c",
    }


def run_config(cfg: int, warmup: int, steps: int, cpu_seconds: float, n_train=None, n_test=None) -> dict:
    import workloads
    from ytm_amd import MultiClassTM

    t0 = time.perf_counter()
    c = workloads.CONFIGS[cfg]
    kw = dict(c["model"], seed=workloads.MODEL_SEED)
    tm = MultiClassTM(**kw)
    if cfg == 4 and n_train is None and n_test is None:
        # the values of workloads.make(4), generated and encoded in chunks
        gen = workloads.CifarStream(c["n_train"], c["n_test"])
        encX = encode_in_chunks(tm, gen.train_rows, c["n_train"], 2048)
        enc_ms = tm.stats()["last_encode_kernel_ms"]
        encXt = encode_in_chunks(tm, gen.test_rows, c["n_test"], 2048)
        y, yt = gen.y, gen.yt
    else:
        X, y, Xt, yt, _ = workloads.make(cfg, n_train, n_test)
        encX = tm.encode(X)
        enc_ms = tm.stats()["last_encode_kernel_ms"]
        encXt = tm.encode(Xt)
        del X, Xt
    dtrain = tm.device_data(encX, y, is_X_encoded=True)
    dtest = tm.device_data(encXt, is_X_encoded=True)
    N, Nt = encX.shape[0], encXt.shape[0]
    log(f"[bench] config {cfg}: {N} / {Nt} samples generated, encoded and resident in {time.perf_counter() - t0:.1f}s")
    # Every training kernel this model may switch to between epochs is compiled and loaded for
    # it here, once (as the reference compiles per model in BaseTM.__init__), not inside a
    # timed epoch.
    t1 = time.perf_counter()
    kinds = tm.load_kernels()
    log(f"[bench] config {cfg}: training kernels {kinds} compiled and loaded in {time.perf_counter() - t1:.1f}s")

    epochs = []
    for e in range(warmup + steps):
        t = time.perf_counter()
        tm.fit_device(dtrain)
        wall = time.perf_counter() - t
        st = tm.stats()
        ep = dict(wall_s=wall, kernel_ms=st["last_fit_kernel_ms"], launches=st["last_fit_launches"],
                  updates=st["last_fit_updates"], feedback=st["last_fit_feedback_samples"],
                  evals=st["last_fit_evaluations"], wait=st["last_fit_wait_frac"], kind=st["train_kind"],
                  wgs=st["train_workgroups"], phase=st["last_fit_phase_us"])
        epochs.append(ep)
        log(f"[bench] config {cfg} epoch {e + 1}{' (timed)' if e >= warmup else ''}: wall {wall:.3f}s "
            f"kernel {ep['kernel_ms']:.1f}ms updates {ep['updates']} ({ep['updates'] / N:.2f}/sample) "
            f"feedback samples {ep['feedback']} evaluations {ep['evals']} workgroups {ep['wgs']} "
            f"kernel {KIND_NAMES.get(ep['kind'], ep['kind'])} wait {ep['wait']:.3f}")
        if os.environ.get("YTM_TRAIN_PROFILE") == "4":
            d = st["last_fit_draws"]
            log(f"[bench]   counter-stream words per sample (lane draw sites): reservoir {d[0] / N:.0f} "
                f"q-skip/update {d[1] / N:.0f} literal {d[2] / N:.0f}")
        elif os.environ.get("YTM_TRAIN_PROFILE"):
            names = {0: ("exchange", "barrier", "D1", "barrier", "D2", "D3+re-eval", "barrier", "step1-slowest-wave"),
                     3: ("stream", "drain", "decide", "apply", "first-row")}.get(
                         ep["kind"], ("stage", "publish+exchange", "next-A-wait", "decide", "apply", "re-eval"))
            log("[bench]   phase us/sample (wave 0): " + " ".join(f"{n} {v:.2f}" for n, v in zip(names, ep["phase"])))
            if ep["kind"] == 3 and ep["feedback"]:
                log("[bench]   per stop, us: " + " ".join(f"{n} {v * N / ep['feedback']:.2f}"
                                                       for n, v in zip(names[1:], ep["phase"][1:5])))
    timed = epochs[warmup:]

    # inference over the test set (resident), best of 3 after one warm call
    cs = tm.score_device(dtest)
    inf = []
    for _ in range(3):
        t = time.perf_counter()
        cs = tm.score_device(dtest)
        inf.append((time.perf_counter() - t, tm.stats()["last_score_kernel_ms"]))
    inf_wall, inf_kern = min(inf)
    acc = float((np.argmax(cs, axis=1) == yt).mean())
    dtrain.release()
    dtest.release()

    kern_s = sum(e["kernel_ms"] for e in timed) / 1e3
    wall_s = sum(e["wall_s"] for e in timed)
    launches = sum(e["launches"] for e in timed)
    upd = sum(e["updates"] for e in timed)
    byts = sum(train_bytes(tm, N, e["updates"]) for e in timed)
    achieved = byts / kern_s / 1e9  # bytes per launch / average launch time
    last = timed[-1]
    res = {
        "workload": c["name"],
        "train_samples": N,
        "test_samples": Nt,
        "clauses": tm.number_of_clauses,
        "classes": tm.number_of_outputs,
        "literal_words": tm.number_of_literal_chunks,
        "patches": tm.number_of_patches,
        "epochs": {"untimed": warmup, "timed": steps},
        "train_samples_per_s": round(N * steps / wall_s, 1),
        "train_kernel_samples_per_s": round(N * steps / kern_s, 1),
        "epoch1_train_kernel_samples_per_s": round(N / (epochs[0]["kernel_ms"] / 1e3), 1),
        "last_epoch_train_kernel_samples_per_s": round(N / (last["kernel_ms"] / 1e3), 1),
        "infer_samples_per_s": round(Nt / inf_wall, 1),
        "infer_kernel_samples_per_s": round(Nt / (inf_kern / 1e3), 1),
        "encode_samples_per_s": round(N / (enc_ms / 1e3), 1) if enc_ms else None,
        "updates_per_sample": round(upd / (N * steps), 3),
        "test_accuracy": round(acc, 4),
        "train_kernel": KIND_NAMES.get(last["kind"], last["kind"]),
        "train_workgroups": last["wgs"],
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "U_s": round(upd / (N * steps), 3),
            "bytes_per_launch": round(byts / max(1, launches), 1),
        },
        # what actually binds the training kernel: the share of its time spent waiting for
        # class sums, and how many samples needed a feedback pass
        "binding": {
            "class_sum_wait_fraction": round(sum(e["wait"] for e in timed) / len(timed), 4),
            "feedback_sample_fraction": round(sum(e["feedback"] for e in timed) / (N * steps), 4),
            "evaluations_per_sample": round(sum(e["evals"] for e in timed) / (N * steps), 3),
        },
        "infer_roofline": {
            "bound": "valu",
            "achieved": round(infer_word_ands(tm, Nt) / (inf_kern / 1e3) / 1e12, 3),
            "peak": round(VALU_PEAK_T, 2),
            "unit": "T word-ANDs/s (C*P*W 32-bit lane-ops per sample, no early exit)",
            "frac": round(infer_word_ands(tm, Nt) / (inf_kern / 1e3) / 1e12 / VALU_PEAK_T, 4),
            "hbm_gbs": round(infer_bytes(tm, Nt) / (inf_kern / 1e3) / 1e9, 2),
        },
        "_ms_per_step": 1e3 * wall_s / steps,
    }
    traffic = load_traffic(cfg)
    if traffic:
        res["roofline"]["traffic"] = traffic["bytes_per_launch"]
        res["roofline"]["traffic_kernel"] = traffic["kernel"]
        if traffic["hbm_gbs"] is not None:
            # the measured bytes of that launch over its own duration: the share of the HBM
            # peak the kernel really uses (the byte model above counts reads it never makes)
            res["roofline"]["traffic_gbs"] = traffic["hbm_gbs"]
            res["roofline"]["traffic_frac"] = round(traffic["hbm_gbs"] / HBM_PEAK_GBS, 4)
    counters = load_counters(cfg)
    if counters:
        # measured instruction mix of the same kernel (epoch 2): how busy its execution units are
        res["binding"]["counters"] = counters
    tm.release()
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_baseline(cfg, kw, encX, y, encXt, cpu_seconds)
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--n-train", type=int, default=None)
    ap.add_argument("--n-test", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-oracle budget per configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the headline configuration")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the training path is "
              "single-GPU by design, see DESIGN.md for how it would shard.", file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)

    cpu = 0.0 if args.no_cpu else args.cpu_seconds
    cfg = args.config
    head = run_config(cfg, args.warmup, args.steps, cpu, args.n_train, args.n_test)
    configs = {str(cfg): head}
    if not args.no_extra:
        for other in (1, 2, 3, 4, 5):
            if other != cfg:
                w, s = EXTRA_EPOCHS[other]
                configs[str(other)] = run_config(other, w, s, cpu)

    import workloads

    kw = workloads.CONFIGS[cfg]["model"]
    out = {
        "metric": "train & infer samples/sec on 1 MI355X; % of HBM-bandwidth roofline",
        "value": head["train_samples_per_s"],
        "unit": "train samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["_ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (seeded generators, workloads.py)",
        "config": {
            "workload": head["workload"],
            "bench_config": cfg,
            "train_samples": head["train_samples"],
            "test_samples": head["test_samples"],
            "clauses": head["clauses"],
            "classes": head["classes"],
            "literal_words": head["literal_words"],
            "patches": head["patches"],
            "T": kw["T"],
            "s": kw["s"],
            "step": "one training epoch (fit over all training samples, in order)",
        },
        "infer_samples_per_s": head["infer_samples_per_s"],
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "configs": {k: {kk: vv for kk, vv in v.items() if not kk.startswith("_")} for k, v in configs.items()},
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    rc = main()
    if rc:
        sys.exit(rc)
