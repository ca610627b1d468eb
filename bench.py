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
import hashlib
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
# Training samples of epoch 1 that the CPU baseline trains (None: the whole epoch), fixed so
# that runs compare; 1000 test samples are scored.
CPU_PREFIX = {1: None, 2: None, 3: 2000, 4: 1000, 5: 1000}
# Sources of the training kernels: a committed rocprofv3 summary records their hash, and is
# reported only while it matches.
KERNEL_SOURCES = ("ytm_amd/csrc/ytm_train.h", "ytm_amd/csrc/ytm_device.h", "ytm_amd/csrc/ytm_types.h",
                  "ytm_amd/csrc/ytm_kernels.hip", "ytm_amd/csrc/ytm_api.hip")


def kernel_source_hash() -> str:
    h = hashlib.sha256()
    for f in KERNEL_SOURCES:
        h.update((ROOT / f).read_bytes())
    return h.hexdigest()[:16]


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


def load_profile(name: str):
    """A committed rocprofv3 summary (profiles/<name>.json), or None when it is absent, or
    measured on kernel sources other than the current ones (its source_sha16 differs)."""
    path = ROOT / "profiles" / f"{name}.json"
    if not path.exists():
        return None
    try:
        d = json.loads(path.read_text())
    except ValueError:
        return None
    if d.get("source_sha16") != kernel_source_hash():
        log(f"[bench] profiles/{name}.json was measured on other kernel sources: not reported")
        return None
    return d


def load_traffic(config: int):
    """HBM bytes per training-kernel launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE (committed summary of the timed epochs), or None."""
    d = load_profile(f"train_cfg{config}_traffic")
    try:
        return None if d is None else {"bytes_per_launch": float(d["bytes_per_launch"]), "kernel": d.get("kernel"),
                                       "hbm_gbs": d.get("hbm_gbs"), "epochs": d.get("epochs")}
    except (KeyError, ValueError):
        return None


def load_counters(config: int):
    """SQ counters of the training kernel (rocprofv3 --pmc, committed summary of the timed
    epochs): VALU busy, instructions per sample, LDS bank conflicts; or None."""
    d = load_profile(f"train_cfg{config}_counters")
    try:
        return None if d is None else {k: d[k] for k in ("kernel", "epochs", "valu_busy", "valu_insts_per_sample",
                                                         "salu_per_valu", "lds_bank_conflict", "wait_frac")}
    except KeyError:
        return None


def _load_state(tm, ta, w) -> None:
    tm.load_state_dict({"state": {"ta_state": ta, "clause_weights": w,
                                  "patch_weights": np.zeros((tm.number_of_clauses, tm.number_of_patches), np.int32),
                                  "min_y": None, "max_y": None}})


def floor_us(kw: dict, mode: str, n: int):
    """Microseconds per sample that the training kernel of a model with the geometry (and so
    the launch shape) of kw takes on a crafted workload of n all-zero samples of class 0, where
    the kernel does the least it can: the floor its class-sum exchange sets.  Weights are +m
    for class 0 and -m for the others with m * C >= T, so firing clauses put every class sum
    at its clip, and no sample needs feedback:
      "stream": every clause empty (it fires on the one patch), the streaming kernel, which
          then never stops;
      "exchange": the resident kernel (one grid-wide exchange per sample).  One patch: empty
          clauses; several patches: every clause holds the last bit of both position
          thermometers, so that it fires on the last patch only (one literal list step, one
          reservoir draw);
      "stop": the streaming kernel with every clause holding literal 0 (a pixel, 0 in every
          sample: it never fires) and weights -1 for class 0, +1 for the others: every class
          sum is 0, every sample needs feedback (probability 1/2), and no branch applies
          (Type II needs a firing clause; target * sign < 0 everywhere): a stop per sample,
          without updates.
    Returns None when the run does not behave as intended (checked from the kernel's
    counters)."""
    from ytm_amd import MultiClassTM

    env = {"stream": "1", "stop": "1", "exchange": "0"}[mode]
    old = os.environ.get("YTM_TRAIN_STREAM")
    os.environ["YTM_TRAIN_STREAM"] = env
    try:
        tm = MultiClassTM(**kw)
        C, K, L, P = tm.number_of_clauses, tm.number_of_outputs, tm.number_of_literals, tm.number_of_patches
        half = tm.number_of_ta_states // 2
        ta = np.full((C, L), half, dtype=np.uint32)
        m = -(-int(kw["T"]) // C)
        w = np.full((C, K), -float(m), dtype=np.float32)
        w[:, 0] = m
        if mode == "stop":
            ta[:, 0] = tm.number_of_ta_states
            w = -w / m
        elif mode == "exchange" and P > 1:
            ty, tx = kw["dim"][1] - kw["patch_dim"][1], kw["dim"][0] - kw["patch_dim"][0]
            ta[:, [ty - 1, ty + tx - 1]] = tm.number_of_ta_states
        _load_state(tm, ta, w)
        X = np.zeros((n, kw["dim"][0] * kw["dim"][1] * kw["dim"][2]), dtype=np.uint32)
        data = tm.device_data(X, np.zeros(n, dtype=np.uint32))
        tm.fit_device(data)
        st = tm.stats()
        data.release()
        tm.release()
    finally:
        if old is None:
            os.environ.pop("YTM_TRAIN_STREAM", None)
        else:
            os.environ["YTM_TRAIN_STREAM"] = old
    want_kind = 0 if mode == "exchange" else 3
    want_fb = n if mode == "stop" else 0
    if st["train_kind"] != want_kind or st["last_fit_feedback_samples"] != want_fb or st["last_fit_updates"] != 0:
        log(f"[bench] floor run {mode}: kernel {st['train_kind']}, feedback samples {st['last_fit_feedback_samples']}, "
            f"updates {st['last_fit_updates']}: not the intended workload, left out")
        return None
    us = 1e3 * st["last_fit_kernel_ms"] / n
    log(f"[bench] floor run {mode}: {n} samples, {us:.3f} us/sample, {st['train_workgroups']} workgroups")
    return us


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


def encode_in_chunks(tm, make_chunk, n: int, chunk: int, binarizer=None):
    """Encoded samples (n, P, W) on the host and the encode kernels' milliseconds, the inputs
    generated and encoded chunk by chunk; with a binarizer, make_chunk gives raw values that
    are binned and encoded in one pass (encode_binarized)."""
    out = np.empty((n, tm.number_of_patches, tm.number_of_literal_chunks), dtype=np.uint32)
    ms = 0.0
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        out[s:e] = tm.encode_binarized(make_chunk(s, e), binarizer) if binarizer else tm.encode(make_chunk(s, e))
        ms += tm.stats()["last_encode_kernel_ms"]
    return out, ms


def cpu_baseline(cfg: int, kw: dict, encX, y, encXt, n_train: int | None) -> dict:
    """The C oracle (a CPU restatement of the reference semantics, oracle/ytm_oracle.c)
    training on the first n_train samples of epoch 1 of the same workload (all of them when
    None) from the same initial state, then scoring 1000 test samples, on this host's cores
    (OpenMP)."""
    from oracle import oracle as orc

    info = cpu_info()
    threads = min(16, info["nproc"] or 1)
    orc.set_threads(threads)
    ref = orc.OracleTM(kw["number_of_clauses_per_class"], kw["T"], kw["s"], kw["dim"], kw["n_classes"],
                       patch_dim=kw.get("patch_dim"), seed=kw["seed"])
    n = encX.shape[0] if n_train is None else min(n_train, encX.shape[0])
    encY = ref.encode_y_multiclass(y[:n])
    t0 = time.perf_counter()
    ref.fit_encoded(encX[:n], encY)
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


def run_config(cfg: int, warmup: int, steps: int, cpu: bool, n_train=None, n_test=None, cpu_samples=None,
               floors: bool = True) -> dict:
    import workloads
    from ytm_amd import MultiClassTM

    t0 = time.perf_counter()
    c = workloads.CONFIGS[cfg]
    kw = dict(c["model"], seed=workloads.MODEL_SEED)
    tm = MultiClassTM(**kw)
    if cfg == 4 and n_train is None and n_test is None:
        # the values of workloads.make(4): its uint8 images, generated in chunks, binned by
        # ThermometerBinarizer(8) and encoded in one pass on the GPU (the binned uint32 array
        # of the training set would be 4.9 GB)
        from ytm_amd.binarizer import ThermometerBinarizer

        gen = workloads.CifarStream(c["n_train"], c["n_test"])
        tb = ThermometerBinarizer(8)
        encX, enc_ms = encode_in_chunks(tm, gen.train_images, c["n_train"], 2048, tb)
        encXt, _ = encode_in_chunks(tm, gen.test_images, c["n_test"], 2048, tb)
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
            f"kernel {KIND_NAMES.get(ep['kind'], ep['kind'])} wait {ep['wait']:.3f} launches {ep['launches']}")
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
            "model": "algorithmic bytes (N*C + U)(2L + 4K) + 4NPW per launch: every TA state read at 2 B and "
                     "every weight at 4 B per sample, updated clauses written back, each sample read once. The "
                     "kernels keep the clause state on chip and do not make these reads, so a frac above 1 is the "
                     "on-chip saving, not HBM use; binding.bound is what limits the kernel",
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
        # measured instruction mix of the same kernel (timed epochs): how busy its execution units are
        res["binding"]["counters"] = counters
    if cfg in (4,):
        # work model of the list walks from the trained state: each clause ANDs the PW-word
        # bitsets of its included literals (no early exit), per sample
        n_inc = tm.get_literals().reshape(tm.number_of_clauses, -1).sum(axis=1, dtype=np.int64)
        pw_words = (tm.number_of_patches + 31) // 32
        ands = float(n_inc.sum()) * pw_words
    tm.release()
    res["binding"]["bound"] = bound_of(cfg, kw, res, timed, N, kern_s, traffic, ands if cfg in (4,) else None,
                                       floors)
    if cpu:
        res["cpu_baseline"] = cpu_baseline(cfg, kw, encX, y, encXt,
                                           cpu_samples if cpu_samples is not None else CPU_PREFIX[cfg])
    return res


def bound_of(cfg: int, kw: dict, res: dict, timed: list, N: int, kern_s: float, traffic, list_ands, floors: bool):
    """What bounds the training kernel in the timed epochs, as {resource, achieved, peak,
    frac} with frac = achieved / peak <= 1, each figure measured in this run or read from a
    committed profile of the current kernel sources:
      configs 1 and 3 (resident kernel): one grid-wide class-sum exchange per sample; peak =
        the samples/s of the same kernel on the same grid when it does nothing but exchange
        (floor_us "exchange");
      config 2 (streaming kernel): the class-sum rows; peak = the samples/s of the timed
        epochs' mix of stops and streamed samples at the kernel's floors (floor_us "stop"
        for each stop, "stream" for every other sample);
      config 4: VALU, the list walks' word-ANDs of the trained state (sum of include counts
        times ceil(P/32) per sample) against 256 CUs x 64 lanes x 2.4 GHz;
      config 5: HBM, the measured traffic of a timed-epoch launch (rocprofv3 FETCH_SIZE +
        WRITE_SIZE, calibrated) against 8 TB/s."""
    steps = len(timed)
    rate = N * steps / kern_s
    if cfg in (1, 3) and floors:
        f = floor_us(kw, "exchange", min(N, 10000))
        if f is None:
            return None
        return {"resource": "class-sum exchange, one per sample (resident kernel)", "unit": "samples/s",
                "achieved": round(rate, 1), "peak": round(1e6 / f, 1), "frac": round(rate * f / 1e6, 4),
                "floor_us_per_sample": round(f, 4)}
    if cfg == 2 and floors:
        fs, fp = floor_us(kw, "stream", 30000), floor_us(kw, "stop", 30000)
        if fs is None or fp is None:
            return None
        stops = sum(e["feedback"] for e in timed)
        t_min = ((N * steps - stops) * fs + stops * fp) / 1e6
        return {"resource": "class-sum rows (streaming kernel): streamed samples and stops", "unit": "samples/s",
                "achieved": round(rate, 1), "peak": round(N * steps / t_min, 1), "frac": round(t_min / kern_s, 4),
                "stream_floor_us_per_sample": round(fs, 4), "stop_floor_us": round(fp, 4), "stops": stops}
    if cfg == 4 and list_ands is not None:
        ach = list_ands * rate / 1e12
        return {"resource": "VALU: list-walk word-ANDs of the trained state (include counts x ceil(P/32))",
                "unit": "T lane-ops/s", "achieved": round(ach, 3), "peak": round(VALU_PEAK_T, 2),
                "frac": round(ach / VALU_PEAK_T, 4), "word_ands_per_sample": list_ands}
    if cfg == 5 and traffic and traffic.get("hbm_gbs"):
        return {"resource": "HBM: measured traffic of a timed-epoch launch", "unit": "GB/s",
                "achieved": traffic["hbm_gbs"], "peak": HBM_PEAK_GBS,
                "frac": round(traffic["hbm_gbs"] / HBM_PEAK_GBS, 4), "epochs": traffic.get("epochs")}
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--n-train", type=int, default=None)
    ap.add_argument("--n-test", type=int, default=None)
    ap.add_argument("--cpu-samples", type=int, default=None,
                    help="training samples of the CPU baseline (default: a fixed prefix per configuration)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-floors", action="store_true", help="skip the floor runs behind binding.bound")
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

    cfg = args.config
    cpu, floors = not args.no_cpu, not args.no_floors
    head = run_config(cfg, args.warmup, args.steps, cpu, args.n_train, args.n_test, args.cpu_samples, floors)
    configs = {str(cfg): head}
    if not args.no_extra:
        for other in (1, 2, 3, 4, 5):
            if other != cfg:
                w, s = EXTRA_EPOCHS[other]
                configs[str(other)] = run_config(other, w, s, cpu, cpu_samples=args.cpu_samples, floors=floors)

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
        "binding": head["binding"],
        "cpu_baseline": head.get("cpu_baseline"),
        "configs": {k: {kk: vv for kk, vv in v.items() if not kk.startswith("_")} for k, v in configs.items()},
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    rc = main()
    if rc:
        sys.exit(rc)
