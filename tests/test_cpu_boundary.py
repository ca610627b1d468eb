"""CPU-only checks of the drop-in boundary: libytm.so loads and exports every entry point
include/ytm.h declares; the Python binding covers them; the reference's hyperparameter
typing (base.py:129-152 pasted into kernel.cu:31-32) is reproduced."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "ytm.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ytm_[a-z_]+)\s*\(", text)))


def test_header_declares_api():
    names = declared_functions()
    for required in ("ytm_create", "ytm_fit", "ytm_fit_dataset", "ytm_score", "ytm_encode", "ytm_transform",
                     "ytm_get_ta_state", "ytm_set_ta_state", "ytm_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(ROOT / "ytm_amd" / "libytm.so"))
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_python_binding_covers_header():
    from ytm_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_params_struct_layout():
    """ytm_params in Python matches the C layout (int32 x 15, double x 2, uint64)."""
    from ytm_amd._lib import YtmParams

    assert ctypes.sizeof(YtmParams) == 15 * 4 + 4 + 8 + 8 + 8  # 4 bytes of padding before s_inv
    assert YtmParams.s_inv.offset == 64 and YtmParams.seed.offset == 80


def test_error_without_gpu_is_raised_not_swallowed():
    import ytm_amd
    from ytm_amd import _lib

    try:
        ytm_amd.MultiClassTM(10, 15, 3.9, (12, 1, 1), 2, seed=1)
    except (ValueError, _lib.YtmError) as exc:  # no device here: libytm reports it
        assert str(exc)
    else:
        pytest.skip("a GPU is visible; covered by the gpu tests")


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_specialised_training_kernels_compile(cfg):
    """hipRTC compiles the per-model training kernels (both draw modes) without a GPU."""
    import workloads
    from ytm_amd import MultiClassTM

    kw = workloads.make(cfg, 2, 2)[4]
    for injected in (False, True):
        kinds = MultiClassTM.compile_kernels(**kw, injected=injected)
        # the streaming kernel (3): one patch, counter stream, at most 64 clauses per workgroup
        # on 256 CUs, clause state within LDS (configs 1 and 2; not config 5's 10000 wide clauses)
        expect = [0, 2] if cfg in (3, 4) else ([0, 1, 3] if cfg in (1, 2) and not injected else [0, 1])
        assert kinds == expect


def test_compile_entry_point_rejects_bad_kind():
    from ytm_amd import MultiClassTM, _lib

    tm = MultiClassTM.__new__(MultiClassTM)
    tm._skip_gpu_init = True
    tm.__init__(10, 15, 3.9, (12, 1, 1), 2, seed=1)
    params = tm._params()
    assert _lib.lib.ytm_compile_train_kernel(ctypes.byref(params), 2, 0, 0) == 1  # 2: several patches only
    assert _lib.lib.ytm_compile_train_kernel(ctypes.byref(params), 7, 0, 0) == 1
    assert b"train_kind" in _lib.lib.ytm_last_error()
    assert _lib.lib.ytm_compile_train_kernel(ctypes.byref(params), 3, 1, 0) == 1  # streaming: counter stream only
    assert b"streaming" in _lib.lib.ytm_last_error()
    assert _lib.lib.ytm_compile_train_kernel(ctypes.byref(params), 0, 0, -1) == 1
    assert b"compute_units" in _lib.lib.ytm_last_error()


@pytest.mark.parametrize(
    "s,expected",
    [
        (10, np.float32(1.0) / np.float32(10)),  # int literal: float division
        (2, 0.5),
        (10.0, 1.0 / 10.0),                      # floating literal: double division
        (3.9, 1.0 / 3.9),
        (np.float32(3.9), 1.0 / 3.9),             # pasted as the text "3.9"
    ],
)
def test_s_inv_typing(s, expected, oracle_mod):
    from ytm_amd.base import typed_s_inv

    assert typed_s_inv(s) == float(expected)
    assert oracle_mod.s_inv_of(s) == float(expected)


def test_s_inv_int_is_not_double():
    from ytm_amd.base import typed_s_inv

    assert typed_s_inv(10) != 0.1  # 1.0f/10 is float(0.1) = 0.10000000149...
    assert typed_s_inv(10.0) == 0.1


@pytest.mark.parametrize(
    "q,K,expected",
    [
        (1.0, 10, 1.0 / 9),                                  # default q (float) -> double
        (1.0, 2, 1.0),                                       # max(1, K-1) = 1
        (1.0, 1, 1.0),
        (3, 10, float(np.float32(3.0) / np.float32(9))),   # int q -> float
        (0.5, 3, 0.25),
    ],
)
def test_q_prob_typing(q, K, expected, oracle_mod):
    from ytm_amd.base import typed_q_prob

    qq = min(q, float(K))  # base.py:81
    assert typed_q_prob(qq, K) == expected
    assert oracle_mod.q_prob_of(qq, K) == expected


def test_q_is_min_of_q_and_classes():
    # base.py:81 turns an int q >= K into float(K) (a double literal).
    assert min(12, float(10)) == 10.0 and isinstance(min(12, float(10)), float)
    assert isinstance(min(3, float(10)), int)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_bench_profile_summaries(cfg):
    """The committed rocprofv3 summaries of each configuration's training kernel (HBM traffic,
    SQ counters) parse, name the kernel the configuration trains with, hold consistent
    figures, and record the hash of the kernel sources they were measured on."""
    import json

    import bench
    tr = json.loads((bench.ROOT / "profiles" / f"train_cfg{cfg}_traffic.json").read_text())
    ct = json.loads((bench.ROOT / "profiles" / f"train_cfg{cfg}_counters.json").read_text())
    assert tr["kernel"].startswith("ytm_jit_train_") and tr["kernel"] == ct["kernel"]
    assert tr["bytes_per_launch"] > 0 and 0 < tr["hbm_gbs"] < bench.HBM_PEAK_GBS
    assert 0.0 <= ct["valu_busy"] <= 1.0 and 0.0 <= ct["lds_bank_conflict"] <= 1.0
    assert ct["valu_insts_per_sample"] > 0
    for d in (tr, ct):  # measured on the kernel sources of this tree
        assert d["source_sha16"] == bench.kernel_source_hash()
    assert tr["epochs"] == ct["epochs"] and tr["bytes_per_launch"] < tr["algorithmic_bytes_per_launch"] * 2


def test_bench_reports_only_current_profiles(tmp_path, monkeypatch):
    """A summary measured on other kernel sources (another source_sha16) is not reported."""
    import json

    import bench
    (tmp_path / "profiles").mkdir()
    d = {"kernel": "ytm_jit_train_stream", "bytes_per_launch": 1.0, "hbm_gbs": 1.0}
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    monkeypatch.setattr(bench, "kernel_source_hash", lambda: "0123456789abcdef")
    (tmp_path / "profiles" / "train_cfg2_traffic.json").write_text(json.dumps(dict(d, source_sha16="fedcba9876543210")))
    assert bench.load_traffic(2) is None
    (tmp_path / "profiles" / "train_cfg2_traffic.json").write_text(json.dumps(dict(d, source_sha16="0123456789abcdef")))
    assert bench.load_traffic(2)["bytes_per_launch"] == 1.0


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_bench_bound_is_a_fraction(cfg, monkeypatch):
    """binding.bound puts each configuration's measured rate against a peak it cannot pass:
    with floors below the measured per-sample time, 0 < frac <= 1 and frac = achieved / peak."""
    import bench
    N, kern_s = 60000, 0.3  # 5 us per sample
    timed = [{"feedback": 1000}, {"feedback": 500}]
    monkeypatch.setattr(bench, "floor_us", lambda kw, mode, n: {"exchange": 2.0, "stream": 0.2, "stop": 4.0}[mode])
    traffic = {"hbm_gbs": 4000.0, "epochs": [6, 7]}
    b = bench.bound_of(cfg, {}, {}, timed, N, 2 * kern_s, traffic, 3.0e7, True)
    assert b is not None and 0.0 < b["frac"] <= 1.0
    assert abs(b["achieved"] / b["peak"] - b["frac"]) < 1e-3
