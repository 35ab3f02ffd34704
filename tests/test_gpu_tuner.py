"""GPU tests of the measure-and-pick autotuner: GemmTuner::tune and auto_gemm
(src/t0/auto_gemm.rs:82-216, 223-272, 555-590; the reference's own GPU test is
test_tune_4096, auto_gemm.rs:660-745).

Bars: the tuned config computes the oracle's result exactly on the reference's
integer pattern (every partial sum is an exact fp32 integer); the choice is
persisted as JSON in the given cache directory and served from memory, then
from disk by a fresh tuner, without re-timing; auto_gemm gives the reference's
known answer Y[0,0] = -6 at (m, k, n) = (128, 64, 128) (auto_gemm.rs:655).
"""
import json
import os

import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def int_pattern_nt(m, k, n):
    """a = (i%7)-3 over A's flat index, b = (j%5)-2 over WT[n, k]'s (auto_gemm.rs:700-701)."""
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(n * k) % 5) - 2).astype(np.float32).reshape(n, k)
    return oracle.bf16_trunc(a), oracle.bf16_trunc(b)


def run_cfg(rt, cfg, m, n, k):
    a, b = int_pattern_nt(m, k, n)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    dy, py = empty_dev(m * n * 4, fill=0xAB)
    rt.gemm(cfg, pa, pb, py, m, n, k)
    return from_dev(dy, np.float32, (m, n)), oracle.gemm_bf16(a, b, "nt")


def test_tune_persists_and_hits_cache(rt, tmp_path):
    m, n, k = 256, 512, 512
    print(f"[tuner] tune {m}x{n}x{k} NT into {tmp_path}", flush=True)
    tuner = t0mi.GemmTuner(str(tmp_path), max_candidates=3, n_iters=3)
    cfg, tf, cached = tuner.tune(rt, m, n, k)
    assert not cached and tf > 0.5, (cfg.name(), tf)  # timed, and the kernel did real work
    y, ref = run_cfg(rt, cfg, m, n, k)
    assert np.array_equal(y, ref), cfg.name()
    # persisted: the reference's JSON keys (auto_gemm.rs:478-492) describe the chosen config
    path = tuner.cache_path(m, n, k)
    assert os.path.isfile(path) and path.startswith(str(tmp_path))
    js = json.load(open(path))
    for key in ("tile_m", "tile_n", "tile_k", "wg_size", "split_k"):
        assert js[key] == getattr(cfg, key) or (key == "split_k" and js[key] in (0, 1) and cfg.split_k in (0, 1))
    assert js["tflops"] > 0
    # memory hit, then a fresh tuner on the same directory reads the file
    cfg2, tf2, cached2 = tuner.tune(rt, m, n, k)
    assert cached2 and cfg2.name() == cfg.name() and tf2 == tf
    cfg3, _, cached3 = t0mi.GemmTuner(str(tmp_path)).tune(rt, m, n, k)
    assert cached3 and cfg3.name() == cfg.name()
    assert "TF" in tuner.report() or cfg.name() in tuner.report()


def test_tune_bf16_out_nn(rt, tmp_path):
    """Layout and output dtype are part of the key: an NN bf16-output tuning gets its own entry."""
    m, n, k = 128, 256, 1024
    tuner = t0mi.GemmTuner(str(tmp_path), max_candidates=2, n_iters=2)
    cfg, tf, cached = tuner.tune(rt, m, n, k, transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16)
    assert not cached and tf > 0 and cfg.transpose == t0mi.NN and cfg.out_dtype == t0mi.OUT_BF16
    assert tuner.cache_path(m, n, k, t0mi.NN, t0mi.OUT_BF16) != tuner.cache_path(m, n, k)
    a = oracle.normal_bf16((m, k), 3, 0.0, 1.0)
    b = oracle.normal_bf16((k, n), 4, 0.0, 1.0)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    dy, py = empty_dev(m * n * 2, fill=0xAB)
    rt.gemm(cfg, pa, pb, py, m, n, k)
    y = oracle.bf16_to_f32(from_dev(dy, np.uint16, (m, n)))
    ref = oracle.gemm_bf16(a, b, "nn")
    # bf16 output: within one bf16 ulp of the fp32 oracle
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6), cfg.name()


def test_auto_gemm_known_answer_through_the_tuner(rt, tmp_path, monkeypatch):
    """auto_gemm (process-wide tuner, NT, f32 out) at the reference's correctness-gate shape."""
    monkeypatch.setenv("HOME", str(tmp_path))  # the process-wide tuner's cache lives under $HOME
    m, k, n = 128, 64, 128
    a, b = int_pattern_nt(m, k, n)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    dy, py = empty_dev(m * n * 4, fill=0xAB)
    print("[tuner] auto_gemm 128x64x128", flush=True)
    tf = rt.auto_gemm(pa, pb, py, m, n, k)
    y = from_dev(dy, np.float32, (m, n))
    assert y[0, 0] == -6.0
    assert np.array_equal(y, oracle.gemm_bf16(a, b, "nt"))
    assert tf > 0
    # a second call is served by the tuner's cache and gives the same result
    dy2, py2 = empty_dev(m * n * 4, fill=0)
    assert rt.auto_gemm(pa, pb, py2, m, n, k) == tf
    assert np.array_equal(from_dev(dy2, np.float32, (m, n)), y)
