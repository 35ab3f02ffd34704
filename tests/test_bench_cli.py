"""bench.py's contract: one GPU only (--gpus N > 1 exits 2 with a message, before
touching a GPU), the committed HBM-traffic figures its roofline objects read, and
(on a GPU) one JSON line per run with the roofline fields for every leg."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def run_bench(*args, timeout=300):
    return subprocess.run([sys.executable, BENCH, *args], cwd=ROOT, capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2", timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_traffic_figures_for_every_leg():
    sys.path.insert(0, ROOT)
    import bench
    for key in ("gemm_4096", "w4a16_decode", "gemm_skinny", "w4a16_prefill"):
        t = bench.load_traffic(key)
        assert isinstance(t, int) and t > 0, key
    # HBM-side traffic is at least the bytes the kernel must move.
    assert bench.load_traffic("gemm_4096") >= 3 * 2 * 4096 * 4096
    assert bench.load_traffic("w4a16_decode") >= 2 * 16 * 4096 + 4096 * 11008 // 2


@pytest.mark.gpu
@pytest.mark.parametrize("leg,unit,bound", [("gemm", "TFLOPS", "mfma"), ("w4a16", "GB/s", "hbm"),
                                            ("skinny", "GB/s", "hbm"), ("prefill", "TFLOPS", "mfma"),
                                            ("shard", "GB/s", "hbm")])
def test_leg_prints_one_json_line(leg, unit, bound):
    r = run_bench("--only", leg, "--steps", "3", "--warmup", "1", "--no-cpu")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    out = json.loads(lines[0])
    assert out["n_gpus"] == 1 and out["unit"] == unit and out["value"] > 0
    roof = out["roofline"]
    assert roof["bound"] == bound and 0 < roof["frac"] < 1
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], rel=1e-3)
    assert roof["traffic"] > 0
