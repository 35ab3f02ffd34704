"""CPU simulation of the gfx950 kernels' index maps (tests/index_maps_sim.cpp, built
with g++ from rust-gpu_amd/csrc/index_maps.h — the header the kernels include):
DMA coverage exactly once, LDS bijections, fragment reads finding the chunk the
MFMA expects, the ping-pong kernel's hoisted per-wave offsets, the W4A16 decode
slot map, and bank-conflict freedom of the swizzles.  The counterpart of the
reference's pure-CPU locks in tests/gemm_memory_safety.rs."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_index_maps_simulation(tmp_path):
    exe = str(tmp_path / "index_maps_sim")
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Werror", "-o", exe,
                    os.path.join(HERE, "index_maps_sim.cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-4000:]
    assert " 0 failures" in r.stdout and int(r.stdout.split()[0]) > 100000, r.stdout
