"""CPU simulation of the gfx950 kernels' index maps (tests/index_maps_sim.cpp, built
with g++ from rust-gpu_amd/csrc/index_maps.h — the header the kernels include):
DMA coverage exactly once, LDS bijections, fragment reads finding the chunk the
MFMA expects (32x32x16 and 16x16x32 operand layouts, the 16x16x32 transpose-read
lane map), the ping-pong kernel's hoisted per-wave offsets, the W4A16 decode slot
map, the persistent decode kernel's NN block (stores a bijection, transpose reads
finding the B operand, each half-wave's read one 256-byte run), and bank-conflict freedom of the swizzles under every LDS bank rule that
reproduces the conflict counts measured on gfx950 (the measured cycles per read of
the probe patterns are data in the simulation).  The counterpart of the reference's
pure-CPU locks in tests/gemm_memory_safety.rs."""
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
    lines = r.stdout.strip().splitlines()
    assert int(lines[0].split()[0]) > 0, r.stdout  # LDS bank rules that fit the measurements
    assert lines[-1].endswith(" 0 failures") and int(lines[-1].split()[0]) > 100000, r.stdout
