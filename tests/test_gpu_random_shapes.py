"""GPU parity over seeded random shapes: t0mi_gemm with the auto_select configuration (both B
layouts, f32 and bf16 out, K = 0 included, every route the cost model and the split-K / column
split take) and t0mi_w4a16_gemm at random row counts (every route: decode slabs, the in-launch
K split for narrow N, the fused kernels, dequant-once with its column split; groups 32..256 and
192), each against the oracle.

Bars: GEMM max|err| <= 1e-2 * sqrt(K) * max|a| * max|b| (plus half a bf16 ulp of the largest
output for bf16 out; K = 0 exactly zero); W4A16 the same bound against the exact-dequant
oracle with relative Frobenius error <= 6e-3 (routes that round each weight to bf16 once).
The shapes are drawn from fixed seeds, so every run checks the same cases.
"""
import random

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


def gemm_case(i):
    g = random.Random(0x6E00 + i)
    m = g.choice([g.randint(1, 64), g.randint(1, 2048)])
    n = 8 * g.randint(1, 320)
    k = 8 * g.randint(0, 512)
    return m, n, k, g.choice([t0mi.NN, t0mi.NT]), g.choice([t0mi.OUT_F32, t0mi.OUT_BF16])


def w4_case(i):
    g = random.Random(0x4E00 + i)
    group = g.choice([32, 64, 128, 256, 192])
    k = group * g.randint(1, max(1, 4096 // group))
    m = g.choice([g.randint(1, 16), g.randint(1, 300), g.randint(1, 1800)])
    n = 8 * g.randint(1, 400)
    return m, k, n, group, g.random() < 0.5


@pytest.mark.parametrize("i", range(40))
def test_gemm_random_shape(rt, i):
    m, n, k, tr, out = gemm_case(i)
    cfg = t0mi.auto_select_layout(m, k, n, tr, out).copy(transpose=tr, out_dtype=out)
    a = oracle.normal_bf16((m, k), 0x100 + i, 0.0, 1.0)
    b = oracle.normal_bf16((k, n) if tr == t0mi.NN else (n, k), 0x200 + i, 0.0, 1.0)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    ob = 4 if out == t0mi.OUT_F32 else 2
    dy, py = empty_dev(m * n * ob, fill=0xCD)
    print(f"[random gemm {i}] {cfg.name()} {m}x{n}x{k}", flush=True)
    rt.gemm(cfg, pa, pb, py, m, n, k)
    y = from_dev(dy, np.float32 if ob == 4 else np.uint16, (m, n))
    y = y if ob == 4 else oracle.bf16_to_f32(y)
    ref = oracle.gemm_bf16(a, b, "nn" if tr == t0mi.NN else "nt")
    assert np.isfinite(y).all()
    if k == 0:
        assert not np.any(y), "K = 0: Y = 0"
        return
    bf = oracle.bf16_to_f32(b) if tr == t0mi.NN else oracle.bf16_to_f32(b).T
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), bf)
    if ob == 2:
        tol += float(np.abs(ref).max()) * 2.0 ** -8
    assert float(np.abs(y - ref).max()) <= tol


@pytest.mark.parametrize("i", range(30))
def test_w4a16_random_shape(rt, i):
    m, k, n, group, zeros = w4_case(i)
    a = oracle.normal_bf16((m, k), 0x300 + i, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), 0x400 + i))
    s = oracle.uniform_bf16((k // group, n), 0x500 + i, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), 0x600 + i)) if zeros else None
    bufs = [to_dev(x) for x in (a, w, s)]
    pz = 0
    if z is not None:
        dz, pz = to_dev(z)
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    print(f"[random w4a16 {i}] {m}x{k}x{n} g{group} zeros={zeros}", flush=True)
    rt.w4a16_gemm(bufs[0][1], bufs[1][1], bufs[2][1], pz, 8, py, m, k, n, group, t0mi.OUT_F32)
    y = from_dev(dy, np.float32, (m, n))
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, 8))
    err, rel = oracle.compare(y, ref)
    assert np.isfinite(y).all() and err <= tol and rel <= 6e-3, (err, tol, rel)
