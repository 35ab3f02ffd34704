"""GPU tests of the W4A16 decode with its K range split over workgroups inside one launch
(w4a16_decode_v2 with XK: the pieces of a 64-column strip are numbered onto the strip's XCD,
store their partials and the last piece sums them in piece order).

Bars: against the exact-dequant oracle within max|err| <= 1e-2 * sqrt(K) * max|a| * max|w|
and relative Frobenius error <= 1e-5 (f32 out); bit-identical results for repeated calls,
across shapes that reuse the exchange counters, and across HIP-graph replays (the counters
reset themselves).  Where a workgroup runs is only reported: the slots are written through
to memory, so the bars hold wherever the pieces ran.
"""
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


def case(m, k, n, group, zeros, seed):
    a = oracle.normal_bf16((m, k), seed + 1, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), seed + 2))
    s = oracle.uniform_bf16((k // group, n), seed + 3, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), seed + 4)) if zeros else None
    return a, w, s, z


def dev_args(a, w, s, z):
    bufs = [to_dev(x) for x in (a, w, s)]
    pz = 0
    if z is not None:
        dz, pz = to_dev(z)
        bufs.append((dz, pz))
    return bufs, (bufs[0][1], bufs[1][1], bufs[2][1], pz)


def xk_state(r):
    # The exchange is on.  A workgroup on another XCD than planned is only reported (its
    # partials then cross XCDs through memory): the results checked are what matters.
    n, misplaced = r.xcd_placement()
    print(f"[xk] xcds={n} misplaced={misplaced}", flush=True)
    return n == 8


def check_oracle(y, a, w, s, z, k, group, zp=8, rel_max=1e-5):
    ref = oracle.w4a16_gemm(a, w, s, z, group, zp)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, zp))
    err, rel = oracle.compare(y, ref)
    assert err <= tol and rel <= rel_max, (err, tol, rel)


def test_placement_probe_found_the_xcds(rt):
    n, misplaced = rt.xcd_placement()
    print(f"[xk] xcds={n} misplaced={misplaced}", flush=True)
    assert n == 8, "MI355X: 8 XCDs, workgroup i on XCD i % 8"


@pytest.mark.parametrize("m,k,n,group,zeros", [
    (16, 4096, 1376, 128, False),   # the column-parallel shard of config 4 over 8 GPUs: 22 strips x 8 pieces
    (16, 4096, 90 * 64, 128, True),  # 90 strips x 2 pieces: the XCD numbering's padding (90 % 8 != 0)
    (7, 2048, 8 * 64 + 8, 64, True),    # a partial last strip, 9 strips x 4 pieces
    (16, 8192, 200, 128, False),    # 4 strips x 8 pieces of 8 waves
    (1, 4096, 4096, 32, False),     # group 32, 64 strips x 4 pieces
    (16, 4096, 4096, 256, True),    # group 256: 8 k-blocks per wave, 2 pieces
    (12, 16384, 128, 128, False),   # 2 strips x 8 pieces of 8 waves x 8 k-blocks
    (16, 65536, 64, 128, False),    # a piece would need 32 k-blocks per wave: one workgroup per strip
    (16, 4096, 11008 - 64, 128, True),  # 171 strips: one workgroup per strip (no split)
])
def test_decode_xk_vs_oracle(rt, m, k, n, group, zeros):
    a, w, s, z = case(m, k, n, group, zeros, 0x910 + m + n)
    bufs, (pa, pw, ps, pz) = dev_args(a, w, s, z)
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    print(f"[xk] {m}x{k}x{n} g{group} zeros={zeros}", flush=True)
    rt.w4a16_gemm(pa, pw, ps, pz, 8, py, m, k, n, group, t0mi.OUT_F32)
    check_oracle(from_dev(dy, np.float32, (m, n)), a, w, s, z, k, group)
    db, pb = empty_dev(m * n * 2, fill=0xCD)
    rt.w4a16_gemm(pa, pw, ps, pz, 8, pb, m, k, n, group, t0mi.OUT_BF16)
    yb = oracle.bf16_to_f32(from_dev(db, np.uint16, (m, n)))
    check_oracle(yb, a, w, s, z, k, group, rel_max=5e-3)
    assert xk_state(rt)


def test_counters_reset_across_shapes(rt):
    # Three shapes whose strips share counters (strip s of any shape uses counter s of its
    # XCD), run A, B, A: each result bit-identical to its first run.
    shapes = [(16, 4096, 2048, 128), (16, 2048, 4096, 64), (16, 4096, 2048, 128)]
    outs = []
    for i, (m, k, n, g) in enumerate(shapes):
        a, w, s, z = case(m, k, n, g, False, 0x920 + (i % 2))
        bufs, (pa, pw, ps, pz) = dev_args(a, w, s, z)
        dy, py = empty_dev(m * n * 4, fill=0)
        rt.w4a16_gemm(pa, pw, ps, pz, 8, py, m, k, n, g, t0mi.OUT_F32)
        outs.append(from_dev(dy, np.float32, (m, n)))
        if i == 0:
            check_oracle(outs[0], a, w, s, z, k, g)
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))


def test_graph_replays_match_eager():
    torch = pytest.importorskip("torch")
    r = t0mi.Runtime(device=0)  # own stream: a graph cannot be captured on the null stream
    try:
        m, k, n, g = 16, 4096, 1376, 128  # the split route: 22 strips x 8 pieces
        a, w, s, z = case(m, k, n, g, True, 0x930)
        bufs, (pa, pw, ps, pz) = dev_args(a, w, s, z)
        torch.cuda.synchronize()
        ys = [empty_dev(m * n * 2, fill=0) for _ in range(3)]
        for dy, py in ys:  # eager once: the exchange buffers exist before the capture
            r.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, g, t0mi.OUT_BF16)
        assert r.wait_idle() == t0mi.OK
        ref = from_dev(ys[0][0], np.uint16, (m, n))
        yf = oracle.bf16_to_f32(ref)
        check_oracle(yf, a, w, s, z, k, g, zp=0, rel_max=5e-3)
        for dy, _ in ys:
            dy[: m * n * 2].fill_(0)
        torch.cuda.synchronize()
        r.capture_begin()
        for dy, py in ys:
            r.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, g, t0mi.OUT_BF16)
        graph = r.capture_end()
        side, pside = empty_dev(m * n * 2, fill=0)
        for rep in range(4):
            for dy, _ in ys:
                dy[: m * n * 2].fill_(0)
            torch.cuda.synchronize()
            graph.launch()
            assert r.wait_idle() == t0mi.OK
            for dy, _ in ys:
                assert np.array_equal(from_dev(dy, np.uint16, (m, n)), ref), rep
            # eager work between the replays, on the same counters
            r.w4a16_gemm(pa, pw, ps, pz, 0, pside, m, k, n, g, t0mi.OUT_BF16)
            assert r.wait_idle() == t0mi.OK
            assert np.array_equal(from_dev(side, np.uint16, (m, n)), ref), rep
        graph.destroy()
        assert xk_state(r)
    finally:
        r.close()
