"""GPU tests of t0mi_set_w4a16_workspace_limit: W4A16 calls whose dequant-once route would need
more conversion buffer than the limit run the fused kernels (weights crossing HBM once, at 4 bits).

Bars: the ping-pong fused kernel bit-identical to the dequant-once route at BASELINE config 5's
full size (same bf16 rounding of each weight, same tile and k order) and, there too, within the
GEMM tolerance of the exact-dequant oracle over all outputs; on a ragged shape, where the
dequant-once GEMM takes another tile and split, both routes within the GEMM tolerance; the 128x128
fused tile kernel (groups that are not multiples of 64) within the GEMM tolerance of the oracle;
a group no fused kernel takes refused with T0MI_ERR_INVALID when the limit forbids the buffer.
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture()
def rt():
    r = runtime()
    yield r
    r.close()


def operands(m, k, n, group, seed):
    a = oracle.normal_bf16((m, k), seed + 1, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), seed + 2))
    s = oracle.uniform_bf16((k // group, n), seed + 3, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), seed + 4))
    return a, w, s, z


def run_both(rt, a, w, s, z, m, k, n, group, out_bf16):
    """Y through the default route and through the fused route (limit 0), raw output bits."""
    bufs = [to_dev(x) for x in (a, w, s, z)]
    (_, pa), (_, pw), (_, ps), (_, pz) = bufs
    ob = 2 if out_bf16 else 4
    dt = np.uint16 if out_bf16 else np.uint32
    outs = []
    for limit in (~0 & (2**64 - 1), 0):
        rt.set_w4a16_workspace_limit(limit)
        dy, py = empty_dev(m * n * ob, fill=0xCD)
        print(f"[w4 limit] {m}x{k}x{n} g{group} limit={limit}", flush=True)
        rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
        outs.append(from_dev(dy, dt, (m, n)))
    return outs


def test_config5_full_fused_bit_identical(rt):
    """BASELINE config 5 (4096 x 4096 x 14336, g128, per-group zeros, bf16 out): the fused
    ping-pong kernel and the dequant-once route give the same bits, and the fused output is
    also checked directly against the exact-dequant oracle, all 58.7M outputs (the whole
    GEMM on the CPU, a few seconds with all cores): within the GEMM tolerance plus half a
    bf16 ulp of the output, relative Frobenius error <= 6e-3 (each weight is rounded to
    bf16 once, as the dequant kernel rounds it)."""
    m, k, n, group = 4096, 4096, 14336, 128
    a, w, s, z = operands(m, k, n, group, 0x5100)
    y_default, y_fused = run_both(rt, a, w, s, z, m, k, n, group, True)
    assert np.array_equal(y_default, y_fused)
    y = oracle.bf16_to_f32(y_fused)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, 8))
    tol += float(np.abs(ref).max()) * 2.0 ** -8
    err, rel = oracle.compare(y, ref)
    assert np.isfinite(y).all() and err <= tol and rel <= 6e-3, (err, tol, rel)


def test_ragged_fused_within_tolerance(rt):
    # ragged M and N, group 64: the dequant-once route's GEMM takes the cost model's tile and
    # split for this shape, so the two routes sum K in different partitions; both are checked
    # against the exact-dequant oracle
    m, k, n, group = 1600, 1024, 1000, 64
    a, w, s, z = operands(m, k, n, group, 0x5200)
    y_default, y_fused = run_both(rt, a, w, s, z, m, k, n, group, False)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, 8))
    for y in (y_default.view(np.float32), y_fused.view(np.float32)):
        err, rel = oracle.compare(y, ref)
        assert err <= tol and rel <= 6e-3, (err, tol, rel)


def test_group32_fused_tile_kernel(rt):
    # group 32 (not a multiple of 64): the 128x128 fused tile kernel from 768 rows
    m, k, n, group = 800, 1024, 512, 32
    a, w, s, z = operands(m, k, n, group, 0x5300)
    y_default, y_fused = run_both(rt, a, w, s, z, m, k, n, group, False)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), wf)
    for y in (y_default.view(np.float32), y_fused.view(np.float32)):
        err, rel = oracle.compare(y, ref)
        assert err <= tol and rel <= 6e-3, (err, tol, rel)


def test_group_without_fused_kernel_refused(rt):
    # group 96 (not a power of two): from 81 rows only the dequant-once route exists
    m, k, n, group = 200, 960, 256, 96
    a, w, s, z = operands(m, k, n, group, 0x5400)
    (da, pa), (dw, pw), (ds, ps), (dz, pz) = [to_dev(x) for x in (a, w, s, z)]
    dy, py = empty_dev(m * n * 4, fill=0)
    rt.set_w4a16_workspace_limit(k * n * 2 - 1)
    with pytest.raises(t0mi.T0miError):
        rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_F32)
    rt.set_w4a16_workspace_limit(k * n * 2)  # exactly the buffer: allowed
    rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_F32)
    y = from_dev(dy, np.float32, (m, n))
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, 8))
    err, rel = oracle.compare(y, ref)
    assert err <= tol, (err, tol)


@pytest.mark.parametrize("m", [100, 191])
def test_non_pow2_group_under_limit_takes_pingpong(rt, m):
    # group 192: a multiple of 64 but not a power of two.  With the dequant-once route ruled
    # out, rows below the ping-pong kernel's usual threshold must still run a kernel that
    # indexes groups by division (the ping-pong kernel), not the 128x128 fused kernel, whose
    # k >> log2(group) would read scales and zero points of the wrong groups.
    k, n, group = 1152, 320, 192
    a, w, s, z = operands(m, k, n, group, 0x5500 + m)
    (da, pa), (dw, pw), (ds, ps), (dz, pz) = [to_dev(x) for x in (a, w, s, z)]
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    rt.set_w4a16_workspace_limit(0)
    print(f"[w4 limit] {m}x{k}x{n} g{group} limit=0", flush=True)
    rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_F32)
    y = from_dev(dy, np.float32, (m, n))
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.dequant_qweight_f32(w, s, z, group, 8))
    err, rel = oracle.compare(y, ref)
    assert err <= tol and rel < 1e-2, (err, tol, rel)
