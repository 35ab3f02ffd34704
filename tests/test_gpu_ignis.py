"""GPU parity tests of the callers around the GEMM path, through the C ABI:
Ignis matmul forward / backward (src/ignis/ops/bf16_matmul.rs:33-423) and the
GPTQ container conversion (src/t0/quant_kernels.rs:177-294).

Bars: the f32 -> bf16 conversion and the GPTQ layout conversion are bit-exact
against the oracle (NaN inputs excluded: the reference's host formula
(bits + 0x7FFF + lsb) >> 16 can carry a NaN payload into the exponent, the
hardware conversion keeps it a quiet NaN); GEMM results are within
max|err| <= 1e-2 * sqrt(K) * max|a| * max|b| of the oracle's sequential-fp32
GEMM on the same bf16-rounded operands, with relative Frobenius error < 1e-5.
"""
import struct

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


def rand_f32(shape, seed, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape) * scale).astype(np.float32)


def check_gemm(y, ref, a_bf, b_bf, k):
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a_bf), oracle.bf16_to_f32(b_bf))
    err, rel = oracle.compare(y, ref)
    assert err <= tol, (err, tol)
    assert rel < 1e-5, rel


@pytest.mark.parametrize("count", [1, 7, 8, 4096, 100003])
def test_f32_to_bf16_bit_exact(rt, count):
    x = rand_f32(count, count, 3.0)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2.0**-8, 1.0 + 3 * 2.0**-9, 3.3895314e38,
                         1e-40, -1e-45, 65504.0], np.float32)
    x[:min(count, len(specials))] = specials[:min(count, len(specials))]
    dx, px = to_dev(x)
    dy, py = empty_dev(count * 2, fill=0xEE)
    rt.f32_to_bf16(px, py, count)
    y = from_dev(dy, np.uint16, (count,))
    assert np.array_equal(y, oracle.bf16_rne(x))


@pytest.mark.parametrize("m,k,n", [(64, 256, 512), (256, 1024, 256), (37, 100, 70), (1, 8, 8), (130, 48, 200)])
def test_matmul_forward(rt, m, k, n):
    x, w = rand_f32((m, k), 1), rand_f32((k, n), 2)
    dx, px = to_dev(x)
    dw, pw = to_dev(w)
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    rt.matmul(px, pw, py, m, k, n)
    y = from_dev(dy, np.float32, (m, n))
    xb, wb = oracle.bf16_rne(x), oracle.bf16_rne(w)
    check_gemm(y, oracle.gemm_bf16(xb, wb, "nn"), xb, wb, k)


# Up to 16 rows with K a multiple of 32 (the one-launch decode kernel): (16, 256, 128),
# (1, 4096, 4096), (7, 2048, 11008), (16, 96, 136); 50 rows: the split-K schedule.
@pytest.mark.parametrize("m,k,n", [(16, 256, 128), (50, 512, 64), (1, 4096, 4096), (7, 2048, 11008), (16, 96, 136)])
def test_matmul_with_wt_bf16(rt, m, k, n):
    x = rand_f32((m, k), 3)
    wt = oracle.bf16_rne(rand_f32((n, k), 4))
    dx, px = to_dev(x)
    dwt, pwt = to_dev(wt)
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    rt.matmul_with_wt_bf16(px, pwt, py, m, k, n)
    y = from_dev(dy, np.float32, (m, n))
    xb = oracle.bf16_rne(x)
    check_gemm(y, oracle.gemm_bf16(xb, wt, "nt"), xb, wt, k)


@pytest.mark.parametrize("m,k,n", [(64, 256, 512), (37, 100, 70), (3, 24, 16)])
def test_matmul_backward_data(rt, m, k, n):
    """dX[m,k] = dY[m,n] . W[k,n]^T (bf16_matmul.rs:216-262)."""
    dy, w = rand_f32((m, n), 5), rand_f32((k, n), 6)
    ddy, pdy = to_dev(dy)
    dw, pw = to_dev(w)
    dd, pd = empty_dev(m * k * 4, fill=0xCD)
    rt.matmul_backward_data(pdy, pw, pd, m, k, n)
    got = from_dev(dd, np.float32, (m, k))
    dyb, wb = oracle.bf16_rne(dy), oracle.bf16_rne(w)
    check_gemm(got, oracle.gemm_bf16(dyb, wb, "nt"), dyb, wb, n)


@pytest.mark.parametrize("m,k,n", [(64, 256, 512), (37, 100, 70), (200, 64, 24)])
def test_matmul_backward_weight(rt, m, k, n):
    """dW[k,n] = X[m,k]^T . dY[m,n] (bf16_matmul.rs:268-316)."""
    x, dy = rand_f32((m, k), 7), rand_f32((m, n), 8)
    dx, px = to_dev(x)
    ddy, pdy = to_dev(dy)
    dd, pd = empty_dev(k * n * 4, fill=0xCD)
    rt.matmul_backward_weight(px, pdy, pd, m, k, n)
    got = from_dev(dd, np.float32, (k, n))
    xb, dyb = oracle.bf16_rne(x), oracle.bf16_rne(dy)
    xtb = np.ascontiguousarray(xb.T)
    check_gemm(got, oracle.gemm_bf16(xtb, dyb, "nn"), xtb, dyb, m)


def gptq_case(rows, cols, group, seed):
    """A GPTQ container (rows = N, cols = K) with bf16-exact scales and zero points 0..15."""
    q = oracle.nibbles((cols, rows), seed)                       # q[k][n]
    packed = oracle.pack_gptq_bytes(q)                            # [N][K/2]
    ng = cols // group
    s_bf = oracle.uniform_bf16((ng, rows), seed + 1, 0.005, 0.02)  # [G][N]
    z = oracle.nibbles((ng, rows), seed + 2)                      # [G][N]
    scales = np.ascontiguousarray(oracle.bf16_to_f32(s_bf).T)     # [N][G] f32
    zeros = np.ascontiguousarray(z.T.astype(np.int32))            # [N][G] i32
    raw = (struct.pack("<3I", rows, cols, group) + packed.tobytes() + scales.astype("<f4").tobytes()
           + zeros.astype("<i4").tobytes())
    return q, s_bf, z, packed, scales, zeros, raw


@pytest.mark.parametrize("rows,cols,group", [(64, 256, 128), (200, 512, 64), (11008, 4096, 128)])
def test_gptq_convert_bit_exact_and_gemm(rt, rows, cols, group):
    q, s_bf, z, packed, scales, zeros, raw = gptq_case(rows, cols, group, 0x31)
    g = t0mi.GptqWeight.from_bytes(raw)
    assert g.info.zeros_in_range == 1 and g.info.scales_bf16_exact == 1
    # Upload the container as one blob; sections are addressed by the parsed offsets.
    dblob, pblob = to_dev(np.frombuffer(raw, np.uint8))
    K, N = cols, rows
    ng = K // group
    dq, pq = empty_dev(K // 8 * N * 4, fill=0xAA)
    ds, ps = empty_dev(ng * N * 2, fill=0xAA)
    dz, pz = empty_dev(ng * N // 8 * 4, fill=0xAA)
    rt.gptq_convert(pblob + g.info.packed_offset, pblob + g.info.scales_offset, pblob + g.info.zeros_offset,
                    rows, cols, group, pq, ps, pz)
    qw = from_dev(dq, np.uint32, (K // 8, N))
    assert np.array_equal(qw, oracle.pack_qweight(q))
    assert np.array_equal(from_dev(ds, np.uint16, (ng, N)), s_bf)
    assert np.array_equal(from_dev(dz, np.uint32, (ng, N // 8)), oracle.pack_qzeros(z))
    if rows > 1024:
        return  # the full-size case pins the conversion; the GEMM below runs on the smaller ones
    m = 5
    a = oracle.normal_bf16((m, K), 0x32, 0.0, 1.0)
    da, pa = to_dev(a)
    dy, py = empty_dev(m * N * 4, fill=0xCD)
    rt.w4a16_gemm(pa, pq, ps, pz, 0, py, m, K, N, group, t0mi.OUT_F32)
    y = from_dev(dy, np.float32, (m, N))
    # Reference composition: GptqWeight dequant (f32, [N][K]) then the sequential GEMM.
    wf = oracle.dequant_gptq_f32(packed, scales, zeros, rows, cols, group)  # [N][K]
    ref = oracle.w4a16_gemm(a, oracle.pack_qweight(q), s_bf, oracle.pack_qzeros(z), group, 0)
    assert np.array_equal(oracle.dequant_qweight_f32(oracle.pack_qweight(q), s_bf, oracle.pack_qzeros(z), group, 0),
                          wf.T)
    err, rel = oracle.compare(y, ref)
    assert err <= oracle.gemm_tolerance(K, oracle.bf16_to_f32(a), wf) and rel < 1e-5, (err, rel)
