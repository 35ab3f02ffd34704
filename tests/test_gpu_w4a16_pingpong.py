"""GPU parity tests of the fused W4A16 ping-pong kernel (csrc/w4a16_pingpong.h),
which t0mi_w4a16_gemm runs for 192..1535 rows when K and the group are
multiples of 64 (dequant fused into the MFMA K-loop, as BASELINE config 5
describes; at config 5's 4096 rows the dequant-once route is faster and runs).

Bars:
  - bit-identical to the two-pass route on the same problem: t0mi_dequant_int4
    (bf16, RNE of the exact (q - z) * s; quant_kernels.rs:24, 95-100) followed
    by t0mi_gemm with the NN 256x256x64 configuration and the same split-K —
    the fused kernel rounds each weight the same way and keeps that GEMM's
    MFMA order and partition boundaries;
  - against the CPU oracle within the GEMM tolerance
    1e-2 * sqrt(K) * max|a| * max|w| (bf16 output: after RNE).
Cases: ragged M and N, constant and per-group zero points, groups 64..256,
split-K 1 and 8, f32 and bf16 output.
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


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def make(m, k, n, group, zeros, seed):
    g = np.random.default_rng(seed)
    a = oracle.bf16_trunc(g.standard_normal((m, k)).astype(np.float32))
    w = g.integers(0, 2**32, (k // 8, n), dtype=np.uint32)
    s = oracle.bf16_trunc(g.uniform(0.005, 0.02, (k // group, n)).astype(np.float32))
    z = g.integers(0, 2**32, (k // group, n // 8), dtype=np.uint32) if zeros else None
    return a, w, s, z


def split_of(m, n, k):
    """The split-K the W4A16 route picks: a power of two up to 8 and the 256 CUs'
    share of 256x256 tiles, halved while a partition would be empty."""
    tiles = -(-m // 256) * -(-n // 256)
    nk = k // 64
    want = min(8, 256 // max(1, tiles))
    sk = 1
    while sk * 2 <= want and sk * 2 <= nk:
        sk *= 2
    while sk > 1 and -(-nk // sk) * (sk - 1) >= nk:
        sk //= 2
    return sk


CASES = [
    # (m, k, n, group, zeros, out_bf16)
    (512, 2048, 4096, 128, True, True),
    (300, 512, 1000, 128, True, True),
    (768, 1024, 2560, 64, False, False),
    (1024, 256, 16384, 128, True, True),   # 256 tiles: no split
    (193, 4096, 1536, 256, True, False),
]


@pytest.mark.parametrize("m,k,n,group,zeros,out_bf16", CASES)
def test_fused_equals_two_pass_bit_for_bit(rt, m, k, n, group, zeros, out_bf16):
    a, w, s, z = make(m, k, n, group, zeros, 100 + m)
    od = t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32
    ob = 2 if out_bf16 else 4
    da, pa = to_dev(a)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    pz = 0
    if zeros:
        dz, pz = to_dev(z)
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    rt.w4a16_gemm(pa, pw, ps, pz, 8, py, m, k, n, group, od)
    fused = from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))
    # Two-pass: bf16 weights (RNE), then the NN 256x256 GEMM with the same split.
    dwb, pwb = empty_dev(k * n * 2)
    rt.dequant_int4(pw, ps, pz, 8, pwb, k, n, group, 2)
    cfg = t0mi.preset("gfx950_256x256_k64_w2x4").copy(transpose=t0mi.NN, split_k=split_of(m, n, k), out_dtype=od)
    dy2, py2 = empty_dev(m * n * ob, fill=0xCD)
    rt.gemm(cfg, pa, pwb, py2, m, n, k)
    two = from_dev(dy2, np.uint16 if out_bf16 else np.float32, (m, n))
    assert np.array_equal(fused, two), f"{np.count_nonzero(fused != two)} elements differ"
    # And the oracle (dequant as the reference defines it, then its CPU loop).
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    ref = oracle.gemm_bf16(a, oracle.bf16_rne(wf), "nn")
    got = bf16_to_f32(fused) if out_bf16 else fused
    tol = 1e-2 * np.sqrt(k) * np.abs(bf16_to_f32(a)).max() * np.abs(wf).max()
    assert np.abs(got - ref).max() <= tol


def _random_cases(n_cases=12, seed=0x4B1D):
    g = np.random.default_rng(seed)
    out = []
    for i in range(n_cases):
        group = int(g.choice([64, 128, 256]))
        k = group * int(g.integers(1, max(2, 2048 // group) + 1))
        n = 8 * int(g.integers(1, 400))
        m = int(g.integers(192, 1536))
        out.append((i, m, k, n, group, bool(g.integers(0, 2)), bool(g.integers(0, 2))))
    return out


@pytest.mark.parametrize("i,m,k,n,group,zeros,out_bf16", _random_cases())
def test_random_shapes_equal_two_pass(rt, i, m, k, n, group, zeros, out_bf16):
    test_fused_equals_two_pass_bit_for_bit(rt, m, k, n, group, zeros, out_bf16)
