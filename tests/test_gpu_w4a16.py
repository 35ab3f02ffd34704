"""GPU parity tests of the W4A16 GEMM and the standalone INT4 dequant against the oracle.

Bars: dequant bit-exact (f32, bf16-truncate, bf16-RNE); GEMM within
max|err| <= 1e-2 * sqrt(K) * max|a| * max|w| with relative Frobenius error bounded.
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


def make_case(m, k, n, group, per_group_zeros, seed=0x40):
    a = oracle.normal_bf16((m, k), seed + 1, 0.0, 1.0)
    q = oracle.nibbles((k, n), seed + 2)
    w = oracle.pack_qweight(q)
    s = oracle.uniform_bf16((k // group, n), seed + 3, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), seed + 4)) if per_group_zeros else None
    return a, q, w, s, z


def run_w4a16(rt, a, w, s, z, m, k, n, group, zp_const=8, out_bf16=True):
    da, pa = to_dev(a)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    pz = 0
    if z is not None:
        dz, pz = to_dev(z)
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xCD)
    rt.w4a16_gemm(pa, pw, ps, pz, zp_const, py, m, k, n, group, t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    y = from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))
    return oracle.bf16_to_f32(y) if out_bf16 else y


def check(y, ref, a, wf, k, rel_max):
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), wf)
    err, rel = oracle.compare(y, ref)
    assert err <= tol, (err, tol)
    assert rel <= rel_max, rel
    return err, rel


@pytest.mark.parametrize("m,k,n,group,pgz", [
    (16, 4096, 11008, 128, False),   # BASELINE config 4 (decode), full size
    (1, 512, 64, 128, False),
    (5, 256, 136, 32, True),
    (16, 1024, 520, 64, True),
    (16, 8192, 256, 128, False),     # K beyond one workgroup's range -> split + reduce
    (32, 384, 200, 128, True),       # M > 16 -> several row slabs
    (76, 256, 136, 64, False),       # 5 slabs, the last one 12 rows
    (80, 384, 200, 128, True),       # two launches: three slabs, then two
    (96, 384, 200, 128, True),       # two launches of three slabs
    (191, 384, 200, 128, True),      # group 128: three launches of four slabs, the last decode row count
    (144, 384, 200, 64, True),       # group 64: three launches of three slabs, the last decode row count
    (70, 384, 136, 96, True),        # slabs with a group that is not a power of two
    (3, 4096, 64, 4096, False),      # group larger than a wave's K range
])
def test_w4a16_vs_oracle(rt, m, k, n, group, pgz):
    a, q, w, s, z = make_case(m, k, n, group, pgz)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    y32 = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=False)
    check(y32, ref, a, wf, k, 1e-5)
    yb = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=True)
    check(yb, ref, a, wf, k, 5e-3)


@pytest.mark.parametrize("m,k,n,group,pgz", [
    (145, 384, 200, 64, True),       # group 64 just above the decode range: 128x128 tiles, split K
    (97, 512, 200, 256, True),       # group 256 (two slabs per launch) above 96 rows: 128x128 tiles
    (150, 256, 136, 32, True),       # group 32 above its decode range (144 rows)
    (191, 256, 136, 64, True),       # last row count of the 128x128 fused kernel (group 64)
    (192, 256, 136, 128, True),      # first of the ping-pong fused kernel
    (300, 512, 264, 64, False),      # ping-pong: ragged M and N tiles
    (300, 512, 264, 32, True),       # group 32: the 128x128 fused kernel
    (200, 352, 136, 32, True),       # K % 64 == 32: the last K tile is half past K
    (767, 256, 136, 32, True),       # group 32: last row count of the 128x128 fused kernel
    (768, 256, 136, 32, True),       # group 32: first of the two-pass route
    (1535, 256, 136, 128, True),     # last row count of the ping-pong kernel
    (1536, 256, 136, 128, True),     # first of the two-pass route (dequant to bf16, dense GEMM)
    (800, 384, 264, 96, True),       # two-pass with a group that is not a power of two
    (100, 384, 136, 96, True),       # fused range, group not a power of two -> two-pass
    (1024, 1024, 512, 128, True),
    (1100, 384, 520, 128, False),
])
def test_w4a16_prefill_vs_oracle(rt, m, k, n, group, pgz):
    """Prefill rows: the dequantised weight is rounded to bf16 (RNE), inside the K-loop
    (fused kernels) or in a dequant pass before the dense GEMM (from 1536 rows on).
    Against the oracle GEMM on RNE(exact dequant) weights the result matches to fp32
    accumulation noise (this pins the in-loop dequant bit for bit up to summation order);
    against the exact-dequant oracle it is within the GEMM tolerance."""
    a, q, w, s, z = make_case(m, k, n, group, pgz, seed=0x60)
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    ref_exact = oracle.w4a16_gemm(a, w, s, z, group, 8)
    ref_rne = oracle.gemm_bf16(a, oracle.bf16_rne(wf), "nn")
    y32 = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=False)
    check(y32, ref_rne, a, wf, k, 1e-5)
    check(y32, ref_exact, a, wf, k, 5e-3)
    yb = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=True)
    check(yb, ref_exact, a, wf, k, 6e-3)


def test_w4a16_prefill_config5_full(rt):
    """BASELINE config 5 at full size (A[4096,4096] x int4 W[4096,14336], g128, per-group
    zeros, bf16 out): all 58.7M outputs against the exact-dequant oracle (the whole GEMM
    on the CPU, a few seconds with all cores) within the GEMM tolerance; the route rounds
    each dequantized weight to bf16 (as the dequant kernel does), hence the 6e-3
    relative bound."""
    m, k, n, group = 4096, 4096, 14336, 128
    a = oracle.normal_bf16((m, k), oracle.seeds(4)[0], 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), oracle.seeds(4)[1]))
    s = oracle.uniform_bf16((k // group, n), oracle.seeds(4)[2], 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), oracle.seeds(4)[3]))
    y = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=True)
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 8)
    check(y, ref, a, wf, k, 6e-3)
    assert np.isfinite(y).all()


def test_w4a16_deterministic(rt):
    m, k, n, group = 16, 4096, 1024, 128
    a, q, w, s, z = make_case(m, k, n, group, False, seed=0x90)
    y1 = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=False)
    y2 = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=False)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_w4a16_integer_exact(rt):
    """Small integer activations and power-of-two scales make every sum exact:
    the fused kernel must then match the oracle bit for bit."""
    m, k, n, group = 16, 512, 128, 128
    rng = np.random.default_rng(5)
    a = oracle.bf16_trunc(rng.integers(-3, 4, size=(m, k)).astype(np.float32))
    q = oracle.nibbles((k, n), 77)
    w = oracle.pack_qweight(q)
    s = oracle.bf16_trunc(np.full((k // group, n), 0.25, np.float32))
    zq = oracle.nibbles((k // group, n), 78)
    z = oracle.pack_qzeros(zq)
    ref = oracle.w4a16_gemm(a, w, s, z, group, 0)
    y = run_w4a16(rt, a, w, s, z, m, k, n, group, out_bf16=False)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("round_mode", [0, 1, 2])
@pytest.mark.parametrize("pgz", [False, True])
@pytest.mark.parametrize("k,n,group", [(512, 264, 128), (48, 72, 12), (96, 8, 32), (256, 2056, 64)])
def test_dequant_bit_exact(rt, round_mode, pgz, k, n, group):
    """Group 12 puts group boundaries inside k-octets; N = 2056 leaves a partial workgroup."""
    q = oracle.nibbles((k, n), 31)
    w = oracle.pack_qweight(q)
    s = oracle.uniform_bf16((k // group, n), 32, -0.05, 0.05)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), 33)) if pgz else None
    ref = oracle.dequant_qweight_f32(w, s, z, group, 8)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    pz = 0
    if z is not None:
        dz, pz = to_dev(z)
    ob = 4 if round_mode == 0 else 2
    dy, py = empty_dev(k * n * ob, fill=0)
    rt.dequant_int4(pw, ps, pz, 8, py, k, n, group, round_mode)
    if round_mode == 0:
        got = from_dev(dy, np.float32, (k, n))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    else:
        got = from_dev(dy, np.uint16, (k, n))
        want = oracle.bf16_trunc(ref) if round_mode == 1 else oracle.bf16_rne(ref)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("m", [16, 200, 800])
@pytest.mark.parametrize("out_bf16", [False, True])
def test_w4a16_k0_writes_zeros(rt, m, out_bf16):
    """K = 0 (every group divides it): the empty contraction is Y = 0 on every route
    (decode, fused, dequant-once row counts), not a division by zero or a stale Y."""
    n = 264
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xCD)
    da, pa = to_dev(np.zeros(16, np.uint16))
    dw, pw = to_dev(np.zeros(16, np.uint32))
    ds, ps = to_dev(np.zeros(16, np.uint16))
    rt.w4a16_gemm(pa, pw, ps, 0, 8, py, m, 0, n, 128, t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    y = from_dev(dy, np.uint8, (m * n * ob,))
    assert not y.any()


@pytest.mark.parametrize("m", [16, 200, 1600])
def test_w4a16_y_alignment_contract(rt, m):
    """Y must be 16-byte aligned on every route (the prefill routes store 16-byte
    vectors); an 8-byte offset is refused before anything runs, a 16-byte offset works."""
    k, n, group = 256, 136, 128
    a, q, w, s, z = make_case(m, k, n, group, True, seed=0xA0)
    da, pa = to_dev(a)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    dz, pz = to_dev(z)
    dy, py = empty_dev(m * n * 2 + 16, fill=0xCD)
    with pytest.raises(t0mi.T0miError) as e:
        rt.w4a16_gemm(pa, pw, ps, pz, 8, py + 8, m, k, n, group, t0mi.OUT_BF16)
    assert e.value.code == t0mi.ERR_INVALID and "16-byte" in str(e.value)
    rt.w4a16_gemm(pa, pw, ps, pz, 8, py + 16, m, k, n, group, t0mi.OUT_BF16)
    raw = from_dev(dy, np.uint8, (m * n * 2 + 16,))
    assert (raw[:16] == 0xCD).all()
    y = oracle.bf16_to_f32(raw[16:].view(np.uint16).reshape(m, n).copy())
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    check(y, oracle.w4a16_gemm(a, w, s, z, group, 8), a, wf, k, 6e-3)


def test_w4a16_rejects_bad_shapes(rt):
    with pytest.raises(t0mi.T0miError):
        rt.w4a16_gemm(16, 16, 16, 0, 8, 16, 16, 4096, 100, 128)   # N % 8 != 0
    with pytest.raises(t0mi.T0miError):
        rt.w4a16_gemm(16, 16, 16, 0, 8, 16, 16, 4000, 128, 128)  # K % group != 0
    with pytest.raises(t0mi.T0miError):
        rt.w4a16_gemm(16, 16, 16, 0, 8, 16, 16, 4096, 128, 48)   # group % 32 != 0


def _random_cases(n_cases=40, seed=0x5EED):
    """Seeded shapes spread over every route of t0mi_w4a16_gemm: decode slabs (up to
    191 rows by group), the fused kernels (128x128 tiles, ping-pong from 192 when K and
    the group are multiples of 64, with and without a K split), dequant-once + dense
    GEMM (1536+ rows, 768+ for other K and groups, or groups that are not powers of
    two), ragged N and K."""
    g = np.random.default_rng(seed)
    groups = [32, 64, 96, 128, 256, 512]
    out = []
    for i in range(n_cases):
        group = int(g.choice(groups))
        k = group * int(g.integers(1, max(2, 2048 // group) + 1))
        k = max(k, 32)
        n = 8 * int(g.integers(1, 160))
        m = int(g.choice([int(g.integers(1, 81)), int(g.integers(81, 1536)), int(g.integers(1536, 1700))],
                         p=[0.45, 0.4, 0.15]))
        out.append((i, m, k, n, group, bool(g.integers(0, 2)), bool(g.integers(0, 2)), int(g.integers(0, 16))))
    return out


@pytest.mark.parametrize("i,m,k,n,group,pgz,out_bf16,zp", _random_cases())
def test_w4a16_random_shapes(rt, i, m, k, n, group, pgz, out_bf16, zp):
    """Every route against the exact-dequant oracle GEMM (the fused and two-pass routes
    round the weight to bf16 first, well inside the GEMM tolerance)."""
    a, q, w, s, z = make_case(m, k, n, group, pgz, seed=0x700 + 16 * i)
    wf = oracle.dequant_qweight_f32(w, s, z, group, zp)
    ref = oracle.w4a16_gemm(a, w, s, z, group, zp)
    y = run_w4a16(rt, a, w, s, z, m, k, n, group, zp_const=zp, out_bf16=out_bf16)
    check(y, ref, a, wf, k, 6e-3)
