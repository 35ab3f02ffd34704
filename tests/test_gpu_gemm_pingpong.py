"""GPU parity tests of the ping-pong schedule of the 256x256x64 2x4-wave GEMM
configuration (csrc/gemm_pingpong.h), NN and NT, which replaces the generic
kernel for that configuration when K (per split-K partition) is a multiple of 64.

Bars:
  - bit-identical to the generic kernel of the same configuration: the generic
    kernel is run on the same problem with K padded by 8 zero columns of A and
    8 zero rows of B (K + 8 is not a multiple of 64, so the generic kernel
    runs); every accumulator then sees the same products in the same order
    plus exact zeros.  (Split-K cases are checked against the oracle and for
    run-to-run determinism only: padding K moves the partition boundaries.);
  - against the CPU oracle: integer-valued inputs exactly, random inputs
    within the GEMM tolerance 1e-2 * sqrt(K) * max|a| * max|b| (bf16 output
    within one bf16 ulp of RNE of the oracle).
Cases cover full tiles (LDS-staged bf16 store), ragged M (rows past M read as
zeros through the buffer record count, including a group with no rows), ragged
N (clamped columns), one to three K tiles (prologue-only and peeled loops),
split-K partial planes, f32 output and the bias / activation epilogue.
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


def rand_bf16(shape, seed):
    g = np.random.default_rng(seed)
    return oracle.bf16_trunc(g.standard_normal(shape).astype(np.float32))


def run(rt, a, b, m, n, k, out_bf16, split_k=1, epilogue=None, bias=None, layout=t0mi.NN):
    cfg = t0mi.preset("gfx950_256x256_k64_w2x4").copy(
        transpose=layout, split_k=split_k, out_dtype=t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    if epilogue is not None:
        cfg = cfg.copy(epilogue=epilogue)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    pbias = 0
    if bias is not None:
        dbias, pbias = to_dev(bias.astype(np.float32))
    rt.gemm(cfg, pa, pb, py, m, n, k, bias=pbias)
    return from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))


def run_generic(rt, a, b, m, n, k, out_bf16, layout=t0mi.NN, **kw):
    """Same problem through the generic kernel: K + 8 with zero padding."""
    ap = np.zeros((m, k + 8), np.uint16)
    ap[:, :k] = a
    if layout == t0mi.NN:
        bp = np.zeros((k + 8, n), np.uint16)
        bp[:k] = b
    else:
        bp = np.zeros((n, k + 8), np.uint16)
        bp[:, :k] = b
    return run(rt, ap, bp, m, n, k + 8, out_bf16, layout=layout, **kw)


def rand_b(layout, n, k, seed):
    return rand_bf16((k, n) if layout == t0mi.NN else (n, k), seed)


def lname(layout):
    return "nn" if layout == t0mi.NN else "nt"


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


CASES = [
    # (m, n, k, out_bf16, split_k)
    (512, 512, 256, True, 1),     # full tiles, staged store
    (300, 512, 192, True, 1),     # ragged M: tile row 1 has 44 rows, its group 1 has none
    (512, 392, 128, True, 1),     # ragged N: clamped B columns (NN), zero rows (NT)
    (260, 264, 64, False, 1),     # one K tile, both ragged, f32 out
    (256, 256, 8192, True, 1),    # long K
    (256, 512, 1024, False, 4),   # split-K f32 planes (256 per partition)
    (384, 256, 1536, True, 2),    # split-K, bf16 out after the reduce, ragged M
]


@pytest.mark.parametrize("layout", [t0mi.NN, t0mi.NT])
@pytest.mark.parametrize("m,n,k,out_bf16,sk", CASES)
def test_bit_identical_to_generic_kernel(rt, m, n, k, out_bf16, sk, layout):
    a = rand_bf16((m, k), 11 + m)
    b = rand_b(layout, n, k, 23 + n)
    y = run(rt, a, b, m, n, k, out_bf16, split_k=sk, layout=layout)
    if sk == 1:
        y_gen = run_generic(rt, a, b, m, n, k, out_bf16, layout=layout)
        assert np.array_equal(y, y_gen), f"{(m, n, k)}: {np.count_nonzero(y != y_gen)} elements differ"
    else:
        assert np.array_equal(y, run(rt, a, b, m, n, k, out_bf16, split_k=sk, layout=layout)), "deterministic"
    # And against the oracle, within the GEMM tolerance.
    ref = oracle.gemm_bf16(a, b, lname(layout))
    got = bf16_to_f32(y) if out_bf16 else y
    amax = np.abs(bf16_to_f32(a)).max()
    bmax = np.abs(bf16_to_f32(b)).max()
    tol = 1e-2 * np.sqrt(k) * amax * bmax
    assert np.abs(got - ref).max() <= tol


@pytest.mark.parametrize("layout", [t0mi.NN, t0mi.NT])
@pytest.mark.parametrize("m,n,k", [(512, 512, 128), (300, 392, 192)])
def test_integer_pattern_exact(rt, m, n, k, layout):
    a = oracle.bf16_trunc(((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k))
    b = oracle.bf16_trunc(((np.arange(k * n) % 5) - 2).astype(np.float32))
    b = b.reshape((k, n) if layout == t0mi.NN else (n, k))
    y = run(rt, a, b, m, n, k, False, layout=layout)
    assert np.array_equal(y, oracle.gemm_bf16(a, b, lname(layout)))
    yb = run(rt, a, b, m, n, k, True, layout=layout)
    assert np.array_equal(yb, oracle.bf16_rne(oracle.gemm_bf16(a, b, lname(layout))))


@pytest.mark.parametrize("layout", [t0mi.NN, t0mi.NT])
@pytest.mark.parametrize("epi", [t0mi.EPI_BIAS_ADD, t0mi.EPI_BIAS_ADD_RELU])
@pytest.mark.parametrize("m,n,out_bf16", [(512, 512, True), (264, 392, True), (512, 256, False)])
def test_bias_epilogue(rt, m, n, out_bf16, epi, layout):
    """GemmConfig epilogues (src/t0/gemm_gen.rs:41-49), applied before the staged store."""
    k = 256
    a = rand_bf16((m, k), 5)
    b = rand_b(layout, n, k, 6)
    bias = np.linspace(-1.0, 1.0, n).astype(np.float32)
    y = run(rt, a, b, m, n, k, out_bf16, epilogue=epi, bias=bias, layout=layout)
    y_gen = run_generic(rt, a, b, m, n, k, out_bf16, epilogue=epi, bias=bias, layout=layout)
    assert np.array_equal(y, y_gen)
    ref = oracle.gemm_bf16(a, b, lname(layout)) + bias
    if epi == t0mi.EPI_BIAS_ADD_RELU:
        ref = np.maximum(ref, 0.0)
    got = bf16_to_f32(y) if out_bf16 else y
    tol = 1e-2 * np.sqrt(k) * np.abs(bf16_to_f32(a)).max() * np.abs(bf16_to_f32(b)).max()
    assert np.abs(got - ref).max() <= tol


@pytest.mark.parametrize("preset", ["gfx950_256x256_k64_w2x4", "gfx950_128x128_k64_w2x2"])
def test_bf16_out_to_8_byte_aligned_y(rt, preset):
    """t0mi_gemm refuses a Y that is not 16-byte aligned; the reference's raw
    dispatch path (gemm_gen kernargs, gpu_context.rs:305-357) checks no
    alignment, so there full tiles with an 8-byte aligned bf16 Y take the
    direct store instead of the staged one (16 bytes per lane), with the same
    results as an aligned Y."""
    m, n, k = 512, 512, 128
    a = rand_bf16((m, k), 31)
    b = rand_bf16((k, n), 32)
    cfg = t0mi.preset(preset).copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    dy, py = empty_dev(m * n * 2 + 16, fill=0xAB)
    with pytest.raises(t0mi.T0miError) as e:
        rt.gemm(cfg, pa, pb, py + 8, m, n, k)
    assert e.value.code == t0mi.ERR_INVALID
    kern = rt.kernel(cfg)
    grid = t0mi.compute_grid_auto(cfg, m, n)
    assert rt.dispatch(kern, grid, t0mi.build_kernargs(pa, pb, py, k, n, m, cfg)) == t0mi.OK
    aligned = from_dev(dy, np.uint16, (m, n))
    tol = 1e-2 * np.sqrt(k) * np.abs(bf16_to_f32(a)).max() * np.abs(bf16_to_f32(b)).max()
    assert np.abs(bf16_to_f32(aligned) - oracle.gemm_bf16(a, b, "nn")).max() <= tol
    dy2, py2 = empty_dev(m * n * 2 + 16, fill=0xAB)
    assert rt.dispatch(kern, grid, t0mi.build_kernargs(pa, pb, py2 + 8, k, n, m, cfg)) == t0mi.OK
    raw = from_dev(dy2, np.uint8, (m * n * 2 + 16,))
    assert np.all(raw[:8] == 0xAB) and np.all(raw[8 + m * n * 2:] == 0xAB)
    assert np.array_equal(raw[8:8 + m * n * 2].view(np.uint16).reshape(m, n), aligned)


def _random_cases(n_cases=24, seed=0x9A9A):
    """Seeded shapes through the 256x256x64 configuration: ragged M and N, K a
    multiple of 64 (ping-pong) or of 8 only (generic kernel), split-K 1..8, NN
    and NT, f32 and bf16 output."""
    g = np.random.default_rng(seed)
    out = []
    for i in range(n_cases):
        m = int(g.integers(1, 700))
        n = 8 * int(g.integers(1, 90))
        k = 64 * int(g.integers(1, 24)) if g.random() < 0.75 else 8 * int(g.integers(1, 190))
        sk = int(g.choice([1, 1, 2, 4, 8]))
        layout = t0mi.NN if g.random() < 0.5 else t0mi.NT
        out.append((i, m, n, k, sk, layout, bool(g.integers(0, 2))))
    return out


@pytest.mark.parametrize("i,m,n,k,sk,layout,out_bf16", _random_cases())
def test_random_shapes(rt, i, m, n, k, sk, layout, out_bf16):
    a = rand_bf16((m, k), 1000 + i)
    b = rand_b(layout, n, k, 2000 + i)
    y = run(rt, a, b, m, n, k, out_bf16, split_k=sk, layout=layout)
    ref = oracle.gemm_bf16(a, b, lname(layout))
    got = bf16_to_f32(y) if out_bf16 else y
    tol = 1e-2 * np.sqrt(k) * np.abs(bf16_to_f32(a)).max() * np.abs(bf16_to_f32(b)).max()
    assert np.abs(got - ref).max() <= tol, (i, m, n, k, sk)
    if sk == 1 and k % 64 == 0:  # ping-pong against the generic kernel
        assert np.array_equal(y, run_generic(rt, a, b, m, n, k, out_bf16, layout=layout)), (i, m, n, k)
