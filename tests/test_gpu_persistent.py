"""GPU parity of the persistent TileGemm presets (tile_persistent_decode,
tile_persistent_128x64_k32, tile_persistent_256x128_k32; src/t0/tile_ir.rs:540-604) against
the CPU oracle, through t0mi_tile_gemm and through the reference's 64-byte persistent kernarg
dispatch.

Routes (one launch each): up to 64 rows with K a multiple of 32 (or K = 0) the persistent
decode kernel (32 x 16 units over the whole K, a grid of at most one workgroup per CU looping
over the units); above that the spec's tile kernel with a grid-stride tile loop; a persistent
spec of the caller's own whose tile has no persistent instantiation runs that tile's one-shot
kernel.  Cases are sized so the loops wrap (more units or tiles than workgroups).

Bars: integer-valued inputs bit-exact (every partial sum is exact in fp32, so any summation
order gives the oracle's value); N(0,1) inputs within max|err| <= 1e-2*sqrt(K)*max|a|*max|b|
(the kernels sum K in another order than the oracle's sequential loop); repeated calls
bit-identical (the schedule is static).
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu

EPI = [t0mi.BIAS_ADD, t0mi.SCALE, t0mi.CLAMP]


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def int_pattern(m, k, n, nn, seed=0):
    a = (((np.arange(m * k) + seed) % 7) - 3).astype(np.float32).reshape(m, k)
    b = (((np.arange(k * n) + 3 * seed) % 5) - 2).astype(np.float32)
    b = b.reshape(k, n) if nn else b.reshape(n, k)
    return oracle.bf16_trunc(a), oracle.bf16_trunc(b)


def run(rt, spec, a, b, m, n, k, bias, out_bf16=False):
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    dbias, pbias = to_dev(bias)
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    print(f"[persistent] {spec.name()} m={m} n={n} k={k} out={'bf16' if out_bf16 else 'f32'}", flush=True)
    rt.tile_gemm(spec, pa, pb, py, m, n, k, bias=pbias, scale=0.5, clamp_min=-300.0, clamp_max=400.0)
    return from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))


def reference(spec, a, b, bias, nn):
    return oracle.epilogue(oracle.gemm_bf16(a, b, "nn" if nn else "nt"), spec.epilogue_ops(), bias=bias,
                           scale=0.5, clamp_min=-300.0, clamp_max=400.0)


def spec_of(preset, nn, **kw):
    return t0mi.tile_preset(preset).copy(transpose=t0mi.NN if nn else t0mi.NT, epilogue=EPI, **kw)


# (m, n, k): row counts around the 16-row MFMA block and the 32-row unit, N tails of 8,
# K = 0, K ranges that leave waves empty or split unevenly (17 and 300 k-blocks over 16
# waves), and unit counts above the grid (the persistent loop wraps).
DECODE_CASES = [
    (1, 8, 32), (1, 4096, 4096), (2, 24, 64), (15, 40, 96), (16, 4096, 4096), (17, 200, 544),
    (31, 16, 512), (32, 136, 9600), (33, 72, 128), (48, 264, 256), (63, 8, 1024), (64, 11008, 512),
    (16, 33280, 256), (5, 64, 0),
]


@pytest.mark.parametrize("nn", [0, 1])
@pytest.mark.parametrize("m,n,k", DECODE_CASES)
def test_decode_kernel_integer_exact(rt, m, n, k, nn):
    spec = spec_of("tile_persistent_decode", nn)
    a, b = int_pattern(m, k, n, nn, seed=m + n)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    y = run(rt, spec, a, b, m, n, k, bias)
    assert np.array_equal(y, reference(spec, a, b, bias, nn))


@pytest.mark.parametrize("nn", [0, 1])
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (16, 4096, 4096), (40, 1000, 2048)])
def test_decode_kernel_random_tolerance(rt, m, n, k, nn):
    spec = spec_of("tile_persistent_decode", nn).copy(epilogue=[])
    a = oracle.normal_bf16((m, k), 11 + m, 0.0, 1.0)
    b = oracle.normal_bf16((k, n) if nn else (n, k), 12 + n, 0.0, 1.0)
    bias = np.zeros(n, np.float32)
    y = run(rt, spec, a, b, m, n, k, bias)
    ref = oracle.gemm_bf16(a, b, "nn" if nn else "nt")
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    err = np.abs(y - ref)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    print(f"[persistent] max|err| {err.max():.3e} (bound {tol:.3e}), rel Frobenius {rel:.2e}", flush=True)
    assert err.max() <= tol


@pytest.mark.parametrize("nn", [0, 1])
def test_decode_kernel_bf16_out(rt, nn):
    # bf16 output: the f32 result rounded to nearest even, exact on the integer pattern
    m, n, k = 16, 520, 1024
    spec = spec_of("tile_persistent_decode", nn, out_dtype=t0mi.OUT_BF16)
    a, b = int_pattern(m, k, n, nn, seed=5)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    y = run(rt, spec, a, b, m, n, k, bias, out_bf16=True)
    assert np.array_equal(y, oracle.bf16_rne(reference(spec, a, b, bias, nn)))


@pytest.mark.parametrize("nn", [0, 1])
def test_decode_kernel_deterministic(rt, nn):
    m, n, k = 16, 4096, 4096
    spec = spec_of("tile_persistent_decode", nn).copy(epilogue=[])
    a = oracle.normal_bf16((m, k), 21, 0.0, 1.0)
    b = oracle.normal_bf16((k, n) if nn else (n, k), 22, 0.0, 1.0)
    bias = np.zeros(n, np.float32)
    y0 = run(rt, spec, a, b, m, n, k, bias)
    y1 = run(rt, spec, a, b, m, n, k, bias)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


# Above 64 rows, or K not a multiple of 32: the spec's tile kernel with the grid-stride loop.
# The large cases have more tiles than the GPU holds workgroups of that kernel at once, so the
# loop wraps: 32 x 64 tiles 8192 (about 20 workgroups per CU fit), 128 x 64 tiles 2048 (6 per
# CU), 256 x 128 tiles 1024 (2 per CU).
TILE_CASES = [
    ("tile_persistent_decode", 65, 200, 96), ("tile_persistent_decode", 16, 136, 40),
    ("tile_persistent_decode", 4096, 4096, 32), ("tile_persistent_128x64_k32", 130, 192, 128),
    ("tile_persistent_128x64_k32", 1000, 1000, 264), ("tile_persistent_128x64_k32", 4096, 4096, 32),
    ("tile_persistent_256x128_k32", 8192, 4096, 32), ("tile_persistent_256x128_k32", 300, 520, 72),
]


@pytest.mark.parametrize("nn", [0, 1])
@pytest.mark.parametrize("preset,m,n,k", TILE_CASES)
def test_tile_loop_integer_exact(rt, preset, m, n, k, nn):
    spec = spec_of(preset, nn)
    a, b = int_pattern(m, k, n, nn, seed=k)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    y = run(rt, spec, a, b, m, n, k, bias)
    assert np.array_equal(y, reference(spec, a, b, bias, nn))


@pytest.mark.parametrize("nn", [0, 1])
def test_caller_persistent_spec_without_tile_loop(rt, nn):
    # tile_64x64_k32 made persistent by the caller: the decode kernel at 16 rows, the
    # 64x64 tile's one-shot kernel at 100 rows; both one plane, split-K ignored as the
    # reference's persistent lowering does (split_k_id = 0).
    spec = t0mi.tile_preset("tile_64x64_k32").copy(transpose=t0mi.NN if nn else t0mi.NT, epilogue=EPI,
                                                   persistent=1, split_k=2)
    for m, n, k in ((16, 192, 256), (100, 192, 256)):
        a, b = int_pattern(m, k, n, nn, seed=m)
        bias = ((np.arange(n) % 9) - 4).astype(np.float32)
        y = run(rt, spec, a, b, m, n, k, bias)
        assert np.array_equal(y, reference(spec, a, b, bias, nn))


def test_persistent_dispatch_kernarg(rt):
    # The reference's dispatch path for a persistent spec: 64-byte kernarg with the counter
    # slot (build_kernargs_m_with_counter, tile_ir.rs:4604-4637), grid [wg_size, 1, 1]
    # (compute_grid, :4645-4652), epilogue arguments after it.
    spec = spec_of("tile_persistent_decode", 0)
    m, n, k = 16, 4096, 1024
    a, b = int_pattern(m, k, n, False, seed=9)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    dbias, pbias = to_dev(bias)
    dy, py = empty_dev(m * n * 4, fill=0xAB)
    dcnt, pcnt = empty_dev(4096, fill=0)
    kern = rt.tile_kernel(spec)
    ka = t0mi.tile_build_kernargs_m_with_counter(pa, pb, py, k, n, m, spec, pcnt, (n // 64).bit_length() - 1,
                                                 (m // 32 + 1) * (n // 64))
    assert len(ka) == 64
    ka = t0mi.tile_append_epilogue_args(spec, ka, bias=pbias, scale=0.5, clamp_min=-300.0, clamp_max=400.0)
    grid = t0mi.tile_compute_grid(spec, m, n)
    assert list(grid) == [spec.wg_size(), 1, 1]
    assert rt.dispatch(kern, grid, ka) == 0, t0mi.last_error()
    y = from_dev(dy, np.float32, (m, n))
    assert np.array_equal(y, reference(spec, a, b, bias, False))
    # the counter is the reference's bookkeeping slot: the gfx950 schedule leaves it untouched
    assert not from_dev(dcnt, np.uint8, (4096,)).any()


def _random_persistent_cases(n_cases=24, seed=0x9E75):
    """Seeded ragged shapes for the three persistent presets: rows 1..300 (both kernels), N and
    K multiples of 8 (K not always a multiple of 32, so the decode rows take the tile loop)."""
    g = np.random.default_rng(seed)
    presets = ["tile_persistent_decode", "tile_persistent_128x64_k32", "tile_persistent_256x128_k32"]
    out = []
    for i in range(n_cases):
        m = int(g.choice([int(g.integers(1, 65)), int(g.integers(65, 300))]))
        n = 8 * int(g.integers(1, 200))
        k = 8 * int(g.integers(0, 160))
        out.append((i, presets[i % 3], m, n, k, int(g.integers(0, 2))))
    return out


@pytest.mark.parametrize("i,preset,m,n,k,nn", _random_persistent_cases())
def test_random_shapes_integer_exact(rt, i, preset, m, n, k, nn):
    # integer inputs: every route (decode kernel, tile loop) must give the oracle's exact values
    spec = spec_of(preset, nn)
    a, b = int_pattern(m, k, n, nn, seed=i)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    y = run(rt, spec, a, b, m, n, k, bias)
    assert np.array_equal(y, reference(spec, a, b, bias, nn))
