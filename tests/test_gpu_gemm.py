"""GPU parity tests of the bf16 GEMM (HIP kernels through the C ABI) against the CPU oracle.

Bars:
  - integer-valued inputs: bit-exact (every partial sum is an exactly
    representable integer, so any summation order gives the same result);
  - random inputs: max|err| <= 1e-2 * sqrt(K) * max|a| * max|b|, relative
    Frobenius error reported and bounded;
  - bf16 output: within 1 bf16 ulp of RNE(oracle) — the GPU's fp32 sum order
    differs from the oracle's sequential order, so the pre-rounding value can
    straddle a rounding boundary.
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu

GOLD = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "torch_ref")


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def int_pattern(m, k, n, nn):
    """a = (i%7)-3 over A's flat index; b = (j%5)-2 over B's flat index
    (src/t0/auto_gemm.rs:235-238): all sums exact in fp32 for these sizes."""
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(k * n) % 5) - 2).astype(np.float32)
    b = b.reshape(k, n) if nn else b.reshape(n, k)
    return oracle.bf16_trunc(a), oracle.bf16_trunc(b)


def run_gemm(rt, cfg, a, b, m, n, k, out_bf16=False, bias=None):
    cfg = cfg.copy(out_dtype=t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    pbias = 0
    if bias is not None:
        dbias, pbias = to_dev(bias.astype(np.float32))
    rt.gemm(cfg, pa, pb, py, m, n, k, bias=pbias)
    return from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))


ALL_VARIANTS = [
    ("tile_32x64_k16", 0, 0), ("tile_64x64_k32", 0, 0), ("tile_128x64_k16", 0, 0), ("tile_64x128_k16", 0, 0),
    ("tile_128x128_k16", 0, 0), ("tile_64x64_k64", 0, 0), ("tile_32x128_k16", 0, 0), ("tile_32x64_k32", 0, 0),
    ("tile_128x64_k32", 0, 0), ("tile_64x64_k16", 0, 0),
    ("gfx950_256x256_k64_w2x4", 0, 0), ("gfx950_256x128_k64_w2x2", 0, 0), ("gfx950_128x256_k64_w2x2", 0, 0),
    ("gfx950_128x128_k64_w2x2", 0, 0), ("gfx950_128x64_k64_w2x2", 0, 0), ("gfx950_64x128_k64_w2x2", 0, 0),
    ("gfx950_64x64_k64_w2x2", 0, 0), ("gfx950_128x128_k32_w2x2", 0, 0),
]


@pytest.mark.parametrize("layout", [t0mi.NT, t0mi.NN])
@pytest.mark.parametrize("name", [v[0] for v in ALL_VARIANTS])
def test_integer_pattern_exact_all_variants(rt, name, layout):
    # Ragged M and N (not tile multiples), K not a multiple of tile_k.
    m, n, k = 200, 136, 264
    cfg = t0mi.preset(name).copy(transpose=layout)
    a, b = int_pattern(m, k, n, layout == t0mi.NN)
    y = run_gemm(rt, cfg, a, b, m, n, k)
    ref = oracle.gemm_bf16(a, b, "nn" if layout == t0mi.NN else "nt")
    assert np.array_equal(y, ref), f"{cfg.name()}: max diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("layout", [t0mi.NT, t0mi.NN])
@pytest.mark.parametrize("name", [v[0] for v in ALL_VARIANTS])
def test_integer_pattern_bf16_out_all_variants(rt, name, layout):
    """bf16 output: interior tiles take the LDS-staged whole-row store, edge
    tiles the direct one; both must equal RNE of the exact integer sums."""
    m, n, k = 520, 264, 128
    cfg = t0mi.preset(name).copy(transpose=layout)
    a, b = int_pattern(m, k, n, layout == t0mi.NN)
    y = run_gemm(rt, cfg, a, b, m, n, k, out_bf16=True)
    ref = oracle.bf16_rne(oracle.gemm_bf16(a, b, "nn" if layout == t0mi.NN else "nt"))
    assert np.array_equal(y, ref), f"{cfg.name()}: {np.count_nonzero(y != ref)} elements differ"


PREBUILT = t0mi.variants()


@pytest.mark.parametrize("idx", range(len(PREBUILT)))
def test_every_prebuilt_kernel_integer_exact(rt, idx):
    """Every kernel of the prebuilt table (tile, wave layout, LDS stages; each layout), also those
    no preset names: ragged M and N, K not a multiple of tile_k, f32 out, equal to the exact
    integer sums."""
    cfg = PREBUILT[idx]
    m, n, k = 200, 136, 264
    a, b = int_pattern(m, k, n, cfg.transpose == t0mi.NN)
    print(f"[prebuilt {idx}] {cfg.name()}", flush=True)
    y = run_gemm(rt, cfg, a, b, m, n, k)
    ref = oracle.gemm_bf16(a, b, "nn" if cfg.transpose == t0mi.NN else "nt")
    assert np.array_equal(y, ref), f"{cfg.name()}: max diff {np.abs(y - ref).max()}"


@pytest.mark.parametrize("layout", [t0mi.NT, t0mi.NN])
@pytest.mark.parametrize("sk", [2, 4, 8])
def test_split_k_exact_and_deterministic(rt, layout, sk):
    m, n, k = 128, 256, 1024
    cfg = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=layout, split_k=sk)
    a, b = int_pattern(m, k, n, layout == t0mi.NN)
    y1 = run_gemm(rt, cfg, a, b, m, n, k)
    ref = oracle.gemm_bf16(a, b, "nn" if layout == t0mi.NN else "nt")
    assert np.array_equal(y1, ref)
    # Random data: two runs are bitwise identical (fixed partition order).
    ar = oracle.normal_bf16((m, k), 11, 0.0, 1.0)
    br = oracle.normal_bf16((k, n) if layout == t0mi.NN else (n, k), 12, 0.0, 1.0)
    r1 = run_gemm(rt, cfg, ar, br, m, n, k)
    r2 = run_gemm(rt, cfg, ar, br, m, n, k)
    assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))


def _check_tol(y, ref, a, b, k, rel_max=1e-5):
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    err, rel = oracle.compare(y, ref)
    assert err <= tol, f"max|err| {err} > tol {tol}"
    assert rel <= rel_max, f"relative Frobenius error {rel}"
    return err, rel


def test_torch_fixtures_nt(rt):
    """benchmarks/torch_ref (M=64, K=256, N=512, NT): h = x . w^T against torch's fp32
    result and against the bf16-rounded torch result."""
    x = np.fromfile(f"{GOLD}/x.bin", np.uint16).reshape(64, 256)
    for w_name, ref_name, bf_name in (("w_gate", "h_gate_f32ref", "h_gate_bf16acc"),
                                      ("w_up", "h_up_f32ref", "h_up_bf16acc")):
        w = np.fromfile(f"{GOLD}/{w_name}.bin", np.uint16).reshape(512, 256)
        ref = np.fromfile(f"{GOLD}/{ref_name}.bin", np.float32).reshape(64, 512)
        bfr = np.fromfile(f"{GOLD}/{bf_name}.bin", np.float32).reshape(64, 512)
        for name in ("tile_64x64_k32", "gfx950_128x128_k64_w2x2", "gfx950_256x256_k64_w2x4"):
            cfg = t0mi.preset(name)
            y = run_gemm(rt, cfg, x, w, 64, 512, 256)
            assert np.abs(y - ref).max() < 2e-6, name
            yb = run_gemm(rt, cfg, x, w, 64, 512, 256, out_bf16=True).astype(np.int32)
            # within one bf16 ulp of torch's bf16 result (bits compared as integers;
            # all values share a sign with their reference or are tiny); almost all identical
            d = np.abs(yb - oracle.bf16_rne(bfr).astype(np.int32))
            assert d.max() <= 1, name
            assert (d == 0).mean() > 0.99, name


def test_torch_fixture_down_projection(rt):
    s = np.fromfile(f"{GOLD}/swiglu_bf16_trunc.bin", np.uint16).reshape(64, 512)
    wd = np.fromfile(f"{GOLD}/w_down.bin", np.uint16).reshape(256, 512)
    ref = np.fromfile(f"{GOLD}/y_bf16_f32acc.bin", np.float32).reshape(64, 256)
    y = run_gemm(rt, t0mi.preset("gfx950_64x64_k64_w2x2"), s, wd, 64, 256, 512)
    assert np.abs(y - ref).max() < 2e-6


@pytest.mark.parametrize("layout", [t0mi.NT, t0mi.NN])
def test_config1_256_uniform(rt, layout):
    """256^3, U(-1,1) bf16, f32 out."""
    m = n = k = 256
    a0, b0, _, _ = oracle.seeds(0)
    a = oracle.uniform_bf16((m, k), a0, -1.0, 1.0)
    b = oracle.uniform_bf16((k, n) if layout == t0mi.NN else (n, k), b0, -1.0, 1.0)
    ref = oracle.gemm_bf16(a, b, "nn" if layout == t0mi.NN else "nt")
    for name in ("tile_64x64_k16", "gfx950_64x64_k64_w2x2", "gfx950_128x128_k64_w2x2"):
        cfg = t0mi.preset(name).copy(transpose=layout)
        y = run_gemm(rt, cfg, a, b, m, n, k)
        _check_tol(y, ref, a, b, k)


def test_bias_relu_epilogue(rt):
    m, n, k = 96, 128, 192
    a = oracle.normal_bf16((m, k), 21, 0.0, 1.0)
    b = oracle.normal_bf16((n, k), 22, 0.0, 1.0)
    bias = np.linspace(-3, 3, n).astype(np.float32)
    ref = oracle.gemm_bf16(a, b, "nt")
    for epi in (t0mi.EPI_BIAS_ADD, t0mi.EPI_BIAS_ADD_RELU):
        cfg = t0mi.preset("gfx950_64x64_k64_w2x2").copy(epilogue=epi)
        y = run_gemm(rt, cfg, a, b, m, n, k, bias=bias)
        want = ref + bias[None, :]
        if epi == t0mi.EPI_BIAS_ADD_RELU:
            want = np.maximum(want, 0)
        _check_tol(y, want, a, b, k)
        for sk in (2, 4):
            y2 = run_gemm(rt, cfg.copy(split_k=sk), a, b, m, n, k, bias=bias)
            _check_tol(y2, want, a, b, k)


def test_bench_shape_4096_full(rt):
    """BASELINE config 2 at full size: 4096^3 NN, N(0,1), bf16 out, the bench's kernel.
    Every one of the 16.7M outputs against the oracle (the whole GEMM on the CPU, ~1 s
    with all cores): within one bf16 rounding of the fp32 result plus the GEMM tolerance,
    and the relative Frobenius error bounded; the row sums (sum_j y[i,j] vs
    a[i,:] . rowsum(B)) as a size-independent property."""
    m = n = k = 4096
    a0, b0, _, _ = oracle.seeds(1)
    a = oracle.normal_bf16((m, k), a0, 0.0, 1.0)
    b = oracle.normal_bf16((k, n), b0, 0.0, 1.0)
    cfg = t0mi.preset("gfx950_256x256_k64_w2x4").copy(transpose=t0mi.NN)
    y = oracle.bf16_to_f32(run_gemm(rt, cfg, a, b, m, n, k, out_bf16=True))
    ref = oracle.gemm_bf16(a, b, "nn")
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    err, rel = oracle.compare(y, ref)
    assert err <= tol and rel < 5e-3, (err, rel)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + tol)
    # full-size property: row sums
    bsum = oracle.bf16_to_f32(b).astype(np.float64).sum(axis=1)
    want = oracle.bf16_to_f32(a).astype(np.float64) @ bsum
    got = y.astype(np.float64).sum(axis=1)
    scale = np.abs(want).max() + 1.0
    assert np.abs(got - want).max() / scale < 2e-2


def test_skinny_shape_sampled(rt):
    """M=128, N=4096, K=4096, N(0,0.02), bf16 out, with the auto-selected config."""
    m, n, k = 128, 4096, 4096
    a0, b0, _, _ = oracle.seeds(2)
    a = oracle.normal_bf16((m, k), a0, 0.0, 0.02)
    b = oracle.normal_bf16((k, n), b0, 0.0, 0.02)
    cfg = t0mi.auto_select(m, k, n).copy(transpose=t0mi.NN)
    y = oracle.bf16_to_f32(run_gemm(rt, cfg, a, b, m, n, k, out_bf16=True))
    ref = oracle.gemm_bf16(a, b, "nn")
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    err, rel = oracle.compare(y, ref)
    assert err <= tol and rel < 5e-3, (cfg.name(), err, rel)


def test_reference_dispatch_path(rt):
    """The drop-in path: kernel_get + build_kernargs + compute_grid_auto + dispatch, with
    the reference's padding contract, on the smoke-test pattern (auto_gemm.rs:223-272)."""
    import t0mi as T
    for name, sk in (("tile_128x64_k16", 1), ("tile_64x64_k32", 1), ("gfx950_128x128_k64_w2x2", 2)):
        cfg = T.preset(name).copy(split_k=sk)
        m, k, n = 128, 128, 128
        a, b = int_pattern(m, k, n, False)
        da, pa = to_dev(a)
        db, pb = to_dev(b)
        dy, py = empty_dev(m * n * 4 * sk, fill=0)
        kern = rt.kernel(cfg)
        ka = T.build_kernargs(pa, pb, py, k, n, m, cfg)
        assert len(ka) == kern.attrs()["kernarg_size"]
        grid = T.compute_grid_auto(cfg, m, n)
        assert rt.dispatch(kern, grid, ka) == 0, T.last_error()
        planes = from_dev(dy, np.float32, (sk, m, n))
        ref = oracle.gemm_bf16(a, b, "nt")
        # split-K writes one partial plane per partition (no reduction), as the reference.
        assert np.array_equal(planes.sum(axis=0, dtype=np.float32) if sk > 1 else planes[0], ref)
    # kernarg length mismatch is refused (gpu_context.rs:319-323)
    cfg = T.preset("tile_64x64_k32")
    kern = rt.kernel(cfg)
    assert rt.dispatch(kern, (64, 1), b"\0" * 44) == T.ERR_KERNARG


def test_auto_gemm_known_answer(rt):
    """auto_gemm.rs:655: Y[0,0] = -6 at (m, k, n) = (128, 64, 128) with the integer pattern."""
    m, k, n = 128, 64, 128
    a, b = int_pattern(m, k, n, False)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    dy, py = empty_dev(m * n * 4, fill=0)
    cfg = t0mi.auto_select(m, k, n)
    rt.gemm(cfg, pa, pb, py, m, n, k)
    y = from_dev(dy, np.float32, (m, n))
    assert y[0, 0] == -6.0
    assert np.array_equal(y, oracle.gemm_bf16(a, b, "nt"))


def _random_gemm_cases(n_cases=30, seed=0xC0FFEE):
    """Seeded ragged shapes (K and N multiples of 8), both layouts and output types; the
    config is the cost model's choice for the shape, or a forced split-K variant."""
    g = np.random.default_rng(seed)
    out = []
    for i in range(n_cases):
        m = int(g.integers(1, 700))
        n = 8 * int(g.integers(1, 90))
        k = 8 * int(g.integers(1, 300))
        out.append((i, m, n, k, int(g.integers(0, 2)), bool(g.integers(0, 2)), int(g.choice([0, 0, 2, 4]))))
    return out


@pytest.mark.parametrize("i,m,n,k,layout,out_bf16,sk", _random_gemm_cases())
def test_random_shapes_auto_selected(rt, i, m, n, k, layout, out_bf16, sk):
    nn = layout == t0mi.NN
    a = oracle.normal_bf16((m, k), 0x900 + 2 * i, 0.0, 1.0)
    b = oracle.normal_bf16((k, n) if nn else (n, k), 0x901 + 2 * i, 0.0, 1.0)
    cfg = t0mi.auto_select_layout(m, k, n, layout, t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    if sk:
        cfg = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=layout, split_k=sk)
    y = run_gemm(rt, cfg, a, b, m, n, k, out_bf16=out_bf16)
    ref = oracle.gemm_bf16(a, b, "nn" if nn else "nt")
    if out_bf16:
        # the GEMM tolerance plus one bf16 rounding step of the output
        tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
        yf = oracle.bf16_to_f32(y)
        assert np.all(np.abs(yf - ref) <= tol + np.abs(ref) * 2.0**-8), cfg.name()
    else:
        _check_tol(y, ref, a, b, k)


def _pad(x, rows, cols):
    out = np.zeros((rows, cols), x.dtype)
    out[:x.shape[0], :x.shape[1]] = x
    return out


@pytest.mark.parametrize("m", [1, 16, 17])
def test_reference_small_m_preset_dispatch(rt, m):
    """GemmConfig::tile_16x64_k16 (gemm_gen.rs:88-90: 16 rows, wg_size 32, wave32) is what
    select_config picks for m <= 16 (bf16_matmul.rs:140-149).  Through kernel_get +
    build_kernargs + compute_grid_auto + dispatch with the reference's padding contract
    (X, WT and Y padded to whole 16 x 64 tiles, K to 16; bf16_matmul.rs:171-199): the grid
    is in work-items of its 32-thread workgroups and defines M; results equal the oracle."""
    cfg = t0mi.preset("tile_16x64_k16")
    n, k = 200, 264
    a0, b0, _, _ = oracle.seeds(16 + m)
    a = oracle.normal_bf16((m, k), a0, 0.0, 1.0)
    wt = oracle.normal_bf16((n, k), b0, 0.0, 1.0)
    mp, np_, kp = -(-m // 16) * 16, -(-n // 64) * 64, -(-k // 16) * 16
    da, pa = to_dev(_pad(a, mp, kp))
    db, pb = to_dev(_pad(wt, np_, kp))
    dy, py = empty_dev(mp * np_ * 4, fill=0xAB)
    kern = rt.kernel(cfg)
    assert kern.name == "t0_gemm_16x64_k16_ldsdb_wgp"
    assert kern.attrs()["wg_size"] == 32
    ka = t0mi.build_kernargs(pa, pb, py, kp, np_, mp, cfg)
    grid = t0mi.compute_grid_auto(cfg, mp, np_)
    assert grid == ((np_ // 64) * 32, mp // 16)
    assert rt.dispatch(kern, grid, ka) == 0, t0mi.last_error()
    y = from_dev(dy, np.float32, (mp, np_))
    ref = oracle.gemm_bf16(_pad(a, mp, kp), _pad(wt, np_, kp), "nt")
    err, rel = oracle.compare(y, ref)
    tol = oracle.gemm_tolerance(kp, oracle.bf16_to_f32(a), oracle.bf16_to_f32(wt))
    assert err <= tol and rel < 1e-5, (m, err, rel)
    assert not y[m:].any() and not y[:, n:].any(), "padding rows/columns are zero products"


@pytest.mark.parametrize("nn", [0, 1])
@pytest.mark.parametrize("out_bf16", [False, True])
def test_reference_small_m_preset_gemm(rt, nn, out_bf16):
    """t0mi_gemm with tile_16x64_k16 on ragged shapes (no padding), both layouts and outputs:
    integer pattern, bit-exact."""
    cfg = t0mi.preset("tile_16x64_k16").copy(transpose=nn)
    for m, n, k in ((1, 136, 264), (16, 64, 128), (17, 200, 520)):
        a, b = int_pattern(m, k, n, nn)
        y = run_gemm(rt, cfg, a, b, m, n, k, out_bf16=out_bf16)
        ref = oracle.gemm_bf16(a, b, "nn" if nn else "nt")
        if out_bf16:
            ref = oracle.bf16_rne(ref)
        assert np.array_equal(y, ref), (m, n, k)


@pytest.mark.parametrize("m", [1, 16, 17])
def test_reference_k48_tile_dispatch(rt, m):
    """TileGemm::tile_128x128_k48 (tile_ir.rs:316) through tile_kernel + build_kernargs_m +
    compute_grid + dispatch (run as three 16-K steps of the 128x128 kernel), and through
    tile_gemm, against the oracle: integer pattern, bit-exact."""
    spec = t0mi.tile_preset("tile_128x128_k48")
    n, k = 136, 240
    a, b = int_pattern(m, k, n, False)
    tm = -(-m // 128) * 128
    da, pa = to_dev(_pad(a, tm, k))
    db, pb = to_dev(b)
    dy, py = empty_dev(m * n * 4, fill=0xAB)
    kern = rt.tile_kernel(spec)
    ka = t0mi.tile_build_kernargs_m(pa, pb, py, k, n, m, spec)
    assert len(ka) == kern.attrs()["kernarg_size"] == 44
    assert rt.dispatch(kern, t0mi.tile_compute_grid(spec, m, n), ka) == 0, t0mi.last_error()
    ref = oracle.gemm_bf16(a, b, "nt")
    assert np.array_equal(from_dev(dy, np.float32, (m, n)), ref)
    dy2, py2 = empty_dev(m * n * 4, fill=0xAB)
    rt.tile_gemm(spec, pa, pb, py2, m, n, k)
    assert np.array_equal(from_dev(dy2, np.float32, (m, n)), ref)


@pytest.mark.parametrize("m,n,k,layout", [(128, 1024, 1024, t0mi.NN), (16, 1000, 2048, t0mi.NT),
                                          (600, 520, 776, t0mi.NN), (3000, 2048, 512, t0mi.NT)])
def test_ranked_candidates_integer_exact(rt, m, n, k, layout):
    """Every configuration the cost model ranks in its first 12 for a shape (the candidates
    GemmTuner times and may pick; cost_model.rs:464-534) computes the exact integer result,
    split-K partitions included."""
    nn = layout == t0mi.NN
    a = oracle.bf16_trunc((((np.arange(m * k) % 7) - 3).astype(np.float32)).reshape(m, k))
    b = oracle.bf16_trunc((((np.arange(k * n) % 5) - 2).astype(np.float32)).reshape((k, n) if nn else (n, k)))
    ref = oracle.gemm_bf16(a, b, "nn" if nn else "nt")
    for cfg, _ in t0mi.auto_schedule_gemm(m, n, k, layout, t0mi.OUT_F32, cap=12):
        print(f"[gemm] ranked {cfg.name()} {m}x{n}x{k}", flush=True)
        y = run_gemm(rt, cfg, a, b, m, n, k)
        assert np.array_equal(y, ref), cfg.name()
