"""GPU parity of the tile_ir surface (TileGemm lowered to the gfx950 kernels) against
the CPU oracle: every lowerable preset, the fused epilogue chain, the reference's
kernarg / grid dispatch path, persistent specs and split-K.

Bars: integer-valued inputs bit-exact (every partial sum is exact in fp32); random
inputs within max|err| <= 1e-2*sqrt(K)*max|a|*max|b| before the epilogue, and for the
transcendental ops (SiLU, GELU) within that bound plus 1e-5 relative (the GPU uses
the hardware exp2 / rcp approximations, as the reference's v_exp_f32 / v_rcp_f32 do).
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu

PRESETS = t0mi.tile_preset_names()


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def int_pattern(m, k, n, nn):
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(k * n) % 5) - 2).astype(np.float32)
    b = b.reshape(k, n) if nn else b.reshape(n, k)
    return oracle.bf16_trunc(a), oracle.bf16_trunc(b)


def run_tile(rt, spec, a, b, m, n, k, bias=None, scale=1.0, lo=0.0, hi=0.0):
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    ob = 2 if spec.out_dtype == t0mi.OUT_BF16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    pbias = 0
    if bias is not None:
        dbias, pbias = to_dev(bias.astype(np.float32))
    rt.tile_gemm(spec, pa, pb, py, m, n, k, bias=pbias, scale=scale, clamp_min=lo, clamp_max=hi)
    return from_dev(dy, np.uint16 if ob == 2 else np.float32, (m, n))


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("nn", [0, 1])
def test_presets_integer_exact(rt, preset, nn):
    # NN tiles narrower than 64 columns run on the 64-column NN kernel; tile_k 48 as three 16-K steps.
    spec = t0mi.tile_preset(preset).copy(transpose=nn)
    m, n, k = 200, 136, 264
    a, b = int_pattern(m, k, n, nn)
    y = run_tile(rt, spec, a, b, m, n, k)
    ref = oracle.gemm_bf16(a, b, "nn" if nn else "nt")
    assert np.array_equal(y, ref), preset


OPS = [("bias", [t0mi.BIAS_ADD]), ("scale", [t0mi.SCALE]), ("relu", [t0mi.RELU]), ("silu", [t0mi.SILU]),
       ("gelu", [t0mi.GELU]), ("abs", [t0mi.ABS]), ("neg", [t0mi.NEG]), ("clamp", [t0mi.CLAMP]),
       ("bias_relu", [t0mi.BIAS_ADD, t0mi.RELU]),
       ("chain", [t0mi.BIAS_ADD, t0mi.SCALE, t0mi.SILU, t0mi.NEG, t0mi.CLAMP, t0mi.ABS])]


@pytest.mark.parametrize("label,ops", OPS)
@pytest.mark.parametrize("split_k", [1, 4])
def test_epilogue_chain(rt, label, ops, split_k):
    m, n, k = 96, 200, 512
    a = oracle.normal_bf16((m, k), 11, 0.0, 1.0)
    b = oracle.normal_bf16((k, n), 12, 0.0, 1.0)
    bias = np.linspace(-3, 3, n).astype(np.float32)
    scale, lo, hi = 0.37, -2.5, 4.0
    spec = t0mi.tile_preset("tile_64x64_k32").copy(transpose=t0mi.NN, split_k=split_k, epilogue=ops)
    y = run_tile(rt, spec, a, b, m, n, k, bias=bias, scale=scale, lo=lo, hi=hi)
    acc = oracle.gemm_bf16(a, b, "nn")
    ref = oracle.epilogue(acc, ops, bias=bias, scale=scale, clamp_min=lo, clamp_max=hi)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    # every op is 1-Lipschitz except scale (|s| < 1 here): the GEMM bound carries through
    err, rel = oracle.compare(y, ref)
    assert err <= tol + 1e-5 * float(np.abs(ref).max()), (label, err, tol)
    assert rel < 1e-4, (label, rel)


def test_epilogue_bf16_out(rt):
    m, n, k = 64, 128, 256
    a = oracle.normal_bf16((m, k), 21, 0.0, 1.0)
    b = oracle.normal_bf16((n, k), 22, 0.0, 1.0)
    ops = [t0mi.BIAS_ADD, t0mi.GELU]
    bias = np.linspace(-1, 1, n).astype(np.float32)
    spec = t0mi.tile_preset("tile_128x64_k16").copy(out_dtype=t0mi.OUT_BF16, epilogue=ops)
    y = oracle.bf16_to_f32(run_tile(rt, spec, a, b, m, n, k, bias=bias))
    ref = oracle.epilogue(oracle.gemm_bf16(a, b, "nt"), ops, bias=bias)
    # within one bf16 ulp of the fp32 reference (plus the GEMM bound)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + tol)


def dispatch_case(rt, spec, m, n, k, use_m=True, persistent_counter=False):
    nn = spec.transpose == t0mi.NN
    a, b = int_pattern(m, k, n, nn)
    bias = ((np.arange(n) % 9) - 4).astype(np.float32)
    tm = -(-m // spec.tile_m) * spec.tile_m
    # X padded to whole tiles, as the reference's callers pad it (src/ignis/ops/bf16_matmul.rs:171-199):
    # with M = 0 in the kernarg the grid's rows are read.
    ap = np.zeros((tm, k), np.uint16)
    ap[:m] = a
    da, pa = to_dev(ap)
    db, pb = to_dev(b)
    dbias, pbias = to_dev(bias)
    dy, py = empty_dev(tm * n * 4, fill=0xAB)
    kern = rt.tile_kernel(spec)
    if persistent_counter:
        ka = t0mi.tile_build_kernargs_m_with_counter(pa, pb, py, k, n, m, spec, 0, 0, 0)
    elif use_m:
        ka = t0mi.tile_build_kernargs_m(pa, pb, py, k, n, m, spec)
    else:
        ka = t0mi.tile_build_kernargs(pa, pb, py, k, n, spec)
    ka = t0mi.tile_append_epilogue_args(spec, ka, bias=pbias, scale=2.0, clamp_min=-50.0, clamp_max=60.0)
    grid = t0mi.tile_compute_grid(spec, m, n)
    assert rt.dispatch(kern, grid, ka) == 0, t0mi.last_error()
    rows = m if use_m else tm
    y = from_dev(dy, np.float32, (rows, n))
    ar = np.zeros((rows, k), np.uint16)
    ar[:m] = a
    ref = oracle.epilogue(oracle.gemm_bf16(ar, b, "nn" if nn else "nt"), spec.epilogue_ops(), bias=bias,
                          scale=2.0, clamp_min=-50.0, clamp_max=60.0)
    return y, ref


def test_dispatch_path_with_m(rt):
    spec = t0mi.tile_preset("tile_128x64_k32").copy(epilogue=[t0mi.BIAS_ADD, t0mi.SCALE, t0mi.CLAMP])
    y, ref = dispatch_case(rt, spec, 200, 136, 264)
    assert np.array_equal(y, ref)


def test_dispatch_path_m_placeholder_uses_grid_rows(rt):
    # build_kernargs leaves M = 0: the grid's padded rows are computed (zero A rows -> epilogue of 0)
    spec = t0mi.tile_preset("tile_64x64_k32").copy(transpose=t0mi.NN, epilogue=[t0mi.BIAS_ADD])
    y, ref = dispatch_case(rt, spec, 100, 128, 96, use_m=False)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("preset", ["tile_persistent_decode", "tile_persistent_128x64_k32",
                                    "tile_persistent_256x128_k32"])
def test_dispatch_persistent(rt, preset):
    spec = t0mi.tile_preset(preset).copy(epilogue=[t0mi.RELU])
    y, ref = dispatch_case(rt, spec, 130, 192, 128, persistent_counter=True)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("m", [1, 16])
def test_persistent_decode_shape(rt, m):
    """tile_persistent_decode at the decode shape it exists for (tile_ir.rs:540-561: M = 1,
    N >= 4096): one dispatch of the cost model's configuration (split-K here), integer
    pattern -> exact, bias + scale + clamp epilogue applied once after the reduction."""
    spec = t0mi.tile_preset("tile_persistent_decode").copy(epilogue=[t0mi.BIAS_ADD, t0mi.SCALE, t0mi.CLAMP])
    print(f"[tile] persistent decode m={m} n=4096 k=4096", flush=True)
    y, ref = dispatch_case(rt, spec, m, 4096, 4096, persistent_counter=True)
    assert np.array_equal(y, ref)


def test_dispatch_split_k_reduced_and_planes(rt):
    m, n, k = 128, 128, 512
    spec = t0mi.tile_preset("tile_64x64_k32").copy(split_k=4, epilogue=[t0mi.NEG])
    y, ref = dispatch_case(rt, spec, m, n, k)   # y_split_stride 0: library reduces, epilogue applied
    assert np.array_equal(y, ref)
    # caller-provided partial planes (y_split_stride = M*N*4): raw partial sums, no epilogue
    a, b = int_pattern(m, k, n, False)
    da, pa = to_dev(a)
    db, pb = to_dev(b)
    dy, py = empty_dev(4 * m * n * 4, fill=0xAB)
    plain = spec.copy(epilogue=[])
    kern = rt.tile_kernel(plain)
    ka = bytearray(t0mi.tile_build_kernargs_m(pa, pb, py, k, n, m, plain))
    ka[36:40] = (m * n * 4).to_bytes(4, "little")
    assert rt.dispatch(kern, t0mi.tile_compute_grid(plain, m, n), bytes(ka)) == 0, t0mi.last_error()
    planes = from_dev(dy, np.float32, (4, m, n))
    for p in range(4):
        ks = slice(p * k // 4, (p + 1) * k // 4)
        assert np.array_equal(planes[p], oracle.gemm_bf16(np.ascontiguousarray(a[:, ks]),
                                                          np.ascontiguousarray(b[:, ks]), "nt"))


def test_auto_selected_spec_runs(rt):
    m, n, k = 512, 512, 512
    spec = t0mi.tile_auto_select(m, k, n, t0mi.NN)
    a, b = int_pattern(m, k, n, True)
    y = run_tile(rt, spec, a, b, m, n, k)
    assert np.array_equal(y, oracle.gemm_bf16(a, b, "nn"))


def test_rejects_tile_without_kernel(rt):
    with pytest.raises(t0mi.T0miError) as e:
        rt.tile_gemm(t0mi.tile_preset("tile_128x128_k48").copy(tile_m=512), 0, 0, 0, 128, 128, 128)
    assert e.value.code == -2


def _gold(name, dtype, shape):
    import os
    return np.fromfile(os.path.join(os.path.dirname(__file__), "golden", "torch_ref", name), dtype).reshape(shape)


@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_torch_bf16_chain_down_projection(rt, out):
    # precision_vs_torch.rs:115-116, 296-316: the down projection of the reference's bf16
    # chain, swiglu_bf16_trunc [64, 512] . W_down[256, 512]^T on tile_64x64_k16 (the
    # preset it picks for M < 128), against torch's bf16 GEMM (fixture y_bf16chain).
    # f32 out: the reference's own bar (max|err| < 0.1), and RNE of our sum equals torch's
    # bf16 value except at rounding boundaries; both: torch's and our fp32 sums differ only
    # in summation order, by at most K * 2^-24 * sum|a*b| per output, and each bf16 output
    # is within half a bf16 ulp of its sum.
    m, k, n = 64, 512, 256
    s = _gold("swiglu_bf16_trunc.bin", np.uint16, (m, k))
    wd = _gold("w_down.bin", np.uint16, (n, k))
    yb = _gold("y_bf16chain.bin", np.float32, (m, n))
    dt = t0mi.OUT_BF16 if out == "bf16" else t0mi.OUT_F32
    spec = t0mi.tile_preset("tile_64x64_k16").copy(transpose=t0mi.NT, out_dtype=dt)
    y = run_tile(rt, spec, s, wd, m, n, k)
    if out == "f32":
        assert np.abs(y - yb).max() < 0.1
        mine = oracle.bf16_to_f32(oracle.bf16_rne(y))
    else:
        mine = oracle.bf16_to_f32(y)
    assert (mine == yb).mean() > 0.995
    sab = np.abs(oracle.bf16_to_f32(s)).astype(np.float64) @ np.abs(oracle.bf16_to_f32(wd)).astype(np.float64).T
    ulp = np.abs(yb).astype(np.float64) * 2.0 ** -7
    assert (np.abs(mine.astype(np.float64) - yb) <= k * 2.0 ** -24 * sab + ulp).all()
