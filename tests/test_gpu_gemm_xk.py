"""GPU tests of the split-K GEMM whose partials are combined inside the launch, through the
output tile's XCD's L2 (gemm_bf16_xk_kernel: the split_k pieces of a tile store their fp32
partials, wait for each other, and each sums one row slice of the tile).

Bars: bit-identical to the plane route (t0mi_gemm_noalloc always writes split-K planes and
sums them in a second launch: same per-piece sums, same order of the final adds, same
epilogue and rounding); the full BASELINE config 3 against the oracle within
max|err| <= 1e-2 * sqrt(K) * max|a| * max|b|; identical results over repeated calls and
HIP-graph replays (the counters reset themselves); no workgroup on another XCD than planned
and no piece left waiting.
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev, torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def run(rt, fn, cfg, a, b, m, n, k, bias=None):
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    ob = 2 if cfg.out_dtype == t0mi.OUT_BF16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    pbias = 0
    if bias is not None:
        dbias, pbias = to_dev(bias.astype(np.float32))
    print(f"[gemm xk] {cfg.name()} {m}x{n}x{k} via {fn}", flush=True)
    getattr(rt, fn)(cfg, pa, pb, py, m, n, k, pbias)
    return from_dev(dy, np.uint16 if ob == 2 else np.uint32, (m, n))


CASES = [
    # (m, n, k, config, layout)
    (128, 4096, 4096, "gfx950_128x128_k64_w2x2_s3", t0mi.NN, 8),    # BASELINE config 3's pick
    (128, 4096, 4096, "gfx950_128x128_k64_w2x2_s3", t0mi.NT, 8),
    (16, 4096, 4096, "gfx950_128x128_k64_w2x2_s3", t0mi.NN, 8),     # decode-sized rows
    (100, 1032, 4096, "gfx950_128x128_k64_w2x2_s3", t0mi.NN, 4),    # ragged M and N (partial tiles)
    (128, 2048, 3000, "gfx950_128x128_k64_w2x2_s3", t0mi.NT, 16),   # K not a tile multiple, 16 pieces
    (256, 4096, 4096, "gfx950_128x128_k64_w2x2_s3", t0mi.NN, 2),
    (32, 11008, 4096, "gfx950_64x128_k64_w2x2", t0mi.NN, 8),
    (128, 11008, 4096, "gfx950_128x256_k64_w2x2", t0mi.NT, 4),
]


@pytest.mark.parametrize("m,n,k,preset,tr,sk", CASES)
@pytest.mark.parametrize("out", [t0mi.OUT_BF16, t0mi.OUT_F32])
def test_bit_identical_to_plane_route(rt, m, n, k, preset, tr, sk, out):
    cfg = t0mi.preset(preset).copy(transpose=tr, out_dtype=out, split_k=sk)
    a = oracle.normal_bf16((m, k), 0xA1 + m, 0.0, 1.0)
    b = oracle.normal_bf16((k, n) if tr == t0mi.NN else (n, k), 0xA2 + n, 0.0, 1.0)
    y_xk = run(rt, "gemm", cfg, a, b, m, n, k)
    y_pl = run(rt, "gemm_noalloc", cfg, a, b, m, n, k)
    assert np.array_equal(y_xk, y_pl)
    assert rt.xcd_placement() == (8, False)


def test_config3_full_vs_oracle(rt):
    m, n, k = 128, 4096, 4096
    cfg = t0mi.auto_select_layout(m, k, n, t0mi.NN, t0mi.OUT_F32)
    assert cfg.split_k > 1, cfg.name()
    a = oracle.normal_bf16((m, k), 0x7503, 0.0, 0.02)
    b = oracle.normal_bf16((k, n), 0x7504, 0.0, 0.02)
    y = run(rt, "gemm", cfg, a, b, m, n, k).view(np.float32)
    ref = oracle.gemm_bf16(a, b, "nn")
    err, rel = oracle.compare(y, ref)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    assert err <= tol and rel < 1e-5, (err, tol, rel)


@pytest.mark.parametrize("out", [t0mi.OUT_BF16, t0mi.OUT_F32])
def test_bias_relu_epilogue_bit_identical(rt, out):
    # gemm_gen's BiasAddReluStoreF32 epilogue: applied once, to the summed value, by the
    # piece that stores each slice (the plane route's reduce applies it the same way).
    m, n, k = 128, 2048, 4096
    cfg = t0mi.preset("gfx950_128x128_k64_w2x2_s3").copy(transpose=t0mi.NN, out_dtype=out, split_k=8, epilogue=2)
    a = oracle.normal_bf16((m, k), 0xB5, 0.0, 1.0)
    b = oracle.normal_bf16((k, n), 0xB6, 0.0, 1.0)
    bias = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    y_xk = run(rt, "gemm", cfg, a, b, m, n, k, bias=bias)
    y_pl = run(rt, "gemm_noalloc", cfg, a, b, m, n, k, bias=bias)
    assert np.array_equal(y_xk, y_pl)
    if out == t0mi.OUT_F32:
        ref = np.maximum(oracle.gemm_bf16(a, b, "nn") + bias, 0.0)
        tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
        assert np.abs(y_xk.view(np.float32) - ref).max() <= tol


@pytest.mark.parametrize("ops", [[t0mi.BIAS_ADD, t0mi.SILU], [t0mi.SCALE, t0mi.CLAMP]])
def test_tile_epilogue_split_k(rt, ops):
    # A TileGemm spec with split-K and a fused epilogue chain: the chain runs once, after the
    # K partitions are summed, on the summed value.
    m, n, k = 128, 1024, 4096
    spec = t0mi.tile_preset("tile_128x128_k64").copy(transpose=t0mi.NN, split_k=8, triple_buffer=1, epilogue=ops)
    a = oracle.normal_bf16((m, k), 0xB1, 0.0, 1.0)
    b = oracle.normal_bf16((k, n), 0xB2, 0.0, 1.0)
    bias = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    (da, pa), (db, pb), (dbias, pbias) = to_dev(a), to_dev(b), to_dev(bias)
    dy, py = empty_dev(m * n * 4, fill=0xAB)
    rt.tile_gemm(spec, pa, pb, py, m, n, k, bias=pbias, scale=0.5, clamp_min=-1.0, clamp_max=2.0)
    y = from_dev(dy, np.float32, (m, n))
    ref = oracle.epilogue(oracle.gemm_bf16(a, b, "nn"), ops, bias=bias, scale=0.5, clamp_min=-1.0, clamp_max=2.0)
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    assert np.abs(y - ref).max() <= tol * 1.01 + 1e-5 * np.abs(ref).max()


def test_graph_replays_match_eager():
    t = torch()
    r = t0mi.Runtime(device=0)  # own stream: a graph cannot be captured on the null stream
    try:
        m, n, k = 128, 4096, 4096
        cfg = t0mi.preset("gfx950_128x128_k64_w2x2_s3").copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16, split_k=8)
        a = oracle.normal_bf16((m, k), 0xC1, 0.0, 1.0)
        b = oracle.normal_bf16((k, n), 0xC2, 0.0, 1.0)
        (da, pa), (db, pb) = to_dev(a), to_dev(b)
        ys = [empty_dev(m * n * 2, fill=0) for _ in range(3)]
        t.cuda.synchronize()
        for _, py in ys:  # eager once: the exchange buffers exist before the capture
            r.gemm(cfg, pa, pb, py, m, n, k)
        assert r.wait_idle() == t0mi.OK
        ref = from_dev(ys[0][0], np.uint16, (m, n))
        r.capture_begin()
        for _, py in ys:
            r.gemm(cfg, pa, pb, py, m, n, k)
        g = r.capture_end()
        side, pside = empty_dev(m * n * 2, fill=0)
        for rep in range(4):
            for dy, _ in ys:
                dy[: m * n * 2].fill_(0)
            t.cuda.synchronize()
            g.launch()
            assert r.wait_idle() == t0mi.OK
            for dy, _ in ys:
                assert np.array_equal(from_dev(dy, np.uint16, (m, n)), ref), rep
            r.gemm(cfg, pa, pb, pside, m, n, k)  # eager work on the same counters between replays
            assert r.wait_idle() == t0mi.OK
            assert np.array_equal(from_dev(side, np.uint16, (m, n)), ref), rep
        g.destroy()
        assert r.xcd_placement() == (8, False)
    finally:
        r.close()
