"""GPU tests of t0mi_gemm_noalloc: t0mi_gemm with its split-K planes in the
library's static per-GPU scratch array instead of the runtime's growable
workspace (no reference counterpart; for callers that cannot allocate).

Bar: bit-identical to t0mi_gemm on the same inputs and config (same kernels,
same partition order in the reduce), on two no-allocation calls in a row, the
second smaller than the first, so the second runs over what the first left in
the scratch.  A request larger than the scratch is refused before anything is
launched.  Every output buffer carries guard bytes that must stay untouched.
"""
import numpy as np
import pytest

import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev, torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def rand_bf16(shape, seed):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def operands(m, n, k, seed, nn=True):
    a = rand_bf16((m, k), seed)
    b = rand_bf16((k, n) if nn else (n, k), seed + 1)
    return a, b


def call(rt, fn, cfg, pa, pb, m, n, k, pbias=0):
    ob = 2 if cfg.out_dtype == t0mi.OUT_BF16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xAB)
    fn(cfg, pa, pb, py, m, n, k, bias=pbias)
    return dy


def result(dy, cfg, m, n):
    return from_dev(dy, np.uint16 if cfg.out_dtype == t0mi.OUT_BF16 else np.float32, (m, n))


SPLITK_BF16 = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=t0mi.NN, split_k=4, out_dtype=t0mi.OUT_BF16)


def test_two_calls_in_a_row_match_gemm(rt):
    """Call 1 (128x4096x4096, split-K 4: 8 MiB of planes), then call 2
    (64x1024x2048: 1 MiB) straight after it on the same stream; both equal
    t0mi_gemm bit for bit."""
    shapes = [(128, 4096, 4096, 10), (64, 1024, 2048, 20)]
    keep, outs = [], []
    for m, n, k, seed in shapes:
        a, b = operands(m, n, k, seed)
        (da, pa), (db, pb) = to_dev(a), to_dev(b)
        keep += [da, db, a, b]
        outs.append((m, n, k, pa, pb, a, b))
    print(f"[no_alloc] split-K 4 NN bf16: {shapes[0][:3]} then {shapes[1][:3]}", flush=True)
    got = [call(rt, rt.gemm_noalloc, SPLITK_BF16, pa, pb, m, n, k) for (m, n, k, pa, pb, _, _) in outs]
    torch().cuda.synchronize()
    for (m, n, k, pa, pb, a, b), dy in zip(outs, got):
        y_na = result(dy, SPLITK_BF16, m, n)
        y_ref = result(call(rt, rt.gemm, SPLITK_BF16, pa, pb, m, n, k), SPLITK_BF16, m, n)
        assert np.array_equal(y_na, y_ref), f"{m}x{n}x{k}: differs from t0mi_gemm"
        # and it is the product (loose fp32 check; parity of t0mi_gemm itself is tested elsewhere)
        ref = bf16_to_f32(a) @ bf16_to_f32(b)
        err = np.abs(bf16_to_f32(y_na) - ref).max()
        assert err <= 1e-2 * np.sqrt(k) * np.abs(ref).max() / 8, (m, n, k, err)


def test_bias_relu_f32_split8_then_smaller(rt):
    """f32 output with the bias + relu epilogue at split-K 8, ragged shapes,
    then a smaller split-K 2 call: equal to t0mi_gemm."""
    cfg8 = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=t0mi.NN, split_k=8,
                                                      epilogue=t0mi.EPI_BIAS_ADD_RELU)
    cfg2 = cfg8.copy(split_k=2)
    runs = []
    for cfg, (m, n, k, seed) in ((cfg8, (200, 520, 1032, 30)), (cfg2, (17, 136, 256, 40))):
        a, b = operands(m, n, k, seed)
        bias = np.random.default_rng(seed + 2).standard_normal(n).astype(np.float32)
        (da, pa), (db, pb), (dbias, pbias) = to_dev(a), to_dev(b), to_dev(bias)
        runs.append((cfg, m, n, k, pa, pb, pbias, [da, db, dbias]))
    print("[no_alloc] bias+relu f32: split-K 8 200x520x1032, then split-K 2 17x136x256", flush=True)
    got = [call(rt, rt.gemm_noalloc, cfg, pa, pb, m, n, k, pbias) for (cfg, m, n, k, pa, pb, pbias, _) in runs]
    for (cfg, m, n, k, pa, pb, pbias, _), dy in zip(runs, got):
        y_ref = result(call(rt, rt.gemm, cfg, pa, pb, m, n, k, pbias), cfg, m, n)
        assert np.array_equal(result(dy, cfg, m, n), y_ref), f"{m}x{n}x{k}"


def test_no_split_and_empty_k(rt):
    """split_k = 1 uses no scratch; K = 0 writes epilogue(0) through one zero
    plane in the scratch, after a call that left other data there."""
    cfg = t0mi.preset("gfx950_256x256_k64_w2x4").copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16)
    m, n, k = 300, 512, 512
    a, b = operands(m, n, k, 50)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    print("[no_alloc] split_k 1 300x512x512, then K=0 64x256", flush=True)
    dy = call(rt, rt.gemm_noalloc, cfg, pa, pb, m, n, k)
    y_ref = result(call(rt, rt.gemm, cfg, pa, pb, m, n, k), cfg, m, n)
    assert np.array_equal(result(dy, cfg, m, n), y_ref)
    # K = 0 right after a split-K call that filled the scratch with partial sums
    big = SPLITK_BF16
    a2, b2 = operands(128, 1024, 1024, 60)
    (da2, pa2), (db2, pb2) = to_dev(a2), to_dev(b2)
    call(rt, rt.gemm_noalloc, big, pa2, pb2, 128, 1024, 1024)
    f32 = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=t0mi.NN)
    dz = call(rt, rt.gemm_noalloc, f32, pa, pb, 64, 256, 0)
    assert np.all(result(dz, f32, 64, 256) == 0)


def test_too_large_is_refused_before_launch(rt):
    """4096 x 4096 at split-K 4 needs 256 MiB of planes: refused with
    T0MI_ERR_INVALID, Y untouched; t0mi_gemm still runs it (growable workspace)."""
    assert t0mi.NOALLOC_SCRATCH_BYTES == 32 << 20
    m, n, k = 4096, 4096, 256
    a, b = operands(m, n, k, 70)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    dy, py = empty_dev(m * n * 2, fill=0xAB)
    print("[no_alloc] 4096x4096 split-K 4: expect refusal", flush=True)
    with pytest.raises(t0mi.T0miError) as e:
        rt.gemm_noalloc(SPLITK_BF16, pa, pb, py, m, n, k)
    assert e.value.code == t0mi.ERR_INVALID and "scratch" in str(e.value)
    torch().cuda.synchronize()
    assert np.all(from_dev(dy, np.uint8, (m * n * 2,)) == 0xAB)
    # the largest that fits: 512 x 4096 x 4 planes = exactly 32 MiB
    m = 512
    a, b = operands(m, n, k, 80)
    (da, pa), (db, pb) = to_dev(a), to_dev(b)
    dy = call(rt, rt.gemm_noalloc, SPLITK_BF16, pa, pb, m, n, k)
    y_ref = result(call(rt, rt.gemm, SPLITK_BF16, pa, pb, m, n, k), SPLITK_BF16, m, n)
    assert np.array_equal(result(dy, SPLITK_BF16, m, n), y_ref)


def test_overlapping_call_from_another_stream_is_refused():
    """The scratch is shared by every runtime on the GPU: a call from a second stream while
    the first stream's call is still queued or running is refused (T0MI_ERR_INVALID); once
    that stream has drained, the second stream's call runs and matches t0mi_gemm."""
    r1, r2 = t0mi.Runtime(device=0), t0mi.Runtime(device=0)  # two runtimes, each its own stream
    try:
        m, n, k = 128, 4096, 4096
        a, b = operands(m, n, k, 40)
        (da, pa), (db, pb) = to_dev(a), to_dev(b)
        big_a, big_b = operands(4096, 4096, 4096, 41)
        (dba, pba), (dbb, pbb) = to_dev(big_a), to_dev(big_b)
        dbig, pbig = empty_dev(4096 * 4096 * 2)
        big = t0mi.auto_select_layout(4096, 4096, 4096, t0mi.NN, t0mi.OUT_BF16)
        torch().cuda.synchronize()
        # ~1 ms of work queued on r1's stream ahead of its no-allocation call
        for _ in range(10):
            r1.gemm(big, pba, pbb, pbig, 4096, 4096, 4096)
        d1 = call(r1, r1.gemm_noalloc, SPLITK_BF16, pa, pb, m, n, k)
        with pytest.raises(t0mi.T0miError) as e:
            call(r2, r2.gemm_noalloc, SPLITK_BF16, pa, pb, m, n, k)
        assert e.value.code == t0mi.ERR_INVALID and "another stream" in str(e.value)
        assert r1.wait_idle() == t0mi.OK
        d2 = call(r2, r2.gemm_noalloc, SPLITK_BF16, pa, pb, m, n, k)
        assert r2.wait_idle() == t0mi.OK
        y1, y2 = result(d1, SPLITK_BF16, m, n), result(d2, SPLITK_BF16, m, n)
        y_ref = result(call(r2, r2.gemm, SPLITK_BF16, pa, pb, m, n, k), SPLITK_BF16, m, n)
        assert r2.wait_idle() == t0mi.OK
        assert np.array_equal(y1, y_ref) and np.array_equal(y2, y_ref)
    finally:
        r1.close()
        r2.close()
