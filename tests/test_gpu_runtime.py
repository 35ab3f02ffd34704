"""GPU tests of the runtime's memory calls (GpuRuntime::alloc / alloc_zero / write /
read, src/ignis/gpu_context.rs:508-545) and of the byte-fill kernel that t0mi_memset,
t0mi_alloc_zero and the K = 0 GEMM use (a kernel rather than a memset node, so the calls
can be recorded into graphs).  Bars: byte-exact."""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import runtime

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def test_alloc_copy_round_trip(rt):
    data = np.random.default_rng(1).integers(0, 256, 100003, dtype=np.uint8)
    p = rt.alloc(data.nbytes)
    rt.h2d(p, data)
    back = np.empty_like(data)
    rt.d2h(p, back)
    assert np.array_equal(back, data)
    rt.free(p)
    with pytest.raises(t0mi.T0miError) as e:
        rt.free(p)
    assert e.value.code == t0mi.ERR_INVALID


@pytest.mark.parametrize("nbytes", [1, 17, (1 << 20) + 5])
def test_alloc_zero(rt, nbytes):
    p = rt.alloc(nbytes)
    rt.h2d(p, np.full(nbytes, 0xA5, np.uint8))
    rt.free(p)
    q = rt.alloc(nbytes, zero=True)  # may reuse the same memory: it must come back zeroed
    back = np.empty(nbytes, np.uint8)
    rt.d2h(q, back)
    assert not back.any()
    rt.free(q)


def test_pool_recycle_reuses_zeroed(rt):
    # BufferPool (gpu_context.rs:31-90): recycle keeps the buffer under its 4096-aligned
    # size, the next alloc of that size hands the same buffer out again, zeroed first.
    rt.pool_clear()
    p = rt.alloc(10000)
    rt.h2d(p, np.full(10000, 0xA5, np.uint8))
    rt.recycle(p)
    assert rt.pool_cached_bytes() == 12288
    with pytest.raises(t0mi.T0miError):
        rt.recycle(p)  # no longer a live allocation
    q = rt.alloc(12000)  # same aligned size: the pooled buffer
    assert q == p and rt.pool_cached_bytes() == 0
    back = np.empty(12288, np.uint8)
    rt.d2h(q, back)
    assert not back.any()
    r = rt.alloc(5000)  # another size: a fresh allocation
    assert r != q
    rt.recycle(q)
    rt.recycle(r)
    assert rt.pool_cached_bytes() == 12288 + 8192
    rt.pool_clear()
    assert rt.pool_cached_bytes() == 0


@pytest.mark.parametrize("n", [1, 128, 129, 1000, 4096])
def test_alloc_f32_zeroed_padded(rt, n):
    # alloc_f32 (gpu_context.rs:520-525): max(4n, 512) bytes rounded up to 512, zeroed,
    # also when the pool hands back a dirty buffer of that size.
    nbytes = (max(4 * n, 512) + 511) // 512 * 512
    p = rt.alloc(nbytes)
    rt.h2d(p, np.full(nbytes, 0x7F, np.uint8))
    rt.recycle(p)
    q = rt.alloc_f32(n)
    back = np.empty(nbytes // 4, np.float32)
    rt.d2h(q, back)
    assert not back.any()
    rt.recycle(q)
    fresh = rt.alloc_f32(n + 5000)
    back = np.empty(n + 5000, np.float32)
    rt.d2h(fresh, back)
    assert not back.any()
    rt.free(fresh)
    rt.pool_clear()


def test_recycled_buffer_used_by_queued_gemm(rt):
    # recycle does not wait: a GEMM queued on the stream that writes the buffer still runs
    # before the buffer's next hand-out, whose zero fill comes after it in stream order.
    m = n = k = 256
    a = oracle.normal_bf16((m, k), 11, 0.0, 1.0)
    b = oracle.normal_bf16((n, k), 12, 0.0, 1.0)
    pa, pb = rt.alloc(a.nbytes), rt.alloc(b.nbytes)
    rt.h2d(pa, a.view(np.uint16))
    rt.h2d(pb, b.view(np.uint16))
    py = rt.alloc_f32(m * n)
    cfg = t0mi.auto_select_layout(m, k, n, t0mi.NT, t0mi.OUT_F32)
    rt.gemm(cfg, pa, pb, py, m, n, k)
    rt.recycle(py)
    again = rt.alloc_f32(m * n)
    assert again == py
    back = np.empty(m * n, np.float32)
    rt.d2h(again, back)
    assert not back.any()
    for p in (pa, pb, again):
        rt.free(p)
    rt.pool_clear()


@pytest.mark.parametrize("offset", [0, 1, 7, 15, 16, 17])
@pytest.mark.parametrize("size", [0, 1, 15, 16, 17, 1000, 4096 + 7, (1 << 20) + 3])
def test_memset_any_offset_and_size(rt, offset, size):
    total = offset + size + 40
    p = rt.alloc(total)
    rt.h2d(p, np.full(total, 0xAA, np.uint8))
    t0mi.check(t0mi.lib().t0mi_memset(rt.handle, p + offset, 0x5C, size))
    assert rt.wait_idle() == t0mi.OK
    back = np.empty(total, np.uint8)
    rt.d2h(p, back)
    want = np.full(total, 0xAA, np.uint8)
    want[offset:offset + size] = 0x5C
    assert np.array_equal(back, want)
    rt.free(p)


@pytest.mark.parametrize("out_bf16", [False, True])
def test_gemm_empty_contraction(rt, out_bf16):
    """K = 0: Y = epilogue(0), here bias + relu, through the cleared workspace."""
    m, n = 70, 136
    cfg = t0mi.preset("gfx950_128x128_k64_w2x2").copy(
        epilogue=t0mi.EPI_BIAS_ADD_RELU, out_dtype=t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    bias = np.linspace(-2.0, 2.0, n).astype(np.float32)
    pb = rt.alloc(bias.nbytes)
    rt.h2d(pb, bias)
    ob = 2 if out_bf16 else 4
    py = rt.alloc(m * n * ob)
    rt.h2d(py, np.full(m * n * ob, 0xEE, np.uint8))
    pa = rt.alloc(16)
    rt.gemm(cfg, pa, pa, py, m, n, 0, bias=pb)
    want = np.broadcast_to(np.maximum(bias, 0.0), (m, n))
    if out_bf16:
        got = np.empty((m, n), np.uint16)
        rt.d2h(py, got)
        assert np.array_equal(got, oracle.bf16_rne(np.ascontiguousarray(want)))
    else:
        got = np.empty((m, n), np.float32)
        rt.d2h(py, got)
        assert np.array_equal(got, want)
    for q in (pb, py, pa):
        rt.free(q)


def test_shared_runtime_from_threads():
    """A runtime shared by threads (the reference shares Arc<GpuRuntime>): split-K GEMMs of
    growing workspace needs and W4A16 decodes, launched concurrently from four threads,
    give results bit-identical to a single-threaded run (the workspace is replaced only
    under the runtime's lock, after its stream has drained)."""
    import threading
    from gpu_helpers import empty_dev, from_dev, to_dev, torch

    rt = t0mi.Runtime(device=0)
    g = np.random.default_rng(5)
    jobs = []
    for i, (m, n, k, sk) in enumerate([(96, 256, 1024, 4), (200, 512, 2048, 8), (64, 1024, 4096, 16), (130, 136, 512, 2)]):
        a = (g.standard_normal((m, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        b = (g.standard_normal((k, n)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        cfg = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=t0mi.NN, split_k=sk)
        da, pa = to_dev(a)
        db, pb = to_dev(b)
        dy, py = empty_dev(m * n * 4, fill=0)
        jobs.append(("gemm", (cfg, pa, pb, py, m, n, k), dy, (m, n), [da, db]))
    K, N = 4096, 1024
    aw = (g.standard_normal((16, K)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    w = g.integers(0, 2**32, (K // 8, N), dtype=np.uint32)
    s = np.full((K // 128, N), 0x3C24, np.uint16)
    daw, paw = to_dev(aw)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    dyw, pyw = empty_dev(16 * N * 4, fill=0)
    jobs.append(("w4", (paw, pw, ps, 0, 8, pyw, 16, K, N, 128, t0mi.OUT_F32), dyw, (16, N), [daw, dw, ds]))
    torch().cuda.synchronize()

    def run(job):
        kind, args = job[0], job[1]
        if kind == "gemm":
            rt.gemm(*args)
        else:
            rt.w4a16_gemm(*args)

    for job in jobs:  # single-threaded reference
        run(job)
    assert rt.wait_idle() == t0mi.OK
    ref = [from_dev(j[2], np.float32, j[3]) for j in jobs]
    for j in jobs:
        j[2][:j[2].t0mi_guard].zero_()  # keep the guard bytes
    torch().cuda.synchronize()
    rt.close()
    rt = t0mi.Runtime(device=0)  # fresh runtime: the workspace grows while the threads run
    errors = []

    def worker(order):
        try:
            for _ in range(5):
                for idx in order:
                    run(jobs[idx])
        except Exception as e:  # reported below
            errors.append(repr(e))

    orders = [[0, 1, 2, 3, 4], [3, 2, 1, 0, 4], [2, 4, 0, 3, 1], [4, 1, 3, 2, 0]]
    threads = [threading.Thread(target=worker, args=(o,)) for o in orders]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert rt.wait_idle() == t0mi.OK
    for j, r in zip(jobs, ref):
        assert np.array_equal(from_dev(j[2], np.float32, j[3]), r), j[0]
    rt.close()
