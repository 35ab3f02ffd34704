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
