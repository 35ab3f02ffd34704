"""GPU tests of batched submission through the C ABI: the DispatchQueue of
src/t0/prefill_dispatch.rs:58-214 and its HIP-graph form.

Bars: a queued batch and a graph replay run the same kernels on the same
inputs as the eager calls, so every output is bit-identical to the eager one.
Each graph is replayed several times with eager work, output resets and
synchronisations between the replays, and every replay is checked.  Calls
that cannot be recorded are refused during capture without spoiling it.
"""
import numpy as np
import pytest

import t0mi
from gpu_helpers import check_guard, empty_dev, to_dev, torch

pytestmark = pytest.mark.gpu


@pytest.fixture()
def rt():
    """A runtime on its own (non-null, default-priority) stream: the null stream cannot be captured."""
    torch().cuda.init()
    r = t0mi.Runtime(device=0)
    yield r
    r.close()


def rand_bf16(shape, seed):
    g = np.random.default_rng(seed)
    x = g.standard_normal(shape).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 pattern serves


def read(d, dtype, shape):
    torch().cuda.synchronize()
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return d[:n].cpu().numpy().view(dtype).reshape(shape).copy()


def check_replay(got, ref, reset_byte, where):
    for name in ref:
        if name == "fill":  # bytes 1..1000 are written, the two ends keep the reset value
            f = got[name]
            assert np.array_equal(f[1:1001], ref[name][1:1001]), where
            assert f[0] == reset_byte and np.all(f[1001:] == reset_byte), where
        else:
            assert np.array_equal(got[name], ref[name]), (where, name)


class Batch:
    """A mixed batch of library calls; outputs are kept as torch byte tensors."""

    def __init__(self, rt):
        self.rt = rt
        self.keep = []
        self.outs = {}
        # 1. raw gemm_gen dispatch (NT, f32 out, tile-aligned: the kernarg carries no M)
        self.cfg_raw = t0mi.preset("tile_64x64_k32")
        m, n, k = 128, 128, 256
        self.raw = self.dev(rand_bf16((m, k), 1)), self.dev(rand_bf16((n, k), 2))
        self.out("raw", m * n * 4)
        self.k_raw = rt.kernel(self.cfg_raw)
        self.ka_raw = t0mi.build_kernargs(self.raw[0], self.raw[1], self.outs["raw"][1], k, n, m, self.cfg_raw)
        self.grid_raw = t0mi.compute_grid_auto(self.cfg_raw, m, n)
        # 2. split-K GEMM through the workspace, NN, bf16 out, ragged M
        self.cfg_sk = t0mi.preset("gfx950_128x128_k64_w2x2").copy(transpose=t0mi.NN, split_k=4,
                                                                  out_dtype=t0mi.OUT_BF16)
        self.sk = self.dev(rand_bf16((200, 1024), 3)), self.dev(rand_bf16((1024, 256), 4))
        self.out("sk", 200 * 256 * 2)
        # 3. tile GEMM with a fused bias + relu epilogue
        self.spec = t0mi.tile_preset("tile_64x64_k32").copy(epilogue=[t0mi.BIAS_ADD, t0mi.RELU])
        self.tile = self.dev(rand_bf16((96, 128), 5)), self.dev(rand_bf16((192, 128), 6))
        self.bias = self.dev(np.random.default_rng(7).standard_normal(192).astype(np.float32))
        self.out("tile", 96 * 192 * 4)
        # 4. W4A16 decode, g128, zero point constant
        g = np.random.default_rng(8)
        self.w4 = (self.dev(rand_bf16((16, 4096), 9)),
                   self.dev(g.integers(0, 2**32, (512, 1024), dtype=np.uint32)),
                   self.dev(np.full((32, 1024), 0x3C24, np.uint16)))
        self.out("w4", 16 * 1024 * 2)
        # 5. byte fill (a kernel, not a memset node)
        self.out("fill", 1000 + 3)
        # 6. Ignis matmul: GPU f32 -> bf16 conversion into the library buffer, then the GEMM
        self.mm = self.dev(g.standard_normal((37, 100)).astype(np.float32)), \
            self.dev(g.standard_normal((100, 72)).astype(np.float32))
        self.out("mm", 37 * 72 * 4)
        torch().cuda.synchronize()

    def dev(self, arr):
        d, p = to_dev(arr)
        self.keep.append(d)
        return p

    def out(self, name, nbytes):
        self.outs[name] = empty_dev(nbytes)

    def reset(self, byte):
        for d, _ in self.outs.values():
            d[:d.t0mi_guard].fill_(byte)  # the guard bytes past each buffer keep their pattern
        torch().cuda.synchronize()

    def run(self):
        rt, o = self.rt, {k: v[1] for k, v in self.outs.items()}
        assert rt.dispatch(self.k_raw, self.grid_raw, self.ka_raw, sync=False) == t0mi.OK, t0mi.last_error()
        rt.gemm(self.cfg_sk, self.sk[0], self.sk[1], o["sk"], 200, 256, 1024)
        rt.tile_gemm(self.spec, self.tile[0], self.tile[1], o["tile"], 96, 192, 128, bias=self.bias)
        rt.w4a16_gemm(self.w4[0], self.w4[1], self.w4[2], 0, 8, o["w4"], 16, 4096, 1024, 128, t0mi.OUT_BF16)
        t0mi.check(t0mi.lib().t0mi_memset(rt.handle, o["fill"] + 1, 0x5A, 1000))
        rt.matmul(self.mm[0], self.mm[1], o["mm"], 37, 100, 72)

    def results(self):
        torch().cuda.synchronize()
        for d, _ in self.outs.values():
            check_guard(d)
        return {k: d[:d.t0mi_guard].cpu().numpy().copy() for k, (d, _) in self.outs.items()}


def test_graph_replays_match_eager(rt):
    b = Batch(rt)
    b.reset(0xEE)
    b.run()
    assert rt.wait_idle() == t0mi.OK
    ref = b.results()
    fill = ref["fill"]
    assert fill[0] == 0xEE and np.all(fill[1:1001] == 0x5A) and np.all(fill[1001:] == 0xEE)
    for name in ("raw", "sk", "tile", "w4", "mm"):
        assert not np.all(ref[name] == 0xEE), f"{name} was not written"

    b.reset(0x00)
    rt.capture_begin()
    b.run()
    g = rt.capture_end()
    assert rt.wait_idle() == t0mi.OK
    assert g.node_count >= 6
    assert all(np.all(v == 0) for v in b.results().values()), "capture must record, not run"

    # Eager work between replays: the same batch's split-K GEMM into another buffer.
    side, pside = empty_dev(200 * 256 * 2)
    for r in range(3):
        b.reset(0x11 * (r + 1))
        rt.gemm(b.cfg_sk, b.sk[0], b.sk[1], pside, 200, 256, 1024)
        assert rt.wait_idle() == t0mi.OK
        g.launch()
        assert rt.wait_idle() == t0mi.OK
        check_replay(b.results(), ref, 0x11 * (r + 1), r)
        assert np.array_equal(read(side, np.uint8, (200 * 256 * 2,)), ref["sk"]), r
    g.destroy()


def test_dispatch_queue_matches_synchronous(rt):
    cfg = t0mi.preset("tile_64x64_k32")
    k = rt.kernel(cfg)
    m = n = 128
    kk = 256
    jobs = []
    keep = []
    for i in range(6):
        da, pa = to_dev(rand_bf16((m, kk), 20 + i))
        db, pb = to_dev(rand_bf16((n, kk), 40 + i))
        y1, p1 = empty_dev(m * n * 4, fill=0xAB)
        y2, p2 = empty_dev(m * n * 4, fill=0xCD)
        y3, p3 = empty_dev(m * n * 4, fill=0xEF)
        keep += [da, db]
        jobs.append((pa, pb, (y1, p1), (y2, p2), (y3, p3)))
    torch().cuda.synchronize()
    grid = t0mi.compute_grid_auto(cfg, m, n)
    for pa, pb, (y1, p1), _, _ in jobs:
        assert rt.dispatch(k, grid, t0mi.build_kernargs(pa, pb, p1, kk, n, m, cfg)) == t0mi.OK
    dq = t0mi.DispatchQueue(rt)
    for pa, pb, _, (y2, p2), _ in jobs:
        dq.submit(k, grid, t0mi.build_kernargs(pa, pb, p2, kk, n, m, cfg))
    assert dq.pending() == 6
    assert dq.flush() == 6
    assert t0mi.batch_dispatch(rt, [(k, grid, t0mi.build_kernargs(pa, pb, p3, kk, n, m, cfg))
                                    for pa, pb, _, _, (y3, p3) in jobs]) == 6
    for _, _, (y1, _), (y2, _), (y3, _) in jobs:
        ref = read(y1, np.float32, (m, n))
        assert np.array_equal(read(y2, np.float32, (m, n)), ref)
        assert np.array_equal(read(y3, np.float32, (m, n)), ref)


def test_capture_refuses_unrecordable_calls(rt):
    b = Batch(rt)
    b.reset(0xEE)
    b.run()  # sizes the workspace and conversion buffer
    assert rt.wait_idle() == t0mi.OK
    ref = b.results()
    b.reset(0)
    wide, pwide = empty_dev(200 * 4096 * 2)  # output of the call that would need a larger workspace
    torch().cuda.synchronize()
    rt.capture_begin()
    assert rt.dispatch(b.k_raw, b.grid_raw, b.ka_raw, sync=True) == t0mi.ERR_CAPTURE
    assert rt.wait_idle() == t0mi.ERR_CAPTURE
    for call in (lambda: rt.alloc(64), lambda: rt.d2h(b.outs["raw"][1], np.empty(4, np.uint8)),
                 lambda: rt.h2d(b.outs["raw"][1], np.zeros(4, np.uint8)),
                 # workspace growth: 16x the split-K planes of the batch (B [64][4096] fits in sk[1])
                 lambda: rt.gemm(b.cfg_sk, b.sk[0], b.sk[1], pwide, 200, 4096, 64)):
        with pytest.raises(t0mi.T0miError) as e:
            call()
        assert e.value.code == t0mi.ERR_CAPTURE
    b.run()
    g = rt.capture_end()
    assert not rt.is_poisoned()
    for r in range(2):
        b.reset(0x33)
        g.launch()
        assert rt.wait_idle() == t0mi.OK
        check_replay(b.results(), ref, 0x33, r)
    # A live graph pins the workspace: growth is refused until it is destroyed.
    big, pbig = empty_dev(200 * 2048 * 2)
    da, pa = to_dev(rand_bf16((200, 8192), 11))
    db, pb = to_dev(rand_bf16((8192, 2048), 12))
    torch().cuda.synchronize()
    with pytest.raises(t0mi.T0miError) as e:
        rt.gemm(b.cfg_sk, pa, pb, pbig, 200, 2048, 8192)
    assert e.value.code == t0mi.ERR_CAPTURE
    g.destroy()
    rt.gemm(b.cfg_sk, pa, pb, pbig, 200, 2048, 8192)
    assert rt.wait_idle() == t0mi.OK
