"""CPU tests of batched submission on the null runtime: the DispatchQueue
contract of src/t0/prefill_dispatch.rs:58-214 (pending count, one flush, poison
refusal, drop without flush, batch_dispatch) and the capture calls' refusal
without a device.  No compute runs here; the GPU tests run the same calls on
real kernels and graphs."""
import pytest

import t0mi


@pytest.fixture()
def rt():
    r = t0mi.Runtime(null=True)
    yield r
    r.close()


def small_dispatch(rt, n=64):
    cfg = t0mi.preset("tile_64x64_k32")
    k = rt.kernel(cfg)
    return k, t0mi.compute_grid_auto(cfg, n, n), t0mi.build_kernargs(0x1000, 0x2000, 0x3000, n, n, n, cfg)


def test_empty_flush(rt):
    """prefill_dispatch.rs:215-220: flushing an empty queue returns 0."""
    dq = t0mi.DispatchQueue(rt)
    assert dq.pending() == 0
    assert dq.flush() == 0


def test_pending_count_and_flush(rt):
    dq = t0mi.DispatchQueue(rt)
    k, grid, ka = small_dispatch(rt)
    k2, grid2, ka2 = small_dispatch(rt, 128)
    dq.submit(k, grid, ka)
    dq.submit(k, grid, ka)
    dq.submit(k2, grid2, ka2)
    assert dq.pending() == 3
    assert rt.last_dispatch() == ((grid2[0], grid2[1], 1), ka2), "submits reach the runtime in order"
    assert dq.flush() == 3
    assert dq.pending() == 0
    assert dq.flush() == 0


def test_submit_checks_like_dispatch(rt):
    """The kernarg-length assert (gpu_context.rs:319-323) holds for queued submits;
    a refused submit is not counted."""
    dq = t0mi.DispatchQueue(rt)
    k, grid, ka = small_dispatch(rt)
    with pytest.raises(t0mi.T0miError) as e:
        dq.submit(k, grid, ka[:36])
    assert e.value.code == t0mi.ERR_KERNARG
    with pytest.raises(t0mi.T0miError) as e:
        dq.submit(k, (grid[0] + 1, grid[1]), ka)
    assert e.value.code == t0mi.ERR_INVALID
    assert dq.pending() == 0


def test_poisoned_queue_refuses_submit(rt):
    """prefill_dispatch.rs:96-99."""
    dq = t0mi.DispatchQueue(rt)
    k, grid, ka = small_dispatch(rt)
    rt.mark_poisoned()
    with pytest.raises(t0mi.T0miError) as e:
        dq.submit(k, grid, ka)
    assert e.value.code == t0mi.ERR_POISONED
    assert "[DispatchQueue] Queue poisoned" in str(e.value)


def test_flush_timeout_poisons(rt):
    """A failed wait at flush poisons the runtime (prefill_dispatch.rs:145-165)."""
    dq = t0mi.DispatchQueue(rt)
    k, grid, ka = small_dispatch(rt)
    dq.submit(k, grid, ka)
    rt.inject_timeout()
    with pytest.raises(t0mi.T0miError) as e:
        dq.flush()
    assert e.value.code == t0mi.ERR_TIMEOUT
    assert rt.is_poisoned()
    assert dq.pending() == 0


def test_drop_async_warns_when_pending(rt, capfd):
    """prefill_dispatch.rs:177-187: dropping with pending dispatches warns."""
    dq = t0mi.DispatchQueue(rt)
    k, grid, ka = small_dispatch(rt)
    dq.submit(k, grid, ka)
    dq.submit(k, grid, ka)
    dq.drop_async()
    assert "2 dispatches dropped without flush()" in capfd.readouterr().err
    quiet = t0mi.DispatchQueue(rt)
    quiet.drop_async()
    assert "dropped" not in capfd.readouterr().err


def test_batch_dispatch(rt):
    """prefill_dispatch.rs:204-214: submit all, flush once, return the count."""
    k, grid, ka = small_dispatch(rt)
    k2, grid2, ka2 = small_dispatch(rt, 192)
    assert t0mi.batch_dispatch(rt, []) == 0
    assert t0mi.batch_dispatch(rt, [(k, grid, ka), (k2, grid2, ka2), (k, grid, ka)]) == 3
    assert rt.last_dispatch() == ((grid[0], grid[1], 1), ka)
    with pytest.raises(t0mi.T0miError) as e:
        t0mi.batch_dispatch(rt, [(k, grid, ka), (k, grid, ka[:8])])
    assert e.value.code == t0mi.ERR_KERNARG


def test_capture_needs_a_device(rt):
    with pytest.raises(t0mi.T0miError) as e:
        rt.capture_begin()
    assert e.value.code == t0mi.ERR_NO_DEVICE
    with pytest.raises(t0mi.T0miError) as e:
        rt.capture_end()
    assert e.value.code == t0mi.ERR_NO_DEVICE
