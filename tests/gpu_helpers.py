"""Device-memory helpers for the GPU parity tests (torch is used only for memory and streams)."""
import numpy as np


def torch():
    import torch as _t
    return _t


def to_dev(arr: np.ndarray):
    """Copy a numpy array to cuda:0 as raw bytes; returns the tensor (keep it alive) and its address."""
    t = torch()
    a = np.ascontiguousarray(arr)
    d = t.from_numpy(a.view(np.uint8).reshape(-1).copy()).to("cuda:0")
    return d, d.data_ptr()


GUARD_BYTES = 4096
GUARD_FILL = 0x5C


class GuardError(AssertionError):
    pass


def empty_dev(nbytes: int, fill: int = None):
    """nbytes of device memory (optionally filled), followed by GUARD_BYTES guard bytes of
    GUARD_FILL: from_dev() fails if a kernel wrote past the end of the buffer."""
    t = torch()
    d = t.empty(nbytes + GUARD_BYTES, dtype=t.uint8, device="cuda:0")
    if fill is not None:
        d[:nbytes].fill_(fill)
    d[nbytes:].fill_(GUARD_FILL)
    d.t0mi_guard = nbytes
    return d, d.data_ptr()


def check_guard(d):
    """Raises GuardError if the guard bytes after an empty_dev() buffer were written."""
    start = getattr(d, "t0mi_guard", None)
    if start is None:
        return
    g = d[start:].cpu().numpy()
    bad = np.nonzero(g != GUARD_FILL)[0]
    if bad.size:
        raise GuardError(f"{bad.size} guard byte(s) written past the {start}-byte buffer "
                         f"(first at +{int(bad[0])})")


def from_dev(d, dtype, shape):
    """The first prod(shape) elements of a device buffer; checks its guard bytes too."""
    t = torch()
    t.cuda.synchronize()
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    check_guard(d)
    return d[:n].cpu().numpy().view(dtype).reshape(shape).copy()


def runtime():
    """A t0mi runtime launching on torch's current stream of cuda:0."""
    import t0mi
    t = torch()
    t.cuda.init()
    return t0mi.Runtime.on_torch_stream(0)
