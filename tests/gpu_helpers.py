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


def empty_dev(nbytes: int, fill: int = None):
    t = torch()
    d = t.empty(max(nbytes, 16), dtype=t.uint8, device="cuda:0")
    if fill is not None:
        d.fill_(fill)
    return d, d.data_ptr()


def from_dev(d, dtype, shape):
    t = torch()
    t.cuda.synchronize()
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return d[:n].cpu().numpy().view(dtype).reshape(shape).copy()


def runtime():
    """A t0mi runtime launching on torch's current stream of cuda:0."""
    import t0mi
    t = torch()
    t.cuda.init()
    return t0mi.Runtime.on_torch_stream(0)
