"""ctypes binding of libt0mi_probes.so: the measurement kernels behind the floors the
GEMM and W4A16 kernels are judged against (streaming read with 16-byte normal or
non-temporal loads, empty launch, MFMA loops of a GEMM wave tile with shader-clock
stamps).  Used by
bench.py --only stream / mfma; not part of the product ABI."""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
PROBES_PATH = os.path.join(_HERE, "libt0mi_probes.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(PROBES_PATH):
            raise ImportError(f"libt0mi_probes.so not built at {PROBES_PATH}; run __graft_entry__.build()")
        L = ctypes.CDLL(PROBES_PATH)
        P, U32, SZ, I = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_int
        L.t0mi_probe_stream.argtypes = [P, P, SZ, I, U32, P]
        L.t0mi_probe_empty.argtypes = [P, U32, P]
        L.t0mi_probe_block.argtypes = [P, P, U32, U32, U32, U32, P]
        L.t0mi_probe_mfma.argtypes = [P, P, U32, U32, U32, P, P, I]
        L.t0mi_probe_mfma_flop.argtypes = [I]
        L.t0mi_probe_lds.argtypes = [P, P, U32, U32, U32, P]
        L.t0mi_probe_lds.restype = I
        L.t0mi_probe_mfma_flop.restype = ctypes.c_uint64
        for f in (L.t0mi_probe_stream, L.t0mi_probe_empty, L.t0mi_probe_mfma, L.t0mi_probe_block):
            f.restype = I
        _lib = L
    return _lib


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc})")


def stream(stream_ptr, src, nbytes, nt, grid, sink):
    _check(lib().t0mi_probe_stream(stream_ptr, src, nbytes, 1 if nt else 0, grid, sink), "t0mi_probe_stream")


def block(stream_ptr, src, rows, pitch, run_bytes, rows_per_wg, sink):
    _check(lib().t0mi_probe_block(stream_ptr, src, rows, pitch, run_bytes, rows_per_wg, sink), "t0mi_probe_block")


def empty(stream_ptr, grid, sink):
    _check(lib().t0mi_probe_empty(stream_ptr, grid, sink), "t0mi_probe_empty")


def mfma(stream_ptr, src, n_frag, iters, grid, out, stamps, variant=0):
    _check(lib().t0mi_probe_mfma(stream_ptr, src, n_frag, iters, grid, out, stamps, variant), "t0mi_probe_mfma")


# MFMA-loop variants: (waves per workgroup, wave tile, instruction, operands re-read from LDS)
MFMA_VARIANTS = {
    0: ("8 waves, 128x64 wave tile, 32x32x16, registers", False),
    1: ("8 waves, 128x64 wave tile, 32x32x16, LDS reads", True),
    2: ("4 waves, 128x128 wave tile, 32x32x16, registers", False),
    3: ("4 waves, 128x128 wave tile, 32x32x16, LDS reads", True),
    4: ("4 waves, 128x128 wave tile, 16x16x32, registers", False),
    5: ("4 waves, 128x128 wave tile, 16x16x32, LDS reads", True),
    6: ("8 waves, 128x64 wave tile, 16x16x32, registers", False),
    7: ("8 waves, 128x64 wave tile, 16x16x32, LDS reads", True),
}


def lds(stream_ptr, table, nbytes, iters, grid, out):
    _check(lib().t0mi_probe_lds(stream_ptr, table, nbytes, iters, grid, out), "t0mi_probe_lds")


def mfma_flop_per_iter(variant):
    """FLOP one workgroup of MFMA-loop `variant` runs per iteration (2^23 for all)."""
    return int(lib().t0mi_probe_mfma_flop(variant))
