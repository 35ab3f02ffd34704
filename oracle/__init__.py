"""CPU oracle for the GEMM hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product library ``libt0mi`` never loads it.

It wraps ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``), a C restatement of:

- ``cpu_gemm_nt_bf16``            src/t0/tile_ir.rs:5021-5038
- bf16 truncation / bf16 RNE      src/t0/tile_ir.rs:4677-4683,
                                  src/ignis/ops/bf16_matmul.rs:372
- the xorshift64 data generator   examples/test_gemm_correctness.rs:45-58
- INT4 unpack / dequant / GPTQ    src/t0/quant_kernels.rs:1-25, 74-100, 188-294

Parity pins live in ``tests/test_oracle.py``.  The reference itself is Rust and
cannot be built in this image (no cargo/rustc), so there is no ``oracle/_ref``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

# Seeds for BASELINE.json configs: A, B, scales, zeros, offset by 0x100 * config index.
SEED_A, SEED_B, SEED_S, SEED_Z = 0x7401, 0x7402, 0x7403, 0x7404


def seeds(config_index: int):
    off = 0x100 * config_index
    return SEED_A + off, SEED_B + off, SEED_S + off, SEED_Z + off


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_trunc.argtypes = [ctypes.c_float]
        L.orc_bf16_trunc.restype = ctypes.c_uint16
        L.orc_bf16_rne.argtypes = [ctypes.c_float]
        L.orc_bf16_rne.restype = ctypes.c_uint16
        L.orc_f32_to_bf16_rne_array.argtypes = [P, P, i64]
        L.orc_f32_to_bf16_trunc_array.argtypes = [P, P, i64]
        L.orc_rand_bf16_ref.argtypes = [P, i64, ctypes.c_uint64]
        L.orc_gen_uniform_bf16.argtypes = [P, i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.orc_gen_normal_bf16.argtypes = [P, i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.orc_gen_nibbles.argtypes = [P, i64, ctypes.c_uint64]
        L.orc_gemm_bf16.argtypes = [P, P, P, i64, i64, i64, ctypes.c_int, ctypes.c_int]
        L.orc_gemm_bf16.restype = ctypes.c_int
        L.orc_gemm_nt_bf16_literal.argtypes = [P, P, P, i64, i64, i64]
        L.orc_pack_qweight.argtypes = [P, P, i64, i64]
        L.orc_unpack_qweight.argtypes = [P, P, i64, i64]
        L.orc_pack_gptq_bytes.argtypes = [P, P, i64, i64]
        L.orc_unpack_gptq_bytes.argtypes = [P, P, i64, i64]
        L.orc_pack_qzeros.argtypes = [P, P, i64, i64]
        L.orc_dequant_qweight_f32.argtypes = [P, P, P, ctypes.c_int, P, i64, i64, i64]
        L.orc_dequant_gptq_f32.argtypes = [P, P, P, P, i64, i64, i64]
        L.orc_w4a16_gemm.argtypes = [P, P, P, P, ctypes.c_int, P, i64, i64, i64, i64, ctypes.c_int]
        L.orc_w4a16_gemm.restype = ctypes.c_int
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_epilogue.argtypes = [P, i64, i64, P, ctypes.c_int, P, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_float]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- bf16 ----

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_rne_array(_p(x), _p(out), x.size)
    return out


def bf16_trunc(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_trunc_array(_p(x), _p(out), x.size)
    return out


# ----------------------------------------------------------- generators ----

def rand_bf16_ref(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().orc_rand_bf16_ref(_p(out), n, seed)
    return out


def uniform_bf16(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().orc_gen_uniform_bf16(_p(out), out.size, seed, lo, hi)
    return out.reshape(shape)


def normal_bf16(shape, seed: int, mu: float, sigma: float) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.uint16)
    lib().orc_gen_normal_bf16(_p(out), out.size, seed, mu, sigma)
    return out.reshape(shape)


def nibbles(shape, seed: int) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.uint8)
    lib().orc_gen_nibbles(_p(out), out.size, seed)
    return out.reshape(shape)


# ----------------------------------------------------------------- GEMM ----

def gemm_bf16(a: np.ndarray, b: np.ndarray, b_layout: str = "nn", nthreads: int = 0) -> np.ndarray:
    """y = a @ b in the reference's sequential-fp32 order.

    a: uint16 bf16 bits [M, K].  b: [K, N] for ``nn`` or [N, K] for ``nt``.
    """
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = a.shape
    if b_layout == "nn":
        assert b.shape[0] == K
        N = b.shape[1]
    else:
        assert b.shape[1] == K
        N = b.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    rc = lib().orc_gemm_bf16(_p(a), _p(b), _p(y), M, N, K, 1 if b_layout == "nn" else 0, nthreads)
    if rc != 0:
        raise MemoryError("oracle gemm: allocation failed")
    return y


def gemm_nt_literal(x: np.ndarray, wt: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wt = np.ascontiguousarray(wt, dtype=np.uint16)
    M, K = x.shape
    N = wt.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_nt_bf16_literal(_p(x), _p(wt), _p(y), M, N, K)
    return y


# ----------------------------------------------------------------- INT4 ----

def pack_qweight(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    K, N = q.shape
    w = np.empty((K // 8, N), dtype=np.uint32)
    lib().orc_pack_qweight(_p(q), _p(w), K, N)
    return w


def unpack_qweight(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    KK, N = w.shape
    q = np.empty((KK * 8, N), dtype=np.uint8)
    lib().orc_unpack_qweight(_p(w), _p(q), KK * 8, N)
    return q


def pack_gptq_bytes(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    K, N = q.shape
    out = np.empty((N, K // 2), dtype=np.uint8)
    lib().orc_pack_gptq_bytes(_p(q), _p(out), K, N)
    return out


def unpack_gptq_bytes(packed: np.ndarray, K: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    N = packed.shape[0]
    q = np.empty((K, N), dtype=np.uint8)
    lib().orc_unpack_gptq_bytes(_p(packed), _p(q), K, N)
    return q


def pack_qzeros(z: np.ndarray) -> np.ndarray:
    z = np.ascontiguousarray(z, dtype=np.uint8)
    G, N = z.shape
    out = np.empty((G, N // 8), dtype=np.uint32)
    lib().orc_pack_qzeros(_p(z), _p(out), G, N)
    return out


def dequant_qweight_f32(w: np.ndarray, scales: np.ndarray, zeros, group: int, zp_const: int = 8) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    KK, N = w.shape
    K = KK * 8
    out = np.empty((K, N), dtype=np.float32)
    zp = None if zeros is None else np.ascontiguousarray(zeros, dtype=np.uint32)
    lib().orc_dequant_qweight_f32(_p(w), _p(scales), None if zp is None else _p(zp), zp_const,
                                  _p(out), K, N, group)
    return out


def dequant_gptq_f32(packed: np.ndarray, scales: np.ndarray, zp: np.ndarray,
                     rows: int, cols: int, group: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    zp = np.ascontiguousarray(zp, dtype=np.int32).reshape(-1)
    out = np.empty(rows * cols, dtype=np.float32)
    lib().orc_dequant_gptq_f32(_p(packed), _p(scales), _p(zp), _p(out), rows, cols, group)
    return out.reshape(rows, cols)


def w4a16_gemm(a: np.ndarray, w: np.ndarray, scales: np.ndarray, zeros, group: int,
               zp_const: int = 8, nthreads: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    M, K = a.shape
    N = w.shape[1]
    assert w.shape[0] * 8 == K
    y = np.empty((M, N), dtype=np.float32)
    zp = None if zeros is None else np.ascontiguousarray(zeros, dtype=np.uint32)
    rc = lib().orc_w4a16_gemm(_p(a), _p(w), _p(scales), None if zp is None else _p(zp), zp_const,
                              _p(y), M, N, K, group, nthreads)
    if rc != 0:
        raise MemoryError("oracle w4a16: allocation failed")
    return y


def epilogue(y: np.ndarray, ops, bias=None, scale: float = 1.0, clamp_min: float = 0.0,
             clamp_max: float = 0.0) -> np.ndarray:
    """tile_ir EpilogueOp chain (src/t0/tile_ir.rs:3400-3540) applied in order to fp32 y[M, N];
    ops are 0..7 = bias, scale, relu, silu, gelu, abs, neg, clamp.  Returns a new array."""
    out = np.ascontiguousarray(y, dtype=np.float32).copy()
    M, N = out.shape
    o = np.ascontiguousarray(list(ops), dtype=np.uint32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    if 0 in list(ops) and (b is None or b.shape != (N,)):
        raise ValueError("bias op needs a [N] float32 bias")
    lib().orc_epilogue(_p(out), M, N, _p(o) if o.size else None, int(o.size), None if b is None else _p(b),
                       scale, clamp_min, clamp_max)
    return out


def num_threads() -> int:
    return lib().orc_num_threads()


# ------------------------------------------------------------ tolerance ----

def gemm_tolerance(K: int, a_f32: np.ndarray, b_f32: np.ndarray) -> float:
    """max|err| <= 1e-2 * sqrt(K) * max|a| * max|b|  (BASELINE.json north_star)."""
    return 1e-2 * np.sqrt(K) * float(np.abs(a_f32).max()) * float(np.abs(b_f32).max())


def compare(out: np.ndarray, ref: np.ndarray):
    """Returns (max_abs_err, relative Frobenius error)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = out - ref
    max_err = float(np.abs(d).max()) if d.size else 0.0
    nref = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(d) / nref) if nref > 0 else float(np.linalg.norm(d))
    return max_err, rel
