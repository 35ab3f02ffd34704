"""t0mi — Python binding of libt0mi, the gfx950 GEMM hot path of T0-GPU.

The product is the C ABI in ``include/t0mi.h`` (implemented in
``rust-gpu_amd/csrc``); this module is a thin ``ctypes`` layer over it for
tests, the benchmark and Python callers.  Names follow the reference's Rust
API (``GemmConfig``, ``auto_select``, ``GemmTuner.tune``, ``GpuRuntime``
dispatch); each wrapper names the reference item it mirrors.

There is no fallback: if ``libt0mi.so`` is missing, importing this module
raises, and every compute call goes through the HIP kernels in the library.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_HERE, "libt0mi.so")

OK = 0
ERR_INVALID, ERR_NO_KERNEL, ERR_HIP, ERR_POISONED, ERR_KERNARG, ERR_TIMEOUT, ERR_NOT_FOUND, ERR_NO_DEVICE = \
    -1, -2, -3, -4, -5, -6, -7, -8
ERR_CAPTURE = -9
NT, NN = 0, 1
EPI_STORE_F32, EPI_BIAS_ADD, EPI_BIAS_ADD_RELU = 0, 1, 2
OUT_F32, OUT_BF16 = 0, 1
NOALLOC_SCRATCH_BYTES = 32 << 20  # T0MI_NOALLOC_SCRATCH_BYTES


def build(jobs: int = 8) -> str:
    """Compile libt0mi.so for gfx950 with the package Makefile (always rebuilds stale objects)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", _PKG_ROOT], check=True)
    return LIB_PATH


class T0miError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"t0mi error {code}: {msg}")
        self.code = code


class GemmConfig(ctypes.Structure):
    """Mirror of ``GemmConfig`` (src/t0/gemm_gen.rs:55-84) plus gfx950 fields."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "tile_m", "tile_n", "tile_k", "wg_size", "use_lds", "double_buffer", "split_k", "lds_pad",
        "n_col_passes", "swap_grid", "wgp_mode", "transpose", "epilogue", "out_dtype", "wave_m", "wave_n",
        "stages")]

    def copy(self, **kw) -> "GemmConfig":
        c = GemmConfig()
        ctypes.memmove(ctypes.byref(c), ctypes.byref(self), ctypes.sizeof(GemmConfig))
        for k, v in kw.items():
            setattr(c, k, v)
        return c

    def name(self) -> str:
        return config_name(self)

    def is_feasible(self) -> bool:
        return bool(lib().t0mi_config_is_feasible(ctypes.byref(self)))

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}

    def __repr__(self):
        return f"GemmConfig({self.name()})"


# tile_ir EpilogueOp (src/t0/tile_ir.rs:40-58)
BIAS_ADD, SCALE, RELU, SILU, GELU, ABS, NEG, CLAMP = range(8)
EPILOGUE_NAMES = ("bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp")


class TileGemm(ctypes.Structure):
    """Mirror of ``TileGemm`` (src/t0/tile_ir.rs:100-152) plus out_dtype."""
    _fields_ = ([(n, ctypes.c_uint32) for n in (
        "tile_m", "tile_n", "tile_k", "wgp_mode", "double_buffer", "triple_buffer", "split_k", "swap_grid",
        "transpose", "acc_swap", "n_epilogue")] + [("epilogue", ctypes.c_uint32 * 8)] +
        [(n, ctypes.c_uint32) for n in ("persistent", "waves_per_wg", "wmma_format", "out_dtype")])

    def copy(self, **kw) -> "TileGemm":
        c = TileGemm()
        ctypes.memmove(ctypes.byref(c), ctypes.byref(self), ctypes.sizeof(TileGemm))
        for k, v in kw.items():
            if k == "epilogue":
                c.set_epilogue(v)
            else:
                setattr(c, k, v)
        return c

    def set_epilogue(self, ops) -> "TileGemm":
        """``with_epilogue`` (tile_ir.rs:709-712)."""
        ops = list(ops)
        if len(ops) > 8:
            raise ValueError("at most 8 epilogue ops")
        self.n_epilogue = len(ops)
        for i in range(8):
            self.epilogue[i] = ops[i] if i < len(ops) else 0
        return self

    def add_epilogue(self, op: int) -> "TileGemm":
        """``add_epilogue`` (tile_ir.rs:704-707)."""
        return self.set_epilogue(self.epilogue_ops() + [op])

    def epilogue_ops(self) -> list:
        return [self.epilogue[i] for i in range(self.n_epilogue)]

    def name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        lib().t0mi_tile_name(ctypes.byref(self), buf, 256)
        return buf.value.decode()

    def n_waves(self) -> int:
        return lib().t0mi_tile_n_waves(ctypes.byref(self))

    def wg_size(self) -> int:
        return lib().t0mi_tile_wg_size(ctypes.byref(self))

    def lds_total(self) -> int:
        return lib().t0mi_tile_lds_total(ctypes.byref(self))

    def kernarg_size(self) -> int:
        return lib().t0mi_tile_kernarg_size(ctypes.byref(self))

    def __repr__(self):
        return f"TileGemm({self.name()})"


_lib = None

# Every symbol declared in include/t0mi.h, with (restype, argtypes).
_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_I = ctypes.c_int
_CFG = ctypes.POINTER(GemmConfig)
_CHARP = ctypes.c_char_p
_F32 = ctypes.c_float
_TS = ctypes.POINTER(TileGemm)
SIGNATURES = {
    "t0mi_last_error": (_CHARP, []),
    "t0mi_abi_version": (_I, []),
    "t0mi_build_target": (_CHARP, []),
    "t0mi_config_preset": (_I, [_CHARP, _CFG]),
    "t0mi_config_preset_names": (_I, [_CHARP, _SZ]),
    "t0mi_gemm_variants": (_I, [_CHARP, _SZ]),
    "t0mi_config_n_waves": (_U32, [_CFG]),
    "t0mi_config_lds_total": (_U32, [_CFG]),
    "t0mi_config_estimated_regs": (_U32, [_CFG]),
    "t0mi_config_is_feasible": (_I, [_CFG]),
    "t0mi_config_name": (_I, [_CFG, _CHARP, _SZ]),
    "t0mi_compute_grid": (_I, [_CFG, _U32, _U32, ctypes.POINTER(_U32)]),
    "t0mi_compute_grid_split_k": (_I, [_CFG, _U32, _U32, _U32, ctypes.POINTER(_U32)]),
    "t0mi_compute_grid_auto": (_I, [_CFG, _U32, _U32, ctypes.POINTER(_U32)]),
    "t0mi_build_kernargs": (_I, [_U64, _U64, _U64, _U32, _U32, _U32, _CFG, _P]),
    "t0mi_build_kernargs_with_bias": (_I, [_U64, _U64, _U64, _U32, _U32, _U32, _CFG, _U64, _P]),
    "t0mi_auto_select": (_I, [_U32, _U32, _U32, _CFG]),
    "t0mi_auto_select_legacy": (_I, [_U32, _U32, _U32, _CFG]),
    "t0mi_auto_select_layout": (_I, [_U32, _U32, _U32, _U32, _U32, _CFG]),
    "t0mi_set_w4a16_workspace_limit": (_I, [_P, _U64]),
    "t0mi_auto_schedule_gemm": (_I, [_U32, _U32, _U32, _U32, _U32, _P, _P, _U32, ctypes.POINTER(_U32)]),
    "t0mi_auto_gemm_plan": (_I, [_U32, _U32, _U32, _U32, _U32, _CFG, ctypes.POINTER(_U32), _CFG]),
    "t0mi_cached_auto_select": (_I, [_U32, _U32, _U32, _CFG]),
    "t0mi_clear_spec_cache": (None, []),
    "t0mi_spec_cache_len": (_SZ, []),
    "t0mi_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "t0mi_ctx_create_on_stream": (_I, [_I, _P, ctypes.POINTER(_P)]),
    "t0mi_ctx_create_null": (_I, [ctypes.POINTER(_P)]),
    "t0mi_ctx_destroy": (None, [_P]),
    "t0mi_ctx_stream": (_P, [_P]),
    "t0mi_is_poisoned": (_I, [_P]),
    "t0mi_mark_poisoned": (None, [_P]),
    "t0mi_set_timeout_ms": (None, [_P, _U32]),
    "t0mi_null_inject_timeout": (_I, [_P]),
    "t0mi_null_last_dispatch": (_I, [_P, ctypes.POINTER(_U32), _P, _SZ, ctypes.POINTER(_SZ)]),
    "t0mi_alloc": (_I, [_P, _SZ, ctypes.POINTER(_U64)]),
    "t0mi_alloc_zero": (_I, [_P, _SZ, ctypes.POINTER(_U64)]),
    "t0mi_free": (_I, [_P, _U64]),
    "t0mi_alloc_f32": (_I, [_P, _SZ, ctypes.POINTER(_U64)]),
    "t0mi_recycle": (_I, [_P, _U64]),
    "t0mi_pool_cached_bytes": (_SZ, [_P]),
    "t0mi_pool_clear": (_I, [_P]),
    "t0mi_xcd_placement": (_I, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32)]),
    "t0mi_h2d": (_I, [_P, _U64, _P, _SZ]),
    "t0mi_d2h": (_I, [_P, _P, _U64, _SZ]),
    "t0mi_memset": (_I, [_P, _U64, _I, _SZ]),
    "t0mi_kernel_get": (_I, [_P, _CFG, ctypes.POINTER(_P)]),
    "t0mi_kernel_attrs": (_I, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32), ctypes.POINTER(_U32)]),
    "t0mi_kernel_name": (_I, [_P, _CHARP, _SZ]),
    "t0mi_dispatch": (_I, [_P, _P, ctypes.POINTER(_U32), _P, _SZ]),
    "t0mi_dispatch_async": (_I, [_P, _P, ctypes.POINTER(_U32), _P, _SZ]),
    "t0mi_wait_idle": (_I, [_P]),
    "t0mi_gemm": (_I, [_P, _CFG, _U64, _U64, _U64, _U64, _U32, _U32, _U32]),
    "t0mi_gemm_noalloc": (_I, [_P, _CFG, _U64, _U64, _U64, _U64, _U32, _U32, _U32]),
    "t0mi_dq_new": (_I, [_P, ctypes.POINTER(_P)]),
    "t0mi_dq_submit": (_I, [_P, _P, ctypes.POINTER(_U32), _P, _SZ]),
    "t0mi_dq_flush": (_I, [_P, ctypes.POINTER(_SZ)]),
    "t0mi_dq_pending": (_SZ, [_P]),
    "t0mi_dq_drop_async": (None, [_P]),
    "t0mi_batch_dispatch": (_I, [_P, _SZ, ctypes.POINTER(_P), ctypes.POINTER(_U32), ctypes.POINTER(_P),
                                 ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "t0mi_capture_begin": (_I, [_P]),
    "t0mi_capture_end": (_I, [_P, ctypes.POINTER(_P)]),
    "t0mi_graph_launch": (_I, [_P]),
    "t0mi_graph_node_count": (_SZ, [_P]),
    "t0mi_graph_destroy": (None, [_P]),
    "t0mi_tuner_create": (_I, [_CHARP, ctypes.POINTER(_P)]),
    "t0mi_tuner_destroy": (None, [_P]),
    "t0mi_tuner_set_params": (None, [_P, _U32, _U32]),
    "t0mi_tuner_tune": (_I, [_P, _P, _U32, _U32, _U32, _U32, _U32, _CFG, ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(_I)]),
    "t0mi_tuner_invalidate": (None, [_P, _U32, _U32, _U32, _U32, _U32]),
    "t0mi_tuner_clear": (None, [_P]),
    "t0mi_tuner_cache_path": (_I, [_P, _U32, _U32, _U32, _U32, _U32, _CHARP, _SZ]),
    "t0mi_tuner_report": (_I, [_P, _CHARP, _SZ]),
    "t0mi_auto_gemm": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32, ctypes.POINTER(ctypes.c_double)]),
    "t0mi_tile_preset": (_I, [_CHARP, _TS]),
    "t0mi_tile_preset_names": (_CHARP, []),
    "t0mi_tile_name": (_I, [_TS, _CHARP, _SZ]),
    "t0mi_tile_n_waves": (_U32, [_TS]),
    "t0mi_tile_wg_size": (_U32, [_TS]),
    "t0mi_tile_lds_total": (_U32, [_TS]),
    "t0mi_tile_auto_select": (_I, [_U32, _U32, _U32, _U32, _TS]),
    "t0mi_tile_kernarg_size": (_U32, [_TS]),
    "t0mi_tile_build_kernargs": (_I, [_U64, _U64, _U64, _U32, _U32, _TS, _P, _SZ]),
    "t0mi_tile_build_kernargs_m": (_I, [_U64, _U64, _U64, _U32, _U32, _U32, _TS, _P, _SZ]),
    "t0mi_tile_build_kernargs_m_with_counter": (_I, [_U64, _U64, _U64, _U32, _U32, _U32, _TS, _U64, _U32, _U32,
                                                     _P, _SZ]),
    "t0mi_tile_append_epilogue_args": (_I, [_TS, _U64, _F32, _F32, _F32, _P, _SZ, ctypes.POINTER(_SZ)]),
    "t0mi_tile_compute_grid": (_I, [_TS, _U32, _U32, ctypes.POINTER(_U32)]),
    "t0mi_tile_kernel_get": (_I, [_P, _TS, ctypes.POINTER(_P)]),
    "t0mi_tile_gemm": (_I, [_P, _TS, _U64, _U64, _U64, _U32, _U32, _U32, _U64, _F32, _F32, _F32]),
    "t0mi_w4a16_gemm": (_I, [_P, _U64, _U64, _U64, _U64, _U32, _U64, _U32, _U32, _U32, _U32, _U32]),
    "t0mi_dequant_int4": (_I, [_P, _U64, _U64, _U64, _U32, _U64, _U32, _U32, _U32, _U32]),
    "t0mi_gptq_parse": (_I, [_P, _SZ, _P]),
    "t0mi_gptq_gpu_buffer_size": (_U64, [_P]),
    "t0mi_gptq_convert": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32, _U64, _U64, _U64]),
    "t0mi_f32_to_bf16": (_I, [_P, _U64, _U64, _U64]),
    "t0mi_matmul_f32": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32]),
    "t0mi_matmul_wt_bf16": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32]),
    "t0mi_matmul_backward_data": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32]),
    "t0mi_matmul_backward_weight": (_I, [_P, _U64, _U64, _U64, _U32, _U32, _U32]),
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"libt0mi.so not built at {LIB_PATH}; run __graft_entry__.build() "
                              f"(make -C {_PKG_ROOT})")
        # One HIP runtime per process: when torch is installed, load it first so
        # libt0mi binds to the HIP runtime torch already mapped (same soname).
        # Loaded the other way round, the two runtimes contend for the device
        # and the second to initialise sees no GPU.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().t0mi_last_error().decode()


def check(rc: int) -> int:
    if rc != OK:
        raise T0miError(rc, last_error())
    return rc


# ------------------------------------------------------------- config ----

def preset(name: str) -> GemmConfig:
    """``GemmConfig::tile_*()`` presets (src/t0/gemm_gen.rs:87-145) and gfx950 presets."""
    c = GemmConfig()
    check(lib().t0mi_config_preset(name.encode(), ctypes.byref(c)))
    return c


def preset_names() -> list:
    buf = ctypes.create_string_buffer(4096)
    lib().t0mi_config_preset_names(buf, 4096)
    return buf.value.decode().split(",")


def variants(transpose: Optional[int] = None) -> list:
    """Configs of every prebuilt gfx950 GEMM kernel (optionally one layout)."""
    buf = ctypes.create_string_buffer(16384)
    lib().t0mi_gemm_variants(buf, 16384)
    out = []
    for e in buf.value.decode().split(","):
        nn = e.endswith("_nn")
        tile, wave, st = e.replace("_nn", "").replace("_s", "_w").split("_w")
        bm, bn, bk = map(int, tile.split("x"))
        wm, wn = map(int, wave.split("x"))
        if transpose is not None and transpose != (NN if nn else NT):
            continue
        c = GemmConfig(tile_m=bm, tile_n=bn, tile_k=bk, wg_size=64 * wm * wn, use_lds=1, double_buffer=1,
                       n_col_passes=1, swap_grid=1, transpose=NN if nn else NT, wave_m=wm, wave_n=wn,
                       stages=0 if int(st) == 2 else int(st))
        out.append(c)
    return out


def config_name(cfg: GemmConfig) -> str:
    buf = ctypes.create_string_buffer(256)
    check_len = lib().t0mi_config_name(ctypes.byref(cfg), buf, 256)
    if check_len < 0:
        raise T0miError(check_len, last_error())
    return buf.value.decode()


def lds_total(cfg: GemmConfig) -> int:
    return lib().t0mi_config_lds_total(ctypes.byref(cfg))


def compute_grid(cfg: GemmConfig, m: int, n: int):
    g = (ctypes.c_uint32 * 2)()
    check(lib().t0mi_compute_grid(ctypes.byref(cfg), m, n, g))
    return (g[0], g[1])


def compute_grid_split_k(cfg: GemmConfig, m: int, n: int, split_k: int):
    g = (ctypes.c_uint32 * 2)()
    check(lib().t0mi_compute_grid_split_k(ctypes.byref(cfg), m, n, split_k, g))
    return (g[0], g[1])


def compute_grid_auto(cfg: GemmConfig, m: int, n: int):
    g = (ctypes.c_uint32 * 2)()
    check(lib().t0mi_compute_grid_auto(ctypes.byref(cfg), m, n, g))
    return (g[0], g[1])


def build_kernargs(x: int, wt: int, y: int, k: int, n: int, m: int, cfg: GemmConfig) -> bytes:
    """``gemm_gen::build_kernargs(x, wt, y, k, n, m, cfg)`` — 40 bytes (gemm_gen.rs:439-458)."""
    buf = (ctypes.c_uint8 * 40)()
    check(lib().t0mi_build_kernargs(x, wt, y, k, n, m, ctypes.byref(cfg), buf))
    return bytes(buf)


def build_kernargs_with_bias(x: int, wt: int, y: int, k: int, n: int, m: int, cfg: GemmConfig, bias: int) -> bytes:
    buf = (ctypes.c_uint8 * 48)()
    check(lib().t0mi_build_kernargs_with_bias(x, wt, y, k, n, m, ctypes.byref(cfg), bias, buf))
    return bytes(buf)


def auto_select(m: int, k: int, n: int) -> GemmConfig:
    """``gemm_gen::auto_select(m, k, n)`` — note the (m, k, n) order."""
    c = GemmConfig()
    check(lib().t0mi_auto_select(m, k, n, ctypes.byref(c)))
    return c


def auto_select_layout(m: int, k: int, n: int, transpose: int = NN, out_dtype: int = OUT_F32) -> GemmConfig:
    """auto_select for a given B layout and output dtype (gfx950 extension of gemm_gen.rs:340)."""
    c = GemmConfig()
    check(lib().t0mi_auto_select_layout(m, k, n, transpose, out_dtype, ctypes.byref(c)))
    return c


def auto_schedule_gemm(m: int, n: int, k: int, transpose: int = NN, out_dtype: int = OUT_F32, cap: int = 64):
    """cost_model::auto_schedule_gemm (src/t0/cost_model.rs:464-534): [(GemmConfig, estimated us)],
    best first, at most cap entries (note the reference's (m, n, k) order)."""
    cfgs = (GemmConfig * cap)()
    est = (ctypes.c_double * cap)()
    count = ctypes.c_uint32(0)
    check(lib().t0mi_auto_schedule_gemm(m, n, k, transpose, out_dtype, ctypes.cast(cfgs, _P), ctypes.cast(est, _P),
                                        cap, ctypes.byref(count)))
    return [(cfgs[i].copy(), est[i]) for i in range(min(cap, count.value))]


def auto_gemm_plan(m: int, n: int, k: int, transpose: int = NN, out_dtype: int = OUT_F32):
    """The schedule of the library's auto-scheduled GEMMs: (head, n_main, tail) -- head over columns
    [0, n_main), tail over [n_main, n) when n_main < n (tail is head otherwise)."""
    head, tail = GemmConfig(), GemmConfig()
    n_main = ctypes.c_uint32(0)
    check(lib().t0mi_auto_gemm_plan(m, n, k, transpose, out_dtype, ctypes.byref(head), ctypes.byref(n_main),
                                    ctypes.byref(tail)))
    return head, n_main.value, tail


def auto_select_legacy(m: int, k: int, n: int) -> GemmConfig:
    c = GemmConfig()
    check(lib().t0mi_auto_select_legacy(m, k, n, ctypes.byref(c)))
    return c


def cached_auto_select(m: int, k: int, n: int) -> GemmConfig:
    c = GemmConfig()
    check(lib().t0mi_cached_auto_select(m, k, n, ctypes.byref(c)))
    return c


# ------------------------------------------------------------ tile_ir ----

def tile_preset(name: str) -> TileGemm:
    """``TileGemm::<name>()`` (src/t0/tile_ir.rs:156-604)."""
    s = TileGemm()
    check(lib().t0mi_tile_preset(name.encode(), ctypes.byref(s)))
    return s


def tile_preset_names() -> list:
    return lib().t0mi_tile_preset_names().decode().split(",")


def tile_auto_select(m: int, k: int, n: int, transpose: int = NT) -> TileGemm:
    """``tile_auto_select(m, k, n, transpose)`` (src/t0/tile_ir.rs:740-870)."""
    s = TileGemm()
    check(lib().t0mi_tile_auto_select(m, k, n, transpose, ctypes.byref(s)))
    return s


def _ka(fn, *args) -> bytes:
    buf = (ctypes.c_uint8 * 128)()
    n = fn(*args, buf, 128)
    if n < 0:
        check(n)
    return bytes(buf[:n])


def tile_build_kernargs(x: int, wt: int, y: int, k: int, n: int, spec: TileGemm) -> bytes:
    """``build_kernargs`` (tile_ir.rs:4570-4593): 44 bytes, M slot 0."""
    return _ka(lib().t0mi_tile_build_kernargs, x, wt, y, k, n, ctypes.byref(spec))


def tile_build_kernargs_m(x: int, wt: int, y: int, k: int, n: int, m: int, spec: TileGemm) -> bytes:
    """``build_kernargs_m`` (tile_ir.rs:4595-4602)."""
    return _ka(lib().t0mi_tile_build_kernargs_m, x, wt, y, k, n, m, ctypes.byref(spec))


def tile_build_kernargs_m_with_counter(x: int, wt: int, y: int, k: int, n: int, m: int, spec: TileGemm,
                                       counter: int, n_tiles_n_shift: int, tiles_per_wg: int) -> bytes:
    """``build_kernargs_m_with_counter`` (tile_ir.rs:4604-4637)."""
    return _ka(lib().t0mi_tile_build_kernargs_m_with_counter, x, wt, y, k, n, m, ctypes.byref(spec), counter,
               n_tiles_n_shift, tiles_per_wg)


def tile_append_epilogue_args(spec: TileGemm, ka: bytes, bias: int = 0, scale: float = 1.0,
                              clamp_min: float = 0.0, clamp_max: float = 0.0) -> bytes:
    """The epilogue kernargs lower_gemm declares (tile_ir.rs:1014-1027), after the GEMM ones."""
    buf = (ctypes.c_uint8 * 128).from_buffer_copy(ka + b"\0" * (128 - len(ka)))
    n = ctypes.c_size_t(len(ka))
    check(lib().t0mi_tile_append_epilogue_args(ctypes.byref(spec), bias, scale, clamp_min, clamp_max, buf, 128,
                                               ctypes.byref(n)))
    return bytes(buf[: n.value])


def tile_compute_grid(spec: TileGemm, m: int, n: int):
    """``compute_grid`` (tile_ir.rs:4645-4666), in work-items."""
    g = (ctypes.c_uint32 * 3)()
    check(lib().t0mi_tile_compute_grid(ctypes.byref(spec), m, n, g))
    return (g[0], g[1], g[2])


# ------------------------------------------------------------ runtime ----

class Kernel:
    """``GpuKernel`` — a prebuilt gfx950 kernel looked up by config name."""

    def __init__(self, handle, rt):
        self.handle = handle
        self._rt = rt  # keeps the owning runtime alive

    def attrs(self):
        lds, wg, ka = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        check(lib().t0mi_kernel_attrs(self.handle, ctypes.byref(lds), ctypes.byref(wg), ctypes.byref(ka)))
        return {"lds_size": lds.value, "wg_size": wg.value, "kernarg_size": ka.value}

    @property
    def name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        lib().t0mi_kernel_name(self.handle, buf, 256)
        return buf.value.decode()


def _grid3(grid: Sequence[int]):
    return (ctypes.c_uint32 * 3)(*(list(grid) + [1] * (3 - len(grid))))


class DispatchQueue:
    """``DispatchQueue`` (src/t0/prefill_dispatch.rs:58-187): asynchronous
    submits on the runtime's stream, one wait at ``flush``."""

    def __init__(self, rt: "Runtime"):
        h = ctypes.c_void_p()
        check(lib().t0mi_dq_new(rt.handle, ctypes.byref(h)))
        self.handle = h
        self._rt = rt

    def submit(self, kernel: Kernel, grid: Sequence[int], ka: bytes) -> None:
        buf = (ctypes.c_uint8 * max(1, len(ka))).from_buffer_copy(ka or b"\0")
        check(lib().t0mi_dq_submit(self.handle, kernel.handle, _grid3(grid), buf, len(ka)))

    def flush(self) -> int:
        n = ctypes.c_size_t()
        check(lib().t0mi_dq_flush(self.handle, ctypes.byref(n)))
        return n.value

    def pending(self) -> int:
        return lib().t0mi_dq_pending(self.handle)

    def drop_async(self) -> None:
        if self.handle:
            lib().t0mi_dq_drop_async(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.drop_async()
        except Exception:
            pass


def batch_dispatch(rt: "Runtime", dispatches) -> int:
    """``batch_dispatch`` (prefill_dispatch.rs:204-214): ``dispatches`` is a
    sequence of (Kernel, grid, kernarg bytes); submit all, flush once."""
    n = len(dispatches)
    kernels = (ctypes.c_void_p * max(1, n))(*[d[0].handle for d in dispatches])
    grids = (ctypes.c_uint32 * max(3, 3 * n))(*[g for d in dispatches for g in _grid3(d[1])])
    bufs = [(ctypes.c_uint8 * max(1, len(d[2]))).from_buffer_copy(d[2] or b"\0") for d in dispatches]
    kas = (ctypes.c_void_p * max(1, n))(*[ctypes.addressof(b) for b in bufs])
    lens = (ctypes.c_size_t * max(1, n))(*[len(d[2]) for d in dispatches])
    count = ctypes.c_size_t()
    check(lib().t0mi_batch_dispatch(rt.handle, n, kernels, grids, kas, lens, ctypes.byref(count)))
    return count.value


class Graph:
    """A batch of library calls recorded from a runtime's stream (HIP graph);
    ``launch`` replays it asynchronously on that stream."""

    def __init__(self, handle, rt: "Runtime"):
        self.handle = handle
        self._rt = rt

    def launch(self) -> None:
        check(lib().t0mi_graph_launch(self.handle))

    @property
    def node_count(self) -> int:
        return lib().t0mi_graph_node_count(self.handle)

    def destroy(self) -> None:
        if self.handle:
            lib().t0mi_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Runtime:
    """``GpuRuntime`` (src/ignis/gpu_context.rs:99-545) over HIP."""

    def __init__(self, device: int = -1, stream: Optional[int] = None, null: bool = False):
        h = ctypes.c_void_p()
        if null:
            check(lib().t0mi_ctx_create_null(ctypes.byref(h)))
        elif stream is not None:
            check(lib().t0mi_ctx_create_on_stream(device, ctypes.c_void_p(stream), ctypes.byref(h)))
        else:
            check(lib().t0mi_ctx_create(device, ctypes.byref(h)))
        self.handle = h

    @classmethod
    def on_torch_stream(cls, device: int = 0):
        import torch
        return cls(device=device, stream=torch.cuda.current_stream(device).cuda_stream)

    def close(self):
        if self.handle:
            lib().t0mi_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return lib().t0mi_ctx_stream(self.handle) or 0

    def is_poisoned(self) -> bool:
        return bool(lib().t0mi_is_poisoned(self.handle))

    def mark_poisoned(self):
        lib().t0mi_mark_poisoned(self.handle)

    def set_timeout_ms(self, ms: int):
        lib().t0mi_set_timeout_ms(self.handle, ms)

    def inject_timeout(self):
        check(lib().t0mi_null_inject_timeout(self.handle))

    def last_dispatch(self):
        g = (ctypes.c_uint32 * 3)()
        buf = (ctypes.c_uint8 * 256)()
        n = ctypes.c_size_t()
        check(lib().t0mi_null_last_dispatch(self.handle, g, buf, 256, ctypes.byref(n)))
        return (g[0], g[1], g[2]), bytes(buf[: n.value])

    # memory
    def alloc(self, nbytes: int, zero: bool = False) -> int:
        p = ctypes.c_uint64()
        f = lib().t0mi_alloc_zero if zero else lib().t0mi_alloc
        check(f(self.handle, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, dptr: int):
        check(lib().t0mi_free(self.handle, dptr))

    def alloc_f32(self, n: int) -> int:
        """``GpuRuntime::alloc_f32``: n floats (at least 512 bytes, rounded to 512), zeroed."""
        p = ctypes.c_uint64()
        check(lib().t0mi_alloc_f32(self.handle, n, ctypes.byref(p)))
        return p.value

    def recycle(self, dptr: int):
        """``GpuRuntime::recycle``: back to the pool, no wait, no free."""
        check(lib().t0mi_recycle(self.handle, dptr))

    def pool_cached_bytes(self) -> int:
        return lib().t0mi_pool_cached_bytes(self.handle)

    def pool_clear(self):
        check(lib().t0mi_pool_clear(self.handle))

    def xcd_placement(self):
        """(XCDs the W4A16 decode's in-launch split-K exchange uses or 0, whether an exchange
        launch found a workgroup on another XCD than its numbering planned).  The second is
        informational: the partials are written through to memory, results do not depend on it."""
        n, bad = ctypes.c_uint32(), ctypes.c_uint32()
        check(lib().t0mi_xcd_placement(self.handle, ctypes.byref(n), ctypes.byref(bad)))
        return n.value, bool(bad.value)

    def h2d(self, dptr: int, host_bytes) -> None:
        import numpy as np
        arr = np.ascontiguousarray(host_bytes)
        check(lib().t0mi_h2d(self.handle, dptr, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))

    def d2h(self, dptr: int, out) -> None:
        check(lib().t0mi_d2h(self.handle, out.ctypes.data_as(ctypes.c_void_p), dptr, out.nbytes))

    # kernels
    def kernel(self, cfg: GemmConfig) -> Kernel:
        """``ensure_kernel_t0(cfg.name(), || generate(&cfg), ..)`` -> prebuilt kernel."""
        h = ctypes.c_void_p()
        check(lib().t0mi_kernel_get(self.handle, ctypes.byref(cfg), ctypes.byref(h)))
        return Kernel(h, self)

    def tile_kernel(self, spec: TileGemm) -> Kernel:
        """``lower_gemm(&spec)`` + compile + load -> the prebuilt gfx950 kernel for the spec."""
        h = ctypes.c_void_p()
        check(lib().t0mi_tile_kernel_get(self.handle, ctypes.byref(spec), ctypes.byref(h)))
        return Kernel(h, self)

    def tile_gemm(self, spec: TileGemm, x: int, wt: int, y: int, m: int, n: int, k: int, bias: int = 0,
                  scale: float = 1.0, clamp_min: float = 0.0, clamp_max: float = 0.0) -> None:
        check(lib().t0mi_tile_gemm(self.handle, ctypes.byref(spec), x, wt, y, m, n, k, bias, scale, clamp_min,
                                   clamp_max))

    def dispatch(self, k: Kernel, grid: Sequence[int], ka: bytes, sync: bool = True) -> int:
        g = _grid3(grid)
        buf = (ctypes.c_uint8 * max(1, len(ka))).from_buffer_copy(ka or b"\0")
        f = lib().t0mi_dispatch if sync else lib().t0mi_dispatch_async
        return f(self.handle, k.handle, g, buf, len(ka))

    def wait_idle(self) -> int:
        return lib().t0mi_wait_idle(self.handle)

    # batched submission as a HIP graph
    def capture_begin(self) -> None:
        check(lib().t0mi_capture_begin(self.handle))

    def capture_end(self) -> Graph:
        h = ctypes.c_void_p()
        check(lib().t0mi_capture_end(self.handle, ctypes.byref(h)))
        return Graph(h, self)

    def gemm(self, cfg: GemmConfig, x: int, b: int, y: int, m: int, n: int, k: int, bias: int = 0) -> None:
        check(lib().t0mi_gemm(self.handle, ctypes.byref(cfg), x, b, y, bias, m, n, k))

    def gemm_noalloc(self, cfg: GemmConfig, x: int, b: int, y: int, m: int, n: int, k: int,
                     bias: int = 0) -> None:
        """gemm() with its split-K planes in the library's static per-GPU scratch
        (NOALLOC_SCRATCH_BYTES): allocates nothing; overlapping calls on one GPU race."""
        check(lib().t0mi_gemm_noalloc(self.handle, ctypes.byref(cfg), x, b, y, bias, m, n, k))

    def w4a16_gemm(self, a: int, qweight: int, scales: int, qzeros: int, zp_const: int, y: int,
                   m: int, k: int, n: int, group: int, out_dtype: int = OUT_BF16) -> None:
        check(lib().t0mi_w4a16_gemm(self.handle, a, qweight, scales, qzeros, zp_const, y, m, k, n, group, out_dtype))

    def set_w4a16_workspace_limit(self, nbytes: int) -> None:
        """Largest dequantized-weight buffer the W4A16 dequant-once route may use on this runtime;
        above it the fused kernels run (no reference counterpart)."""
        check(lib().t0mi_set_w4a16_workspace_limit(self.handle, nbytes))

    def dequant_int4(self, qweight: int, scales: int, qzeros: int, zp_const: int, out: int,
                     k: int, n: int, group: int, round_mode: int) -> None:
        check(lib().t0mi_dequant_int4(self.handle, qweight, scales, qzeros, zp_const, out, k, n, group, round_mode))

    # ---- Ignis matmul caller (src/ignis/ops/bf16_matmul.rs:33-423) ----
    def f32_to_bf16(self, src: int, dst: int, count: int) -> None:
        """f32 -> bf16 round-to-nearest-even on the GPU (bf16_matmul.rs:372)."""
        check(lib().t0mi_f32_to_bf16(self.handle, src, dst, count))

    def matmul(self, x: int, w: int, y: int, m: int, k: int, n: int) -> None:
        """``matmul`` forward (bf16_matmul.rs:33-96): Y[m,n] = bf16(X) . bf16(W), f32 in and out."""
        check(lib().t0mi_matmul_f32(self.handle, x, w, y, m, k, n))

    def matmul_with_wt_bf16(self, x: int, wt_bf16: int, y: int, m: int, k: int, n: int) -> None:
        """``matmul_with_wt_bf16`` (bf16_matmul.rs:99-134): X f32 [m,k], WT bf16 [n,k]."""
        check(lib().t0mi_matmul_wt_bf16(self.handle, x, wt_bf16, y, m, k, n))

    def matmul_backward_data(self, dy: int, w: int, dx: int, m: int, k: int, n: int) -> None:
        """``gemm_backward_data`` (bf16_matmul.rs:216-262): dX = dY . W^T."""
        check(lib().t0mi_matmul_backward_data(self.handle, dy, w, dx, m, k, n))

    def matmul_backward_weight(self, x: int, dy: int, dw: int, m: int, k: int, n: int) -> None:
        """``gemm_backward_weight`` (bf16_matmul.rs:268-316): dW = X^T . dY."""
        check(lib().t0mi_matmul_backward_weight(self.handle, x, dy, dw, m, k, n))

    def gptq_convert(self, packed: int, scales_f32: int, zeros_i32: int, rows: int, cols: int, group: int,
                     qweight: int, scales_bf16: int, qzeros: int) -> None:
        """GPTQ sections (device) -> t0mi_w4a16_gemm layouts (K = cols, N = rows)."""
        check(lib().t0mi_gptq_convert(self.handle, packed, scales_f32, zeros_i32, rows, cols, group, qweight,
                                      scales_bf16, qzeros))

    def auto_gemm(self, a: int, b: int, c: int, m: int, n: int, k: int) -> float:
        tf = ctypes.c_double()
        check(lib().t0mi_auto_gemm(self.handle, a, b, c, m, n, k, ctypes.byref(tf)))
        return tf.value


class GptqInfo(ctypes.Structure):
    """``t0mi_gptq_info``: the header and section offsets of a GPTQ byte container."""
    _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("n_groups", ctypes.c_uint32), ("packed_offset", ctypes.c_uint64), ("packed_bytes", ctypes.c_uint64),
                ("scales_offset", ctypes.c_uint64), ("zeros_offset", ctypes.c_uint64),
                ("total_bytes", ctypes.c_uint64), ("zeros_in_range", ctypes.c_uint32),
                ("scales_bf16_exact", ctypes.c_uint32)]


class GptqWeight:
    """``GptqWeight`` (src/t0/quant_kernels.rs:188-294): rows = output features (N),
    cols = input features (K); packed INT4 bytes [rows][cols/2] (element 2i = low
    nibble of byte i), f32 scales and i32 zero points at [row * n_groups + g]."""

    def __init__(self, raw: bytes, info: GptqInfo):
        self.raw = raw
        self.info = info
        self.rows, self.cols, self.group_size, self.n_groups = info.rows, info.cols, info.group_size, info.n_groups

    @classmethod
    def from_bytes(cls, raw: bytes) -> "GptqWeight":
        """``GptqWeight::from_bytes`` (quant_kernels.rs:242-286); raises T0miError where the reference panics."""
        info = GptqInfo()
        buf = ctypes.create_string_buffer(bytes(raw), len(raw)) if len(raw) else ctypes.create_string_buffer(1)
        check(lib().t0mi_gptq_parse(buf, len(raw), ctypes.byref(info)))
        return cls(bytes(raw), info)

    def gpu_buffer_size(self) -> int:
        """``GptqWeight::gpu_buffer_size`` (quant_kernels.rs:289-293)."""
        return int(lib().t0mi_gptq_gpu_buffer_size(ctypes.byref(self.info)))

    @property
    def packed_weights(self) -> bytes:
        i = self.info
        return self.raw[i.packed_offset:i.packed_offset + i.packed_bytes]

    @property
    def scales_bytes(self) -> bytes:
        i = self.info
        return self.raw[i.scales_offset:i.zeros_offset]

    @property
    def zeros_bytes(self) -> bytes:
        i = self.info
        return self.raw[i.zeros_offset:i.total_bytes]


class GemmTuner:
    """``GemmTuner`` (src/t0/auto_gemm.rs:46-527)."""

    def __init__(self, cache_dir: Optional[str] = None, max_candidates: int = 8, n_iters: int = 5):
        h = ctypes.c_void_p()
        check(lib().t0mi_tuner_create(cache_dir.encode() if cache_dir else None, ctypes.byref(h)))
        self.handle = h
        lib().t0mi_tuner_set_params(h, max_candidates, n_iters)

    def __del__(self):
        try:
            if self.handle:
                lib().t0mi_tuner_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    def tune(self, rt: Runtime, m: int, n: int, k: int, transpose: int = NT, out_dtype: int = OUT_F32):
        """``GemmTuner::tune(rt, m, n, k)`` -> (config, tflops, from_cache)."""
        c = GemmConfig()
        tf = ctypes.c_double()
        fc = ctypes.c_int()
        check(lib().t0mi_tuner_tune(self.handle, rt.handle, m, n, k, transpose, out_dtype, ctypes.byref(c),
                                    ctypes.byref(tf), ctypes.byref(fc)))
        return c, tf.value, bool(fc.value)

    def invalidate(self, m, n, k, transpose=NT, out_dtype=OUT_F32):
        lib().t0mi_tuner_invalidate(self.handle, m, n, k, transpose, out_dtype)

    def clear(self):
        lib().t0mi_tuner_clear(self.handle)

    def cache_path(self, m, n, k, transpose=NT, out_dtype=OUT_F32) -> str:
        buf = ctypes.create_string_buffer(1024)
        lib().t0mi_tuner_cache_path(self.handle, m, n, k, transpose, out_dtype, buf, 1024)
        return buf.value.decode()

    def report(self) -> str:
        buf = ctypes.create_string_buffer(65536)
        lib().t0mi_tuner_report(self.handle, buf, 65536)
        return buf.value.decode()
