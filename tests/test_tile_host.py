"""Host-side contract of the tile_ir surface (no GPU): TileGemm presets, names, LDS
and grid arithmetic, kernarg layouts and tile_auto_select.

Known answers come from the reference's own tests and comments:
  tests/tile_gemm_contract.rs:54-70   (dimension identities, LDS self-consistency)
  tests/tile_gemm_contract.rs:97-118  (build_kernargs_m 44-byte field layout)
  tests/tile_gemm_contract.rs:190-200 (triple-buffer LDS: 40960 / 61440 for 256x64 k32)
  src/t0/tile_ir.rs:245-252           (64x128 k32 with acc_swap: LDS 57344 B)
  src/t0/tile_ir.rs:740-860           (tile_auto_select rules; 4096^3 -> 128x128 k64 -> 64x128 k32)
  src/t0/tile_ir.rs:677-701           (name format)
"""
import struct

import pytest

import t0mi

REF_PRESETS = [
    "tile_128x64_k16", "tile_64x64_k16", "tile_64x64_k32", "tile_64x64_k64", "tile_32x64_k16", "tile_128x64_k32",
    "tile_64x128_k32", "tile_64x128_k16", "tile_128x128_k16", "tile_128x128_k32", "tile_128x128_k48",
    "tile_128x128_k16_swap", "tile_128x128_k32_swap", "tile_256x64_k32_wgp", "tile_256x64_k64_wgp",
    "tile_128x128_k64", "tile_128x64_k64", "tile_32x32_k16", "tile_32x128_k16", "tile_128x32_k16",
    "tile_64x256_k32", "tile_128x256_k32", "tile_256x128_k32", "tile_persistent_decode",
    "tile_persistent_128x64_k32", "tile_persistent_256x128_k32",
]


def test_preset_list_matches_reference():
    assert sorted(t0mi.tile_preset_names()) == sorted(REF_PRESETS)
    with pytest.raises(t0mi.T0miError):
        t0mi.tile_preset("tile_999x1_k16")


@pytest.mark.parametrize("preset,name", [
    ("tile_128x64_k16", "tile_gemm_128x64_k16_db"),
    ("tile_128x128_k32", "tile_gemm_128x128_k32_wgp_swap"),      # double_buffer false, acc_swap true
    ("tile_256x64_k32_wgp", "tile_gemm_256x64_k32_db_wgp"),
    ("tile_persistent_decode", "tile_gemm_32x64_k16_db_mg_persistent"),
    ("tile_persistent_256x128_k32", "tile_gemm_256x128_k32_db_swap_persistent"),
])
def test_names(preset, name):
    assert t0mi.tile_preset(preset).name() == name


def test_name_tags_split_nn_epilogue():
    s = t0mi.tile_preset("tile_64x64_k32").copy(split_k=4, transpose=t0mi.NN)
    s.set_epilogue([t0mi.BIAS_ADD, t0mi.SILU, t0mi.CLAMP])
    assert s.name() == "tile_gemm_64x64_k32_db_sk4_nn_bias_silu_clamp"
    # gfx950 extension only shows when used
    assert s.copy(out_dtype=t0mi.OUT_BF16).name().endswith("_clamp_bf16o")


def test_dimension_identities_and_lds_consistency():
    for p in REF_PRESETS:
        s = t0mi.tile_preset(p)
        nw = s.waves_per_wg or s.tile_m // 32
        assert s.n_waves() == nw and s.wg_size() == nw * 32
        per = (s.tile_m + s.tile_n) * s.tile_k * 2
        gemm_lds = per * 2 if s.double_buffer else per
        rows_per_wave = s.tile_m // nw
        swap = (rows_per_wave // 16) * (s.tile_n // 16 * 8) * 32 * 4 * nw if s.acc_swap else 0
        assert s.lds_total() == gemm_lds + swap + (16 if s.persistent else 0), p


def test_lds_known_answers():
    s = t0mi.tile_preset("tile_256x64_k32_wgp")
    assert s.lds_total() == 40960
    assert s.copy(triple_buffer=1).lds_total() == 61440
    assert t0mi.tile_preset("tile_64x128_k32").lds_total() == 57344
    # the 128x128 family with acc_swap exceeds 64 KB (the reason for the auto-select fallback)
    assert t0mi.tile_preset("tile_128x128_k64").lds_total() > 65536


@pytest.mark.parametrize("m,k,n,want", [
    (4096, 4096, 4096, "tile_64x128_k32"),     # 128x128 k64 -> over 64 KB -> fallback
    (1024, 4096, 4096, "tile_64x128_k32"),
    (4096, 4096, 128, "tile_64x128_k32"),
    (2048, 2048, 2048, "tile_256x64_k32_wgp"),
    (128, 2048, 2048, "tile_64x64_k32"),       # m < 256 in the 2048 class
    (1024, 1024, 1024, "tile_64x64_k32"),
    (512, 512, 512, "tile_64x64_k32"),         # the k64 branch is disabled in the reference
    (256, 256, 256, "tile_64x64_k32"),
    (256, 16, 256, "tile_64x64_k16"),
    (32, 256, 256, "tile_64x256_k32"),         # min_dim < 64, wide N
    (128, 256, 32, "tile_64x64_k32"),          # n = 32 is not narrow (< 32): general rectangular
    (128, 256, 16, "tile_128x32_k16"),         # tall M, narrow N
    (16, 256, 128, "tile_64x64_k32"),          # wide N (>=128) with k32
    (16, 16, 128, "tile_32x128_k16"),
    (16, 16, 16, "tile_32x32_k16"),
    (48, 16, 48, "tile_32x64_k16"),
])
def test_tile_auto_select_rules(m, k, n, want):
    s = t0mi.tile_auto_select(m, k, n, t0mi.NT)
    ref = t0mi.tile_preset(want)
    assert s.name() == ref.name(), (m, k, n)
    assert s.split_k <= 1
    assert t0mi.tile_auto_select(m, k, n, t0mi.NN).transpose == t0mi.NN


def test_build_kernargs_m_field_layout():
    s = t0mi.tile_preset("tile_64x64_k16").copy(split_k=4)
    ka = t0mi.tile_build_kernargs_m(0xA000, 0xB000, 0xC000, 64, 128, 32, s)
    assert len(ka) == 44
    assert struct.unpack_from("<QQQIIIII", ka) == (0xA000, 0xB000, 0xC000, 64, 128, 2, 0, 32)
    ka0 = t0mi.tile_build_kernargs(0xA000, 0xB000, 0xC000, 64, 128, s)
    assert len(ka0) == 44 and struct.unpack_from("<I", ka0, 40)[0] == 0   # M placeholder
    for sk, shift in ((1, 0), (2, 1), (8, 3), (16, 4), (3, 0)):
        ka = t0mi.tile_build_kernargs_m(1, 2, 3, 64, 64, 64, s.copy(split_k=sk))
        assert struct.unpack_from("<I", ka, 32)[0] == shift


def test_persistent_kernargs_64_bytes():
    s = t0mi.tile_preset("tile_persistent_128x64_k32")
    ka = t0mi.tile_build_kernargs_m_with_counter(1, 2, 3, 256, 512, 128, s, 0xD000, 3, 7)
    assert len(ka) == 64
    assert struct.unpack_from("<QII", ka, 48) == (0xD000, 3, 7)
    assert struct.unpack_from("<I", ka, 60)[0] == 7
    assert len(t0mi.tile_build_kernargs_m(1, 2, 3, 256, 512, 128, s)) == 64
    assert s.kernarg_size() == 64


@pytest.mark.parametrize("ops,size,offs", [
    ([], 44, {}),
    ([t0mi.BIAS_ADD], 56, {"bias": 48}),
    ([t0mi.SCALE], 48, {"scale": 44}),
    ([t0mi.BIAS_ADD, t0mi.SCALE, t0mi.CLAMP], 68, {"bias": 48, "scale": 56, "lo": 60, "hi": 64}),
    ([t0mi.CLAMP, t0mi.RELU], 52, {"lo": 44, "hi": 48}),
    ([t0mi.SILU, t0mi.GELU, t0mi.ABS, t0mi.NEG], 44, {}),
])
def test_epilogue_kernarg_layout(ops, size, offs):
    s = t0mi.tile_preset("tile_64x64_k32").copy(epilogue=ops)
    assert s.kernarg_size() == size
    ka = t0mi.tile_build_kernargs_m(1, 2, 3, 64, 64, 64, s)
    full = t0mi.tile_append_epilogue_args(s, ka, bias=0xBEEF0, scale=0.5, clamp_min=-1.0, clamp_max=2.0)
    assert len(full) == size
    if "bias" in offs:
        assert struct.unpack_from("<Q", full, offs["bias"])[0] == 0xBEEF0
    if "scale" in offs:
        assert struct.unpack_from("<f", full, offs["scale"])[0] == 0.5
    if "lo" in offs:
        assert struct.unpack_from("<ff", full, offs["lo"]) == (-1.0, 2.0)
        assert offs["hi"] == offs["lo"] + 4


def test_epilogue_args_after_persistent_base():
    s = t0mi.tile_preset("tile_persistent_decode").copy(epilogue=[t0mi.BIAS_ADD, t0mi.SCALE])
    assert s.kernarg_size() == 64 + 8 + 4
    ka = t0mi.tile_build_kernargs_m_with_counter(1, 2, 3, 64, 64, 64, s, 0, 0, 0)
    full = t0mi.tile_append_epilogue_args(s, ka, bias=0x1000, scale=2.0)
    assert struct.unpack_from("<Qf", full, 64) == (0x1000, 2.0)
    with pytest.raises(t0mi.T0miError):
        t0mi.tile_append_epilogue_args(s, ka[:44], bias=0x1000)


def test_compute_grid():
    s = t0mi.tile_preset("tile_128x64_k16")
    assert t0mi.tile_compute_grid(s, 4096, 4096) == (64 * 128, 32, 1)
    mg = s.copy(swap_grid=0, split_k=2)
    assert t0mi.tile_compute_grid(mg, 4096, 4096) == (32 * 128, 64 * 2, 1)
    for m in (1, 31, 127, 128, 129, 4095):
        for n in (1, 63, 64, 65, 4096):
            gx, gy, gz = t0mi.tile_compute_grid(s, m, n)
            assert gx % s.wg_size() == 0 and gz == 1
            assert (gx // s.wg_size()) * s.tile_n >= n and gy * s.tile_m >= m
    p = t0mi.tile_preset("tile_persistent_256x128_k32")
    assert t0mi.tile_compute_grid(p, 4096, 4096) == (p.wg_size(), 1, 1)


def test_kernel_get_errors_null_runtime():
    rt = t0mi.Runtime(null=True)
    try:
        # tile_128x128_k48 (tile_ir.rs:316) runs as three 16-K steps of the 128x128x16 kernel, and
        # NN tiles narrower than 64 columns on the 64-column NN kernel: same names and kernargs.
        k48 = rt.tile_kernel(t0mi.tile_preset("tile_128x128_k48"))
        assert k48.name == "tile_gemm_128x128_k48_db"
        rt.tile_kernel(t0mi.tile_preset("tile_32x32_k16").copy(transpose=t0mi.NN))
        bad = t0mi.tile_preset("tile_64x64_k32").copy(wmma_format=3)
        with pytest.raises(t0mi.T0miError):
            rt.tile_kernel(bad)
        with pytest.raises(t0mi.T0miError) as e:
            rt.tile_kernel(t0mi.tile_preset("tile_64x64_k32").copy(tile_m=512))
        assert e.value.code == -2  # T0MI_ERR_NO_KERNEL: no kernel covers a 512-row tile
        for p in REF_PRESETS:
            k = rt.tile_kernel(t0mi.tile_preset(p))
            a = k.attrs()
            assert a["kernarg_size"] == (64 if "persistent" in p else 44)
            assert a["wg_size"] == t0mi.tile_preset(p).wg_size()
            assert k.name == t0mi.tile_preset(p).name()
    finally:
        rt.close()


def test_null_dispatch_records_tile_kernargs():
    rt = t0mi.Runtime(null=True)
    try:
        s = t0mi.tile_preset("tile_64x64_k32").copy(epilogue=[t0mi.BIAS_ADD])
        k = rt.tile_kernel(s)
        ka = t0mi.tile_append_epilogue_args(s, t0mi.tile_build_kernargs_m(16, 32, 48, 64, 64, 64, s), bias=64)
        grid = t0mi.tile_compute_grid(s, 64, 64)
        assert rt.dispatch(k, grid, ka) == 0
        g, rec = rt.last_dispatch()
        assert g == grid and rec == ka
        assert rt.dispatch(k, grid, ka[:44]) == -5   # kernarg length mismatch
        short_grid = (s.wg_size(), 0, 1)
        assert rt.dispatch(k, short_grid, t0mi.tile_append_epilogue_args(
            s, t0mi.tile_build_kernargs_m(16, 32, 48, 64, 128, 64, s), bias=64)) == -1  # grid misses N
    finally:
        rt.close()
