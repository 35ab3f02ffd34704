"""CPU tests of libt0mi's C ABI: symbol exports, the host-side contracts restated
from the reference (configs, names, grids, kernargs, selection, tuner cache) and
the runtime's control path on the null backend (no compute, no GPU)."""
import json
import os
import re

import pytest

import t0mi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "t0mi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(t0mi_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = t0mi.lib()
    names = header_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in include/t0mi.h but not exported: {missing}"
    assert set(names) == set(t0mi.SIGNATURES), "binding and header disagree"
    assert L.t0mi_build_target() == b"gfx950"
    assert L.t0mi_abi_version() == 1


def test_integration_rust_binding_covers_the_header():
    """INTEGRATION.md's Rust `extern "C"` block declares every function of include/t0mi.h
    exactly once, with as many parameters as the C declaration."""
    text = open(os.path.join(ROOT, "include", "t0mi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    c_params = {}
    for name, params in re.findall(r"\b(t0mi_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", text):
        ps = [p for p in " ".join(params.split()).split(",") if p.strip() and p.strip() != "void"]
        c_params[name] = len(ps)
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = doc[doc.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    rust = re.findall(r"pub fn (t0mi_[a-z0-9_]+)\(([^)]*)\)", block, flags=re.S)
    names = [n for n, _ in rust]
    assert len(names) == len(set(names)), "a function declared twice"
    assert set(names) == set(c_params), (sorted(set(c_params) - set(names)), sorted(set(names) - set(c_params)))
    for name, params in rust:
        n = len([p for p in params.split(",") if p.strip()])
        assert n == c_params[name], (name, n, c_params[name])


def test_library_has_no_oracle_dependency():
    """The product must not link or embed the CPU oracle."""
    blob = open(t0mi.LIB_PATH, "rb").read()
    assert b"orc_gemm" not in blob and b"liboracle" not in blob


# ------------------------------------------------------------- configs ----

def test_reference_preset_names_unchanged():
    """GemmConfig::name (gemm_gen.rs:215-235) is the kernel cache key: reference
    presets keep their reference names."""
    c = t0mi.preset("tile_32x64_k16")
    assert c.name() == "t0_gemm_32x64_k16_ldsdb_wgp"
    assert t0mi.preset("tile_32x64_direct").name() == "t0_gemm_32x64_k16_direct_wgp"
    assert t0mi.preset("tile_128x128_2pass").name() == "t0_gemm_128x64_k16_ldsdb_2p_wgp"
    # epilogue tags (gemm_gen.rs:612-624)
    assert c.copy(epilogue=t0mi.EPI_BIAS_ADD).name().endswith("_bias")
    assert c.copy(epilogue=t0mi.EPI_BIAS_ADD_RELU).name().endswith("_bias_relu")
    assert "_sk4" in c.copy(split_k=4).name()
    assert "_mg" in c.copy(swap_grid=0).name()
    assert "_nn" in c.copy(transpose=t0mi.NN).name()
    # gfx950 extensions only appear when used
    assert c.copy(out_dtype=t0mi.OUT_BF16).name().endswith("_bf16o")
    assert t0mi.preset("gfx950_256x256_k64_w2x4").name() == "t0_gemm_256x256_k64_ldsdb_w2x4"


def test_feasibility_gfx950():
    # Every reference preset runs, including the wave32 tile_16x64_k16 (wg 32, 16 rows) that
    # bf16_matmul.rs:140-149 selects for m <= 16: it keeps its name, grid and kernargs and runs
    # on the 32x64 kernel that covers its tile.
    for n in t0mi.preset_names():
        assert t0mi.preset(n).is_feasible(), n
    small = t0mi.preset("tile_16x64_k16")
    assert small.name() == "t0_gemm_16x64_k16_ldsdb_wgp"
    assert t0mi.compute_grid_auto(small, 17, 100) == (2 * 32, 2), "work-items: 2 column tiles x wg 32, 2 row tiles"
    big = t0mi.preset("gfx950_256x256_k64_w2x4")
    assert t0mi.lds_total(big) == 2 * (256 + 256) * 64 * 2 <= 160 * 1024
    assert not big.copy(tile_k=48).is_feasible()
    assert not big.copy(split_k=3).is_feasible()
    assert not big.copy(wave_m=3, wave_n=3).is_feasible()
    with pytest.raises(t0mi.T0miError):
        t0mi.preset("no_such_preset")


def test_grid_coverage_enumeration():
    """tests/tile_gemm_contract.rs:73-93: grid_x multiple of wg, tiles cover M and N."""
    dims = [1, 31, 32, 33, 63, 64, 127, 128, 255, 256, 4095, 4096]
    for name in ("tile_128x64_k16", "tile_128x64_k32", "tile_64x64_k32", "gfx950_256x256_k64_w2x4"):
        cfg = t0mi.preset(name)
        for m in dims:
            for n in dims:
                gx, gy = t0mi.compute_grid_auto(cfg, m, n)
                assert gx % cfg.wg_size == 0
                tiles_m = -(-m // cfg.tile_m)
                tiles_n = -(-n // cfg.tile_n)
                assert gy == tiles_m and gx // cfg.wg_size == tiles_n
        mg = cfg.copy(swap_grid=0)
        gx, gy = t0mi.compute_grid(mg, 300, 70)
        assert gx == -(-300 // cfg.tile_m) * cfg.wg_size and gy == -(-70 // cfg.tile_n)
    cfg = t0mi.preset("tile_64x64_k32").copy(split_k=4)
    assert t0mi.compute_grid_auto(cfg, 256, 128) == (2 * 64, 4 * 4)
    with pytest.raises(t0mi.T0miError):
        t0mi.compute_grid_split_k(cfg, 64, 64, 3)


def test_kernarg_layouts():
    """gemm_gen.rs:439-484 and tests/tile_gemm_contract.rs:119-131."""
    rd64 = lambda b, o: int.from_bytes(b[o:o + 8], "little")
    rd32 = lambda b, o: int.from_bytes(b[o:o + 4], "little")
    no_sk = t0mi.preset("tile_128x64_k16")
    ka = t0mi.build_kernargs(1, 2, 3, 64, 64, 64, no_sk)
    assert len(ka) == 40 and rd32(ka, 36) == 0
    assert (rd64(ka, 0), rd64(ka, 8), rd64(ka, 16), rd32(ka, 24), rd32(ka, 28), rd32(ka, 32)) == (1, 2, 3, 64, 64, 0)
    sk2 = no_sk.copy(split_k=2)
    ka2 = t0mi.build_kernargs(1, 2, 3, 64, 64, 256, sk2)
    assert rd32(ka2, 36) == 256 * 64 * 4, "split_k > 1: y_split_stride = M*N*4"
    kb = t0mi.build_kernargs_with_bias(0x1000, 0x2000, 0x3000, 64, 64, 128, t0mi.preset("tile_32x64_k16"), 0x4000)
    assert len(kb) == 48 and rd64(kb, 40) == 0x4000


def test_auto_select_domain_sample_feasible_and_prebuilt():
    """tests/tile_gemm_contract.rs:166-180 + gemm_gen.rs:576-601."""
    n_checked = 0
    for m in (16, 31, 64, 128, 256, 1024, 4096):
        for n in (32, 64, 128, 256, 4096):
            for k in (16, 32, 64, 256, 4096):
                c = t0mi.auto_select(m, k, n)
                assert c.is_feasible(), (m, k, n, c.name())
                rt = t0mi.Runtime(null=True)
                rt.kernel(c)  # a prebuilt kernel exists for every auto_select result
                n_checked += 1
    assert n_checked >= 100
    assert t0mi.auto_select(1024, 1024, 1024).tile_m >= 64
    assert t0mi.auto_select(8192, 8192, 8192).tile_m >= 64
    assert 128 % t0mi.auto_select(128, 4096, 4096).tile_m == 0
    big = t0mi.auto_select(4096, 4096, 4096)
    assert (big.tile_m, big.tile_n) == (256, 256), big.name()


def test_auto_schedule_gemm_ranking():
    """cost_model.rs:464-534: feasible configs best first; the head is auto_select's pick for the
    layout; every entry has a prebuilt kernel; cap bounds what is written, not the count."""
    for (m, n, k) in ((128, 4096, 4096), (4096, 4096, 4096), (16, 11008, 4096), (100, 200, 64)):
        for tr in (t0mi.NT, t0mi.NN):
            ranked = t0mi.auto_schedule_gemm(m, n, k, tr, t0mi.OUT_BF16, cap=256)
            assert ranked, (m, n, k, tr)
            est = [e for _, e in ranked]
            assert est == sorted(est) and all(e > 0 for e in est)
            pick = t0mi.auto_select_layout(m, k, n, tr, t0mi.OUT_BF16)
            assert ranked[0][0].name() == pick.name()
            rt = t0mi.Runtime(null=True)
            for c, _ in ranked:
                assert c.is_feasible() and c.transpose == tr
                rt.kernel(c)
            short = t0mi.auto_schedule_gemm(m, n, k, tr, t0mi.OUT_BF16, cap=3)
            assert [c.name() for c, _ in short] == [c.name() for c, _ in ranked[:3]]
    with pytest.raises(t0mi.T0miError):
        t0mi.auto_schedule_gemm(0, 64, 64)


def test_auto_gemm_plan_column_split():
    """The column split of the library's auto-scheduled GEMMs: the head is the ranking's first
    entry; a split only where the head's tiles fill whole rounds of the GPU (256 CUs x the tile's
    workgroups per CU) and part of one more, after the most whole columns of tiles that fit in
    the whole rounds; the tail is the ranking's head for the remaining columns."""
    cases = {  # (m, n, k, layout) -> the first column of the tail (n: no split)
        (4096, 14336, 4096, t0mi.NN): 12288,     # BASELINE config 5's GEMM: 896 tiles = 3.5 rounds
        (1536, 11008, 4096, t0mi.NN): 10752,     # 258 tiles: 252 of them fill one round
        (2048, 14336, 4096, t0mi.NN): 14336,     # 448 tiles, last round 75 % full: one launch
        (3072, 14336, 4096, t0mi.NN): 14336,     # 672 tiles: two whole rounds, last 62.5 % full
        (4096, 4352, 1024, t0mi.NT): 4096,
        (4096, 4096, 4096, t0mi.NN): 4096,       # whole rounds: nothing to split
        (4096, 11008, 4096, t0mi.NN): 11008,     # last round 69 % full: the model keeps one launch
        (768, 11008, 4096, t0mi.NN): 11008,      # under one round
        (128, 4096, 4096, t0mi.NN): 4096,        # split-K head: never split
    }
    for (m, n, k, tr), want in cases.items():
        head, n1, tail = t0mi.auto_gemm_plan(m, n, k, tr, t0mi.OUT_BF16)
        ranked = t0mi.auto_schedule_gemm(m, n, k, tr, t0mi.OUT_BF16, cap=1)
        assert head.name() == ranked[0][0].name()
        assert n1 == want, ((m, n, k, tr), n1)
        if n1 == n:
            assert tail.name() == head.name()
            continue
        tm, tn = -(-m // head.tile_m), -(-n // head.tile_n)
        whole = (tm * tn // 256) * 256  # tiles of the whole rounds
        assert n1 % head.tile_n == 0 and whole - tm < tm * (n1 // head.tile_n) <= whole
        assert tail.name() == t0mi.auto_schedule_gemm(m, n - n1, k, tr, t0mi.OUT_BF16, cap=1)[0][0].name()
    with pytest.raises(t0mi.T0miError):
        t0mi.auto_gemm_plan(0, 64, 64)


def test_auto_select_legacy():
    """gemm_gen.rs:636-646: small squares use split-K with tile_m 64; 1024^3 uses tile_m 128."""
    c = t0mi.auto_select_legacy(256, 256, 256)
    assert c.split_k > 1 and c.tile_m == 64
    assert t0mi.auto_select_legacy(1024, 1024, 1024).tile_m == 128
    for args in ((4096, 4096, 4096), (128, 4096, 4096), (7, 100, 9)):
        assert t0mi.auto_select_legacy(*args).is_feasible()


def test_cached_auto_select():
    """src/t0/prefill_spec_cache.rs:142-218: cache hits return the same config."""
    L = t0mi.lib()
    L.t0mi_clear_spec_cache()
    assert L.t0mi_spec_cache_len() == 0
    a = t0mi.cached_auto_select(512, 4096, 1024)
    b = t0mi.cached_auto_select(512, 4096, 1024)
    assert a.name() == b.name() == t0mi.auto_select(512, 4096, 1024).name()
    assert L.t0mi_spec_cache_len() == 1
    t0mi.cached_auto_select(16, 4096, 4096)
    assert L.t0mi_spec_cache_len() == 2
    L.t0mi_clear_spec_cache()
    assert L.t0mi_spec_cache_len() == 0


# ------------------------------------------------------ runtime control ----

def test_null_runtime_dispatch_contract():
    """gpu_context.rs:305-357: kernarg length must match; dispatch records grid and bytes."""
    rt = t0mi.Runtime(null=True)
    cfg = t0mi.preset("tile_64x64_k32")
    k = rt.kernel(cfg)
    assert k.attrs() == {"lds_size": 2 * (64 + 64) * 32 * 2, "wg_size": 64, "kernarg_size": 40}
    assert k.name == cfg.name()
    assert rt.kernel(cfg).handle.value == k.handle.value, "kernels are cached by name"
    kb = rt.kernel(cfg.copy(epilogue=t0mi.EPI_BIAS_ADD))
    assert kb.attrs()["kernarg_size"] == 48
    ka = t0mi.build_kernargs(0x1000, 0x2000, 0x3000, 128, 128, 128, cfg)
    grid = t0mi.compute_grid_auto(cfg, 128, 128)
    assert rt.dispatch(k, grid, ka[:36]) == t0mi.ERR_KERNARG
    assert "kernarg mismatch" in t0mi.last_error()
    assert rt.dispatch(k, grid, ka) == t0mi.OK
    g, got = rt.last_dispatch()
    assert g == (grid[0], grid[1], 1) and got == ka
    assert rt.dispatch(k, (grid[0] + 1, grid[1]), ka) == t0mi.ERR_INVALID  # not a multiple of wg
    small = rt.kernel(t0mi.preset("tile_16x64_k16"))
    assert small.name == "t0_gemm_16x64_k16_ldsdb_wgp"
    assert small.attrs()["wg_size"] == 32 and small.attrs()["kernarg_size"] == 40
    with pytest.raises(t0mi.T0miError):
        rt.kernel(t0mi.preset("tile_16x64_k16").copy(wg_size=48))


def test_null_runtime_timeout_poisons():
    """aql.rs:509-545 + gpu_context.rs:311-313, 352-355: a timed-out wait poisons the
    runtime and every later dispatch is refused."""
    rt = t0mi.Runtime(null=True)
    cfg = t0mi.preset("tile_64x64_k32")
    k = rt.kernel(cfg)
    ka = t0mi.build_kernargs(0x1000, 0x2000, 0x3000, 64, 64, 64, cfg)
    grid = t0mi.compute_grid_auto(cfg, 64, 64)
    assert not rt.is_poisoned()
    rt.inject_timeout()
    assert rt.dispatch(k, grid, ka) == t0mi.ERR_TIMEOUT
    assert rt.is_poisoned()
    assert rt.dispatch(k, grid, ka) == t0mi.ERR_POISONED
    assert rt.wait_idle() == t0mi.ERR_POISONED
    with pytest.raises(t0mi.T0miError) as e:
        rt.gemm(cfg, 0x1000, 0x2000, 0x3000, 64, 64, 64)
    assert e.value.code == t0mi.ERR_POISONED


def test_gemm_argument_validation():
    rt = t0mi.Runtime(null=True)
    cfg = t0mi.preset("gfx950_128x128_k64_w2x2")
    with pytest.raises(t0mi.T0miError):
        rt.gemm(cfg, 0x1000, 0x2000, 0x3000, 64, 64, 100)   # K % 8
    with pytest.raises(t0mi.T0miError):
        rt.gemm(cfg, 0x1000, 0x2000, 0x3000, 64, 60, 64)    # N % 8
    with pytest.raises(t0mi.T0miError):
        rt.gemm(cfg, 0x1008, 0x2000, 0x3000, 64, 64, 64)    # alignment
    with pytest.raises(t0mi.T0miError):
        rt.gemm(cfg.copy(epilogue=t0mi.EPI_BIAS_ADD), 0x1000, 0x2000, 0x3000, 64, 64, 64)  # null bias
    rt.gemm(cfg, 0x1000, 0x2000, 0x3000, 64, 64, 64)  # valid: null backend computes nothing
    # the no-allocation variant: same checks, plus the scratch limit (checked before any launch)
    text = open(os.path.join(ROOT, "include", "t0mi.h")).read()
    assert "#define T0MI_NOALLOC_SCRATCH_BYTES (32u << 20)" in text and t0mi.NOALLOC_SCRATCH_BYTES == 32 << 20
    sk4 = cfg.copy(split_k=4)
    rt.gemm_noalloc(sk4, 0x1000, 0x2000, 0x3000, 512, 4096, 256)  # 4 planes of 8 MiB: fits exactly
    for m, n, k, c in ((513, 4096, 256, sk4), (4096, 4096, 0, cfg)):  # one row more; K = 0 zero plane of 64 MiB
        with pytest.raises(t0mi.T0miError) as e:
            rt.gemm_noalloc(c, 0x1000, 0x2000, 0x3000, m, n, k)
        assert e.value.code == t0mi.ERR_INVALID and "scratch" in str(e.value)
    with pytest.raises(t0mi.T0miError):
        rt.gemm_noalloc(cfg, 0x1000, 0x2000, 0x3000, 64, 64, 100)  # K % 8, as t0mi_gemm
    # W4A16 alignment contract: A, qweight and Y 16-byte, scales 8-byte, qzeros 4-byte
    # (checked before the null backend returns).
    w4 = t0mi.Runtime(null=True)
    w4.w4a16_gemm(0x1000, 0x2000, 0x3000, 0x4000, 8, 0x5000, 16, 4096, 11008, 128)
    for bad in ((0x1008, 0x2000, 0x3000, 0x4000, 0x5000), (0x1000, 0x2000, 0x3000, 0x4000, 0x5008),
                (0x1000, 0x2000, 0x3004, 0x4000, 0x5000), (0x1000, 0x2000, 0x3000, 0x4002, 0x5000)):
        a_, w_, s_, z_, y_ = bad
        with pytest.raises(t0mi.T0miError) as e:
            w4.w4a16_gemm(a_, w_, s_, z_, 8, y_, 16, 4096, 11008, 128)
        assert e.value.code == t0mi.ERR_INVALID and "aligned" in str(e.value)
    with pytest.raises(t0mi.T0miError) as e:
        t0mi.Runtime(null=True).w4a16_gemm(0x1000, 0x2000, 0x3000, 0, 16, 0x4000, 16, 4096, 11008, 128)
    assert e.value.code == t0mi.ERR_INVALID  # zp_const outside 0..15


# --------------------------------------------------------------- tuner ----

def test_tuner_cache_roundtrip(tmp_path):
    """GemmTuner disk cache (auto_gemm.rs:435-501): a JSON entry is served without a
    device; corrupt or stale entries are ignored (the tuner then needs a device)."""
    tuner = t0mi.GemmTuner(str(tmp_path))
    p = tuner.cache_path(4096, 4096, 4096)
    assert p.endswith("gemm_4096x4096x4096.json")
    assert tuner.cache_path(4096, 4096, 4096, t0mi.NN, t0mi.OUT_BF16).endswith("gemm_4096x4096x4096_nn_bf16o.json")
    rt = t0mi.Runtime(null=True)
    with pytest.raises(t0mi.T0miError) as e:
        tuner.tune(rt, 4096, 4096, 4096)
    assert e.value.code == t0mi.ERR_NO_DEVICE
    # reference-format JSON (auto_gemm.rs:478-492) plus the gfx950 wave fields
    entry = {"tile_m": 256, "tile_n": 256, "tile_k": 64, "wg_size": 512, "split_k": 1, "lds_pad": 0,
             "n_col_passes": 1, "wgp": False, "swap": True, "wave_m": 2, "wave_n": 4, "tflops": 1234.5,
             "all": [["t0_gemm_256x256_k64_ldsdb_w2x4", 1234.5]]}
    with open(p, "w") as f:
        f.write(json.dumps(entry, separators=(",", ":")))
    cfg, tf, cached = tuner.tune(rt, 4096, 4096, 4096)
    assert cached and tf == pytest.approx(1234.5) and cfg.name() == "t0_gemm_256x256_k64_ldsdb_w2x4"
    assert "4096x4096x4096" in tuner.report()
    # a second tuner on the same directory reads the same file
    cfg2, _, cached2 = t0mi.GemmTuner(str(tmp_path)).tune(rt, 4096, 4096, 4096)
    assert cached2 and cfg2.name() == cfg.name()
    # corrupt cache -> ignored (needs a device to re-tune)
    p2 = tuner.cache_path(512, 512, 512)
    with open(p2, "w") as f:
        f.write('{"tile_m":12')
    with pytest.raises(t0mi.T0miError):
        tuner.tune(rt, 512, 512, 512)
    # stale entry naming a kernel that is not prebuilt -> ignored
    p3 = tuner.cache_path(1024, 1024, 1024)
    with open(p3, "w") as f:
        f.write(json.dumps(dict(entry, tile_m=96)))
    with pytest.raises(t0mi.T0miError):
        tuner.tune(rt, 1024, 1024, 1024)
    tuner.invalidate(4096, 4096, 4096)
    assert not os.path.exists(p)
    tuner.clear()
    assert not os.path.exists(p2)
