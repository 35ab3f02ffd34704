"""GPU tests of the column split of the library's auto-scheduled GEMMs (t0mi_auto_gemm_plan):
where the ranking's head tile leaves a partly filled last round, the calls that schedule their own
GEMM (the Ignis matmul callers, the dequant-once W4A16 route) run the head over the columns of
the whole rounds and a second launch, with its own tile and split, over the rest.

Bars: with an unsplit tail every output element sums its K products in the same ascending order
as one launch of the head over all columns, so the split result is bit-identical to that launch
(t0mi_gemm with the head config); with a split-K tail the head's columns stay bit-identical and
the tail's columns are within the GEMM tolerance of the oracle; the guard bytes after Y are
untouched (the second launch writes inside the first launch's row length).
"""
import numpy as np
import pytest

import oracle
import t0mi
from gpu_helpers import empty_dev, from_dev, runtime, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


def rand_f32(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def check_close(y, ref, a_bf, b_bf, k, rel_max=1e-5):
    tol = oracle.gemm_tolerance(k, oracle.bf16_to_f32(a_bf), oracle.bf16_to_f32(b_bf))
    err, rel = oracle.compare(y, ref)
    assert err <= tol, (err, tol)
    assert rel < rel_max, rel


@pytest.mark.parametrize("m,k,n", [(4096, 1024, 4352), (2304, 1024, 7424)])
def test_matmul_wt_bf16_split_bit_identical_to_one_launch(rt, m, k, n):
    """matmul_with_wt_bf16 (bf16_matmul.rs:99-134) at shapes whose plan splits the columns with
    an unsplit tail: the same bits as the head config over all columns in one launch."""
    head, n1, tail = t0mi.auto_gemm_plan(m, n, k, t0mi.NT, t0mi.OUT_F32)
    assert n1 < n and tail.split_k in (0, 1), (head.name(), n1, tail.name())
    x = rand_f32((m, k), 0xA1)
    wt = oracle.bf16_rne(rand_f32((n, k), 0xA2))
    dx, px = to_dev(x)
    dwt, pwt = to_dev(wt)
    dy, py = empty_dev(m * n * 4, fill=0xCD)
    print(f"[auto split] wt_bf16 {m}x{k}x{n}: {head.name()} to column {n1}, then {tail.name()}", flush=True)
    rt.matmul_with_wt_bf16(px, pwt, py, m, k, n)
    y = from_dev(dy, np.float32, (m, n))
    xb = oracle.bf16_rne(x)
    dxb, pxb = to_dev(xb)
    dy1, py1 = empty_dev(m * n * 4, fill=0xAB)
    rt.gemm(head.copy(transpose=t0mi.NT, out_dtype=t0mi.OUT_F32), pxb, pwt, py1, m, n, k)
    y1 = from_dev(dy1, np.float32, (m, n))
    assert np.array_equal(y.view(np.uint32), y1.view(np.uint32)), f"{np.count_nonzero(y != y1)} elements differ"
    # and the oracle, on rows that cross both launches' columns
    rows = slice(m - 48, m)
    check_close(y[rows], oracle.gemm_bf16(xb[rows], wt, "nt", nthreads=8), xb[rows], wt, k)


def test_w4a16_two_pass_split_k_tail(rt):
    """The dequant-once W4A16 route (1536 rows) at a shape whose plan gives the tail columns a
    split-K tile: the head's columns bit-identical to dequant + one launch of the head config,
    the tail's columns within the GEMM tolerance of the oracle."""
    m, k, n, group = 1536, 2048, 11008, 128
    head, n1, tail = t0mi.auto_gemm_plan(m, n, k, t0mi.NN, t0mi.OUT_BF16)
    assert n1 < n and tail.split_k > 1, (head.name(), n1, tail.name())
    a = oracle.normal_bf16((m, k), 0xB1, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), 0xB2))
    s = oracle.uniform_bf16((k // group, n), 0xB3, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), 0xB4))
    bufs = [to_dev(v) for v in (a, w, s, z)]
    (_, pa), (_, pw), (_, ps), (_, pz) = bufs
    dy, py = empty_dev(m * n * 2, fill=0xCD)
    print(f"[auto split] w4a16 {m}x{k}x{n} g{group}: {head.name()} to column {n1}, then {tail.name()}", flush=True)
    rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_BF16)
    y = from_dev(dy, np.uint16, (m, n))
    dwb, pwb = empty_dev(k * n * 2)
    rt.dequant_int4(pw, ps, pz, 0, pwb, k, n, group, 2)
    dy1, py1 = empty_dev(m * n * 2, fill=0xAB)
    rt.gemm(head.copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16), pa, pwb, py1, m, n, k)
    y1 = from_dev(dy1, np.uint16, (m, n))
    assert np.array_equal(y[:, :n1], y1[:, :n1]), f"{np.count_nonzero(y[:, :n1] != y1[:, :n1])} elements differ"
    wb = oracle.bf16_rne(oracle.dequant_qweight_f32(w, s, z, group, 0))
    cols = slice(n1, n)
    ref = oracle.gemm_bf16(a, np.ascontiguousarray(wb[:, cols]), "nn", nthreads=8)
    # bf16 output: each element rounded once more (relative 2^-9 at most)
    check_close(oracle.bf16_to_f32(y[:, cols]), ref, a, wb[:, cols], k, rel_max=3e-3)


def test_w4a16_fused_size_takes_split_plan(rt):
    """1280 rows (under the dequant-once threshold of 1536): the fused ping-pong kernel's 280
    tiles of 256 x 256 would overflow one round, and the dense GEMM's plan splits the columns,
    so the call runs dequant-once with that plan: bit-identical to dequant + one launch of the
    head config (the tail is unsplit), and within the GEMM tolerance of the fused route that a
    zero workspace limit forces (a different K split for the same sums)."""
    m, k, n, group = 1280, 1024, 14336, 128
    head, n1, tail = t0mi.auto_gemm_plan(m, n, k, t0mi.NN, t0mi.OUT_BF16)
    assert n1 < n and tail.split_k in (0, 1), (head.name(), n1, tail.name())
    a = oracle.normal_bf16((m, k), 0xC1, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), 0xC2))
    s = oracle.uniform_bf16((k // group, n), 0xC3, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), 0xC4))
    bufs = [to_dev(v) for v in (a, w, s, z)]
    (_, pa), (_, pw), (_, ps), (_, pz) = bufs
    print(f"[auto split] w4a16 {m}x{k}x{n} g{group}: {head.name()} to column {n1}, then {tail.name()}", flush=True)
    outs = []
    for limit in (2**64 - 1, 0):
        rt.set_w4a16_workspace_limit(limit)
        dy, py = empty_dev(m * n * 2, fill=0xCD)
        rt.w4a16_gemm(pa, pw, ps, pz, 0, py, m, k, n, group, t0mi.OUT_BF16)
        outs.append(from_dev(dy, np.uint16, (m, n)))
    rt.set_w4a16_workspace_limit(2**64 - 1)
    y, y_fused = outs
    dwb, pwb = empty_dev(k * n * 2)
    rt.dequant_int4(pw, ps, pz, 0, pwb, k, n, group, 2)
    dy1, py1 = empty_dev(m * n * 2, fill=0xAB)
    rt.gemm(head.copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16), pa, pwb, py1, m, n, k)
    y1 = from_dev(dy1, np.uint16, (m, n))
    assert np.array_equal(y, y1), f"{np.count_nonzero(y != y1)} elements differ"
    wb = oracle.bf16_rne(oracle.dequant_qweight_f32(w, s, z, group, 0))
    rows = slice(m - 32, m)
    ref = oracle.gemm_bf16(np.ascontiguousarray(a[rows]), wb, "nn", nthreads=8)
    for out in (y, y_fused):
        check_close(oracle.bf16_to_f32(out[rows]), ref, a[rows], wb, k, rel_max=3e-3)
