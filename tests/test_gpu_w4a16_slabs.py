"""GPU parity of the multi-slab W4A16 decode launch (csrc/w4a16_decode.h, RS = 2
to 4): for groups 32..256 t0mi_w4a16_gemm runs the decode kernel over up to four
16-row slabs per launch (group 128; three for groups 32 and 64, two for 256) in
one pass over the weights, spread evenly over the fewest launches.  Every row goes through the
operations of a 16-row launch of its own slab, so the result must be
bit-identical to calling t0mi_w4a16_gemm on each 16-row slab separately where that call
takes the one-slab kernel with one workgroup per 64-column strip (N > 8192 columns, or a
K range one piece cannot take); where N has few enough strips that a 16-row call splits K
over workgroups inside the launch (its pieces summed in another order), the rows agree
within the fp32 reordering bound 2 * K * 2^-24 * sum|a*w| (plus one bf16 ulp for bf16 out);
and within the GEMM tolerance of the oracle (w = (q - z) * s, quant_kernels.rs:24, 95-100).
Cases: 17..191 rows (odd remainders, a trailing one- or two-slab launch), groups
32..256 (256: two chunks per wave, at most two slabs), per-group and constant zero points, f32 and bf16
output, K beyond one workgroup's range (split-K planes of 64 rows + reduce),
and the full decode width N = 11008.
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


def inputs(m, k, n, group, zeros, seed):
    a = oracle.normal_bf16((m, k), seed, 0.0, 1.0)
    w = oracle.pack_qweight(oracle.nibbles((k, n), seed + 1))
    s = oracle.uniform_bf16((k // group, n), seed + 2, 0.005, 0.02)
    z = oracle.pack_qzeros(oracle.nibbles((k // group, n), seed + 3)) if zeros else None
    return a, w, s, z


def call(rt, pa, pw, ps, pz, zp, m, k, n, group, out_bf16):
    ob = 2 if out_bf16 else 4
    dy, py = empty_dev(m * n * ob, fill=0xCD)
    rt.w4a16_gemm(pa, pw, ps, pz, zp, py, m, k, n, group, t0mi.OUT_BF16 if out_bf16 else t0mi.OUT_F32)
    return from_dev(dy, np.uint16 if out_bf16 else np.float32, (m, n))


CASES = [
    # (m, k, n, group, zeros, out_bf16)
    (17, 512, 200, 128, True, True),
    (31, 1024, 520, 64, False, True),
    (32, 4096, 11008, 128, False, True),   # the decode shape with 32 rows
    (33, 256, 136, 32, True, False),       # three slabs, the last one row
    (48, 2048, 1000, 256, True, True),     # group 256: two chunks per wave, two slabs then one
    (64, 8192, 256, 128, False, False),    # K split across workgroups: one four-slab launch, 64-row planes + reduce
    (80, 384, 200, 128, True, True),       # three slabs, then two
    (47, 512, 64, 64, False, True),
    (48, 4096, 2048, 64, True, True),      # three slabs, 8-wave workgroups, no K split
    (96, 4096, 520, 32, False, False),     # two three-slab launches, group 32
    (112, 1024, 520, 128, True, True),     # group 128: four slabs, then three
    (191, 4096, 1000, 128, False, True),   # group 128: three four-slab launches, the last 15 rows
]


@pytest.mark.parametrize("m,k,n,group,zeros,out_bf16", CASES)
def test_multi_slab_launch_equals_16_row_calls(rt, m, k, n, group, zeros, out_bf16):
    a, w, s, z = inputs(m, k, n, group, zeros, 7 * m + k)
    da, pa = to_dev(a)
    dw, pw = to_dev(w)
    ds, ps = to_dev(s)
    pz = 0
    if zeros:
        dz, pz = to_dev(z)
    y = call(rt, pa, pw, ps, pz, 8, m, k, n, group, out_bf16)
    wf = oracle.dequant_qweight_f32(w, s, z, group, 8)
    # A 16-row call splits K inside the launch when 2 pieces per 64-column strip fit the
    # 256 CUs and a piece holds whole groups (the one-slab route's rule, csrc/w4a16.hip).
    split = -(-n // 64) * 2 <= 256 and k // 32 >= 2 * max(4, group // 32)
    bound = None
    if split:
        sab = np.abs(oracle.bf16_to_f32(a)).astype(np.float64) @ np.abs(wf).astype(np.float64)
        bound = 2 * k * 2.0 ** -24 * sab
    for r0 in range(0, m, 16):
        mr = min(16, m - r0)
        ys = call(rt, pa + r0 * k * 2, pw, ps, pz, 8, mr, k, n, group, out_bf16)
        if not split:
            assert np.array_equal(y[r0:r0 + mr], ys), f"rows {r0}..{r0 + mr}: {np.count_nonzero(y[r0:r0 + mr] != ys)} differ"
            continue
        y1 = (oracle.bf16_to_f32(y[r0:r0 + mr]) if out_bf16 else y[r0:r0 + mr]).astype(np.float64)
        y2 = (oracle.bf16_to_f32(ys) if out_bf16 else ys).astype(np.float64)
        lim = bound[r0:r0 + mr] + (2.0 ** -7 * np.abs(y2) if out_bf16 else 0.0)
        assert (np.abs(y1 - y2) <= lim).all(), f"rows {r0}..{r0 + mr}"
    ref = oracle.gemm_bf16(a, oracle.bf16_rne(wf), "nn")
    got = oracle.bf16_to_f32(y) if out_bf16 else y
    assert np.abs(got - ref).max() <= oracle.gemm_tolerance(k, oracle.bf16_to_f32(a), wf)
