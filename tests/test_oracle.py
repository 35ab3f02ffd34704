"""Pins of the CPU oracle against the reference's own known answers, golden
vectors and closed forms (no GPU).  Each check names what it would catch."""
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden", "torch_ref")


# --------------------------------------------------------------- bf16 -----

def test_bf16_truncation_known_answers():
    """tests/tile_gemm_contract.rs:137-154 (reference): truncation semantics."""
    f = lambda v: int(oracle.bf16_trunc(np.array([v], np.float32))[0])
    assert f(1.0) == 0x3F80
    assert f(-1.0) == 0xBF80
    assert f(0.0) == 0
    assert f(np.inf) == 0x7F80
    assert f(-np.inf) == 0xFF80
    slightly_over = np.array([0x3F8000FF], np.uint32).view(np.float32)[0]  # 1 + 2^-9-ish
    assert f(slightly_over) == 0x3F80, "truncation drops the low mantissa bits"
    nan = np.float32(np.nan)
    assert f(nan) == (int(np.array([nan]).view(np.uint32)[0]) >> 16)
    for bits in (0x3F80, 0xBF80, 0x007F, 0x8000):
        assert f(oracle.bf16_to_f32(np.array([bits], np.uint16))[0]) == bits, "round trip is idempotent"


def test_bf16_rne_closed_form():
    """Round-to-nearest-even (src/ignis/ops/bf16_matmul.rs:372): ties go to even,
    above-half rounds up, below-half rounds down; NaN stays NaN (added handling)."""
    u = lambda b: np.array([b], np.uint32).view(np.float32)
    r = lambda b: int(oracle.bf16_rne(u(b))[0])
    assert r(0x3F808000) == 0x3F80  # exact tie, even stays
    assert r(0x3F818000) == 0x3F82  # exact tie, odd rounds up to even
    assert r(0x3F808001) == 0x3F81  # just above half
    assert r(0x3F807FFF) == 0x3F80  # just below half
    assert r(0xBF818000) == 0xBF82  # sign symmetric
    assert r(0x7F7FFFFF) == 0x7F80  # overflow to inf
    assert r(0x7F800001) & 0x7FC0 == 0x7FC0  # NaN with low payload stays a (quiet) NaN
    # against an independent float64 nearest-even rounding on random values
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(37.0)
    got = oracle.bf16_to_f32(oracle.bf16_rne(x)).astype(np.float64)
    # bf16 keeps 8 significant bits: ulp = 2^(e-8) for x = m * 2^e, m in [0.5, 1)
    _, e = np.frexp(x.astype(np.float64))
    bf_ulp = np.ldexp(1.0, e - 8)
    err = np.abs(got - x.astype(np.float64))
    assert np.all(err <= bf_ulp / 2)
    # and it is the nearest of the two bf16 neighbours (truncation and truncation + 1 ulp)
    lo = oracle.bf16_to_f32(oracle.bf16_trunc(x)).astype(np.float64)
    hi = lo + np.sign(x) * bf_ulp
    assert np.all(err <= np.minimum(np.abs(lo - x), np.abs(hi - x)) + 1e-30)


# ---------------------------------------------------------- generators -----

def test_reference_xorshift_generator():
    """examples/test_gemm_correctness.rs:45-58: the first draws for seed 1, recomputed
    here with Python integers (xorshift64 <<13 >>7 <<17, high 32 bits / u32::MAX)."""
    s = (1 ^ 0xDEADBEEFCAFEBABE) & (2**64 - 1)
    want = []
    for _ in range(8):
        s ^= (s << 13) & (2**64 - 1)
        s ^= s >> 7
        s ^= (s << 17) & (2**64 - 1)
        u = np.float32(s >> 32) / np.float32(4294967295.0)
        f = np.float32(u * np.float32(2.0)) - np.float32(1.0)
        want.append(f)
    got = oracle.rand_bf16_ref(8, 1)
    assert np.array_equal(got, oracle.bf16_rne(np.array(want, np.float32)))


def test_generators_moments_and_determinism():
    a = oracle.normal_bf16((512, 512), 0x7401, 0.0, 1.0)
    v = oracle.bf16_to_f32(a)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert np.array_equal(a, oracle.normal_bf16((512, 512), 0x7401, 0.0, 1.0))
    u = oracle.bf16_to_f32(oracle.uniform_bf16((100000,), 3, 0.005, 0.02))
    assert u.min() >= 0.005 - 1e-4 and u.max() <= 0.02 + 1e-4
    q = oracle.nibbles((100000,), 4)
    assert q.max() == 15 and q.min() == 0 and abs(q.mean() - 7.5) < 0.05


# ---------------------------------------------------------------- GEMM -----

def _load(name, dtype, shape):
    return np.fromfile(os.path.join(GOLD, name), dtype).reshape(shape)


def test_golden_torch_fixtures_f32():
    """benchmarks/torch_ref: h = x . w^T (torch fp32 matmul of bf16 inputs).  Our
    sequential-fp32 sum must agree to fp32 rounding (a dropped term, a transposed
    operand or a wrong index would miss by orders of magnitude)."""
    x = _load("x.bin", np.uint16, (64, 256))
    for w, r in (("w_gate.bin", "h_gate_f32ref.bin"), ("w_up.bin", "h_up_f32ref.bin")):
        y = oracle.gemm_bf16(x, _load(w, np.uint16, (512, 256)), "nt")
        ref = _load(r, np.float32, (64, 512))
        assert np.abs(y - ref).max() < 5e-7
    s = _load("swiglu_bf16_trunc.bin", np.uint16, (64, 512))
    y = oracle.gemm_bf16(s, _load("w_down.bin", np.uint16, (256, 512)), "nt")
    assert np.abs(y - _load("y_bf16_f32acc.bin", np.float32, (64, 256))).max() < 5e-7


def test_golden_torch_fixtures_bf16_rne():
    """h_*_bf16acc (torch bf16 matmul) equals RNE of the fp32 product in all but
    rounding-boundary cases: pins the RNE bf16 output epilogue, not truncation."""
    x = _load("x.bin", np.uint16, (64, 256))
    y = oracle.gemm_bf16(x, _load("w_gate.bin", np.uint16, (512, 256)), "nt")
    bf = _load("h_gate_bf16acc.bin", np.float32, (64, 512))
    rne = oracle.bf16_to_f32(oracle.bf16_rne(y))
    trunc = oracle.bf16_to_f32(oracle.bf16_trunc(y))
    assert (rne == bf).mean() > 0.999
    assert (trunc == bf).mean() < 0.7


def test_golden_torch_fixtures_bf16_chain():
    """The bf16 chain of benchmarks/gen_torch_ref.py, which precision_vs_torch.rs:115-116
    checks its down projection against: swiglu_bf16chain = silu(h_gate_bf16acc) *
    h_up_bf16acc in fp32; swiglu_bf16_trunc its bf16 rounding (torch's .to(bfloat16),
    round-to-nearest-even); y_bf16chain = torch.mm of bf16 operands, bf16 output (K = 512).
    Pins the oracle's SiLU epilogue op and RNE on these data, and the bf16-output GEMM:
    RNE of the oracle's fp32 sum must be torch's bf16 value except at rounding
    boundaries (torch sums in another order), and never more than one bf16 ulp away."""
    gate = _load("h_gate_bf16acc.bin", np.float32, (64, 512))
    up = _load("h_up_bf16acc.bin", np.float32, (64, 512))
    chain = _load("swiglu_bf16chain.bin", np.float32, (64, 512))
    silu = oracle.epilogue(gate, [3])  # op 3: SiLU
    sw = (silu * up).astype(np.float32)
    rel = np.abs(sw - chain) / np.maximum(np.abs(chain), 1e-30)
    assert rel.max() < 1e-5, "SiLU(gate) * up, fp32"
    assert (oracle.epilogue(gate, [2]) * up != chain).mean() > 0.5, "a ReLU in place of SiLU is caught"
    trunc = _load("swiglu_bf16_trunc.bin", np.uint16, (64, 512))
    assert np.array_equal(oracle.bf16_rne(chain), trunc), "torch's bf16 cast is RNE"
    y = oracle.gemm_bf16(trunc, _load("w_down.bin", np.uint16, (256, 512)), "nt")
    yb = _load("y_bf16chain.bin", np.float32, (64, 256))
    mine = oracle.bf16_to_f32(oracle.bf16_rne(y))
    assert (mine == yb).mean() > 0.995
    ulp = np.abs(yb.view(np.uint32).astype(np.int64) - mine.view(np.uint32).astype(np.int64)) >> 16
    assert ulp.max() <= 1
    assert (oracle.bf16_to_f32(oracle.bf16_trunc(y)) == yb).mean() < 0.7, "truncation would be caught"


def test_fast_loop_bit_identical_to_literal_reference_order():
    """The vectorised i-k-j loop must reproduce cpu_gemm_nt_bf16's i-j-k sequential
    fp32 order bit for bit (tile_ir.rs:5021-5038)."""
    a = oracle.normal_bf16((33, 300), 1, 0.0, 1.0)
    b = oracle.normal_bf16((70, 300), 2, 0.0, 1.0)
    y = oracle.gemm_bf16(a, b, "nt")
    assert np.array_equal(y.view(np.uint32), oracle.gemm_nt_literal(a, b).view(np.uint32))
    y1 = oracle.gemm_bf16(a, b, "nt", nthreads=1)
    assert np.array_equal(y.view(np.uint32), y1.view(np.uint32)), "thread count must not change results"
    # NN on the transposed matrix gives identical values
    y2 = oracle.gemm_bf16(a, np.ascontiguousarray(b.T), "nn")
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_integer_pattern_known_answer():
    """auto_gemm.rs:235-238 / :655: a=(i%7)-3, b=(j%5)-2 -> exact sums; Y[0,0] = -6 at (128,64,128)."""
    m, k, n = 128, 64, 128
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(n * k) % 5) - 2).astype(np.float32).reshape(n, k)
    y = oracle.gemm_bf16(oracle.bf16_trunc(a), oracle.bf16_trunc(b), "nt")
    assert y[0, 0] == -6.0
    exact = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32)
    assert np.array_equal(y, exact)


def test_bruteforce_tiny_and_closed_forms():
    rng = np.random.default_rng(1)
    for (m, k, n) in ((1, 1, 1), (2, 3, 4), (5, 17, 3), (7, 64, 9)):
        a = oracle.bf16_rne(rng.standard_normal((m, k)).astype(np.float32))
        b = oracle.bf16_rne(rng.standard_normal((k, n)).astype(np.float32))
        y = oracle.gemm_bf16(a, b, "nn")
        ref = oracle.bf16_to_f32(a).astype(np.float64) @ oracle.bf16_to_f32(b).astype(np.float64)
        assert np.abs(y - ref).max() <= 1e-5 * (1 + np.abs(ref).max())
    # identity and rank-1
    eye = oracle.bf16_trunc(np.eye(16, dtype=np.float32))
    x = oracle.normal_bf16((16, 16), 9, 0.0, 1.0)
    assert np.array_equal(oracle.gemm_bf16(x, eye, "nn"), oracle.bf16_to_f32(x))
    u = oracle.bf16_trunc(np.arange(1, 9, dtype=np.float32).reshape(8, 1))
    v = oracle.bf16_trunc(np.arange(1, 5, dtype=np.float32).reshape(1, 4))
    assert np.array_equal(oracle.gemm_bf16(u, v, "nn"), np.outer(np.arange(1, 9), np.arange(1, 5)).astype(np.float32))


def test_tolerance_rule():
    a = np.array([[0.5, -2.0]], np.float32)
    b = np.array([[3.0], [1.0]], np.float32)
    assert oracle.gemm_tolerance(4, a, b) == pytest.approx(1e-2 * 2 * 2.0 * 3.0)
    assert oracle.compare(np.array([1.0, 2.0]), np.array([1.0, 2.0])) == (0.0, 0.0)


# ---------------------------------------------------------------- INT4 -----

def test_nibble_known_answers():
    """quant_kernels.rs:346-382, 441-469: 0xAB -> lo 11 / hi 10; 0xD7 -> 7 / 13;
    lo nibble is element 2i."""
    packed = np.array([[0xAB, 0xD7]], np.uint8)  # one row (n), K = 4
    q = oracle.unpack_gptq_bytes(packed, 4)
    assert q[:, 0].tolist() == [11, 10, 7, 13]
    assert int(q[2, 0]) - 8 == -1 and int(q[3, 0]) - 8 == 5
    assert np.array_equal(oracle.pack_gptq_bytes(q), packed)


def test_dequant_formula_known_answers():
    """quant_kernels.rs:359-364: (12 - 8) * 0.5 = 2.0; group index 200 // 128 = 1."""
    K, N, g = 256, 8, 128
    q = np.zeros((K, N), np.uint8)
    q[200, 3] = 12
    q[127, 3] = 12
    w = oracle.pack_qweight(q)
    s = np.zeros((K // g, N), np.float32)
    s[1, 3] = 0.5   # group 1 (k = 128..255)
    s[0, 3] = 0.25  # group 0
    wf = oracle.dequant_qweight_f32(w, oracle.bf16_trunc(s), None, g, 8)
    assert wf[200, 3] == 2.0
    assert wf[127, 3] == 1.0
    assert wf[0, 3] == -8 * 0.25
    assert wf[0, 0] == 0.0  # scale 0 -> 0 (and -8 * 0 = -0.0 compares equal)


def test_gptq_from_bytes_layout_16x16():
    """quant_kernels.rs:385-422: a 16x16 g16 container of 0xAB bytes, scale 1.0, zp 8:
    elements alternate (0xB - 8, 0xA - 8) = (3, 2) along each row."""
    rows, cols, g = 16, 16, 16
    packed = np.full((rows, cols // 2), 0xAB, np.uint8)
    out = oracle.dequant_gptq_f32(packed, np.ones(rows, np.float32), np.full(rows, 8, np.int32), rows, cols, g)
    assert np.array_equal(out[:, 0::2], np.full((rows, cols // 2), 3.0, np.float32))
    assert np.array_equal(out[:, 1::2], np.full((rows, cols // 2), 2.0, np.float32))


def test_layout_round_trips_and_cross_layout_dequant():
    """qweight [K/8][N] u32 <-> q[K][N] <-> GPTQ bytes [N][K/2]; dequant of both
    layouts agrees element for element (catches a transposed or nibble-swapped layout)."""
    K, N, g = 256, 24, 64
    q = oracle.nibbles((K, N), 5)
    w = oracle.pack_qweight(q)
    assert np.array_equal(oracle.unpack_qweight(w), q)
    packed = oracle.pack_gptq_bytes(q)
    assert np.array_equal(oracle.unpack_gptq_bytes(packed, K), q)
    # word (kk, n) nibble e is q[8kk+e, n]; GPTQ byte (n, i) low nibble is q[2i, n]
    assert (int(w[3, 5]) >> 8) & 0xF == q[26, 5]
    assert packed[5, 13] & 0xF == q[26, 5]
    s_bf = oracle.uniform_bf16((K // g, N), 6, -0.1, 0.1)
    zq = oracle.nibbles((K // g, N), 7)
    wf = oracle.dequant_qweight_f32(w, s_bf, oracle.pack_qzeros(zq), g, 0)
    gptq = oracle.dequant_gptq_f32(packed, oracle.bf16_to_f32(s_bf).T.copy(), zq.astype(np.int32).T.copy(), N, K, g)
    assert np.array_equal(wf.T, gptq)
    # closed form: (q - z) * s is exact in fp32, compare with float64
    ref = (q.astype(np.float64) - np.repeat(zq, g, axis=0)) * np.repeat(oracle.bf16_to_f32(s_bf), g, axis=0)
    assert np.array_equal(wf.astype(np.float64), ref)


def test_w4a16_oracle_is_dequant_then_gemm():
    m, K, N, g = 3, 256, 16, 128
    a = oracle.normal_bf16((m, K), 8, 0.0, 1.0)
    q = oracle.nibbles((K, N), 9)
    w = oracle.pack_qweight(q)
    s = oracle.uniform_bf16((K // g, N), 10, 0.005, 0.02)
    y = oracle.w4a16_gemm(a, w, s, None, g, 8)
    wf = oracle.dequant_qweight_f32(w, s, None, g, 8)
    # sequential fp32 in k order, restated in numpy for a tiny case
    af = oracle.bf16_to_f32(a)
    ref = np.zeros((m, N), np.float32)
    for kk in range(K):
        ref = (ref + (af[:, kk:kk + 1] * wf[kk:kk + 1, :]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("zeros", [False, True])
def test_w4a16_oracle_against_float64_brute_force_from_raw_nibbles(zeros):
    """orc_w4a16_gemm pinned by a float64 brute force written from the definitions
    alone, in pure Python: the packed words are assembled bit by bit from raw
    nibbles (word (kk, n) holds q[8kk+e][n] in bits 4e..4e+3, quant_kernels.rs:3-10),
    zero points either the constant 8 or a nibble per (group, column) (u32 word
    (g, n/8), bits 4(n%8)), w = (q - z) * s (quant_kernels.rs:24, 95-100).
    The oracle sums in fp32, so it may differ from the float64 sum by at most
    K * 2^-24 * sum|a w| per output; a swapped nibble order, a transposed word, a
    wrong group index or a dropped zero point is off by far more."""
    import random
    import struct
    M, K, N, g = 2, 256, 32, 128
    rnd = random.Random(1234 + zeros)
    q = [[rnd.randrange(16) for _ in range(N)] for _ in range(K)]
    z = [[rnd.randrange(16) if zeros else 8 for _ in range(N)] for _ in range(K // g)]
    # bf16 bit patterns: activations roughly N(0,1), scales in [2^-8, 2^-5)
    def bf16_bits(x):
        return struct.unpack("<I", struct.pack("<f", x))[0] >> 16
    def bits_to_float(h):
        return struct.unpack("<f", struct.pack("<I", h << 16))[0]
    a_bits = [[bf16_bits(rnd.gauss(0.0, 1.0)) for _ in range(K)] for _ in range(M)]
    s_bits = [[bf16_bits(2.0 ** rnd.uniform(-8, -5)) for _ in range(N)] for _ in range(K // g)]
    words = [[sum(q[8 * kk + e][n] << (4 * e) for e in range(8)) for n in range(N)] for kk in range(K // 8)]
    zwords = [[sum(z[gi][8 * nn + e] << (4 * e) for e in range(8)) for nn in range(N // 8)]
              for gi in range(K // g)]
    y64 = [[0.0] * N for _ in range(M)]
    bound = [[0.0] * N for _ in range(M)]
    for i in range(M):
        for n in range(N):
            acc = mag = 0.0
            for k in range(K):
                wv = (q[k][n] - z[k // g][n]) * bits_to_float(s_bits[k // g][n])
                av = bits_to_float(a_bits[i][k])
                acc += av * wv
                mag += abs(av * wv)
            y64[i][n], bound[i][n] = acc, mag
    a = np.array(a_bits, np.uint16)
    w = np.array(words, np.uint32)
    s = np.array(s_bits, np.uint16)
    zw = np.array(zwords, np.uint32) if zeros else None
    y = oracle.w4a16_gemm(a, w, s, zw, g, 8)
    y64, bound = np.array(y64), np.array(bound)
    err = np.abs(y.astype(np.float64) - y64)
    assert np.all(err <= K * 2.0 ** -24 * bound + 1e-30), float((err / (bound + 1e-30)).max())
    # the check has teeth: the same sums with the nibbles read high-first miss it
    q_swapped = oracle.unpack_qweight(w)[np.arange(K) ^ 7]
    y_bad = oracle.w4a16_gemm(a, oracle.pack_qweight(q_swapped), s, zw, g, 8)
    assert np.any(np.abs(y_bad.astype(np.float64) - y64) > K * 2.0 ** -24 * bound)


# ------------------------------------------------------- epilogue chain ----

def test_epilogue_closed_forms():
    """Each EpilogueOp (src/t0/tile_ir.rs:3400-3540) against values fixed by its definition."""
    y = np.array([[-3.0, -0.5, 0.0, 0.5, 3.0, 40.0, -40.0, 1.0]], dtype=np.float32)
    bias = np.arange(8, dtype=np.float32)
    assert np.array_equal(oracle.epilogue(y, [0], bias=bias), y + bias)
    assert np.array_equal(oracle.epilogue(y, [1], scale=0.25), y * np.float32(0.25))
    assert np.array_equal(oracle.epilogue(y, [2]), np.maximum(y, 0))
    assert np.array_equal(oracle.epilogue(y, [5]), np.abs(y))
    assert np.array_equal(oracle.epilogue(y, [6]), -y)
    assert np.array_equal(oracle.epilogue(y, [7], clamp_min=-1.0, clamp_max=2.0), np.clip(y, -1.0, 2.0))
    silu = oracle.epilogue(y, [3])[0]
    assert silu[2] == 0.0
    assert abs(silu[5] - 40.0) < 1e-5 and abs(silu[6]) < 1e-15      # tails: x and 0
    assert abs(silu[7] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7           # silu(1) = sigmoid(1)
    assert abs(silu[0] - (-3.0 / (1.0 + np.exp(3.0)))) < 1e-6
    gelu = oracle.epilogue(y, [4])[0]
    assert gelu[2] == 0.0
    assert abs(gelu[7] - 1.0 / (1.0 + np.exp(-1.702))) < 1e-7          # sigmoid form at 1
    assert abs(gelu[4] - 3.0 / (1.0 + np.exp(-1.702 * 3.0))) < 1e-6


def test_epilogue_order_of_application():
    """Ops apply in list order: bias then relu differs from relu then bias."""
    y = np.array([[-2.0, 1.0]], dtype=np.float32)
    b = np.array([1.0, -3.0], dtype=np.float32)
    assert np.array_equal(oracle.epilogue(y, [0, 2], bias=b), [[0.0, 0.0]])
    assert np.array_equal(oracle.epilogue(y, [2, 0], bias=b), [[1.0, -2.0]])
    assert np.array_equal(oracle.epilogue(y, [6, 7], clamp_min=-1.5, clamp_max=1.5), [[1.5, -1.0]])
    assert np.array_equal(oracle.epilogue(y, []), y)
    with pytest.raises(ValueError):
        oracle.epilogue(y, [0])
