"""CPU tests of the GPTQ container parser and the host-side checks of the Ignis
matmul / GPTQ conversion entry points (null backend: arguments are validated,
nothing is launched).

Known answers come from the reference's own host tests of GptqWeight
(src/t0/quant_kernels.rs:385-422 from_bytes, :472-481 gpu_buffer_size).
"""
import struct

import numpy as np
import pytest

import t0mi


def container(rows, cols, group, packed, scales, zeros):
    return (struct.pack("<3I", rows, cols, group) + np.asarray(packed, np.uint8).tobytes()
            + np.asarray(scales, "<f4").tobytes()
            + np.asarray(zeros, "<i4").tobytes())


def test_from_bytes_known_answer_16x16():
    """quant_kernels.rs:385-422: 16x16, group 16, 0xAB bytes, scales 1.0, zero points 8."""
    raw = container(16, 16, 16, [0xAB] * 128, [1.0] * 16, [8] * 16)
    g = t0mi.GptqWeight.from_bytes(raw)
    assert (g.rows, g.cols, g.group_size, g.n_groups) == (16, 16, 16, 1)
    assert len(g.packed_weights) == 128 and set(g.packed_weights) == {0xAB}
    assert np.all(np.frombuffer(g.scales_bytes, "<f4") == 1.0) and len(g.scales_bytes) == 64
    assert np.all(np.frombuffer(g.zeros_bytes, "<i4") == 8) and len(g.zeros_bytes) == 64
    assert g.info.zeros_in_range == 1 and g.info.scales_bf16_exact == 1
    assert (g.info.packed_offset, g.info.scales_offset, g.info.zeros_offset, g.info.total_bytes) == (12, 140, 204, 268)


def test_gpu_buffer_size_known_answer():
    """quant_kernels.rs:472-481: 128 + 16*4 + 16*4 = 256."""
    g = t0mi.GptqWeight.from_bytes(container(16, 16, 16, [0] * 128, [1.0] * 16, [8] * 16))
    assert g.gpu_buffer_size() == 256


def test_section_offsets_general():
    rows, cols, group = 24, 256, 64
    ng = cols // group
    raw = container(rows, cols, group, np.arange(rows * cols // 2) % 256, np.linspace(-1, 1, ng * rows),
                    np.arange(ng * rows) % 16)
    g = t0mi.GptqWeight.from_bytes(raw + b"trailing bytes are ignored")
    assert g.n_groups == ng
    assert g.info.packed_bytes == rows * cols // 2
    assert g.info.total_bytes == 12 + rows * cols // 2 + 8 * ng * rows
    assert np.array_equal(np.frombuffer(g.zeros_bytes, "<i4"), np.arange(ng * rows) % 16)


@pytest.mark.parametrize("raw,why", [
    (b"\x10\x00\x00\x00" * 2, "too short"),
    (container(16, 16, 16, [0] * 128, [1.0] * 16, [8] * 16)[:-1], "truncated"),
    (container(16, 16, 16, [0] * 128, [1.0] * 16, [8] * 16)[:12 + 127], "truncated"),
])
def test_from_bytes_rejects_where_the_reference_panics(raw, why):
    with pytest.raises(t0mi.T0miError) as e:
        t0mi.GptqWeight.from_bytes(raw)
    assert e.value.code == t0mi.ERR_INVALID and why in str(e.value)


@pytest.mark.parametrize("rows,cols,group", [
    (1589614079, 4095720868, 1),   # sections total 3 * 2^64 + 26 bytes: wrapped, 26 looked valid
    (0xFFFFFFFE, 0xFFFFFFFF, 1),   # n_groups * rows * 8 bytes of sections: past 2^64
    (0xFFFFFFFE, 0xFFFFFFFE, 2),
    (0x80000000, 0xFFFFFFFF, 1),
    (0xFFFFFFFE, 64, 1),           # large but below 2^64: plainly truncated
])
def test_header_sizes_past_the_buffer_are_refused(rows, cols, group):
    """Header values near 2^32 make the section sizes reach or pass 2^64 bytes; the
    parser must refuse them as truncated (checked before any section is read), not
    wrap the total and scan past the buffer.  The first header's total wraps to 26
    bytes, which 64-bit arithmetic accepted for this 4108-byte buffer, and the flag
    scan then read ~3e18 bytes past it."""
    raw = struct.pack("<3I", rows, cols, group) + bytes(4096)
    with pytest.raises(t0mi.T0miError) as e:
        t0mi.GptqWeight.from_bytes(raw)
    assert e.value.code == t0mi.ERR_INVALID and "truncated" in str(e.value)


def test_random_headers_parse_or_refuse():
    """Seeded random headers over short buffers: every call either parses with all
    sections inside the buffer or raises T0miError (no other outcome)."""
    rng = np.random.default_rng(0x6707)
    for _ in range(2000):
        rows, cols, group = (int(v) for v in rng.integers(0, 2**32, size=3, dtype=np.uint64))
        if rng.random() < 0.5:
            rows, cols = rows % 64, cols % 64
            group = group % 70
        body = rng.integers(0, 256, size=int(rng.integers(0, 600)), dtype=np.uint8).tobytes()
        raw = struct.pack("<3I", rows, cols, group) + body
        try:
            g = t0mi.GptqWeight.from_bytes(raw)
        except t0mi.T0miError as e:
            assert e.code == t0mi.ERR_INVALID
            continue
        assert g.info.total_bytes <= len(raw)
        assert g.info.total_bytes == 12 + rows * cols // 2 + 8 * (cols // group) * rows


def test_odd_element_count_is_an_error():
    """rows * cols odd: two INT4 values per byte cannot hold it (the reference's
    rows * cols / 2 would drop the last nibble)."""
    raw = container(3, 5, 5, [0] * 8, [1.0] * 3, [8] * 3)
    with pytest.raises(t0mi.T0miError) as e:
        t0mi.GptqWeight.from_bytes(raw)
    assert e.value.code == t0mi.ERR_INVALID and "odd" in str(e.value)


def test_group_size_zero_is_an_error():
    with pytest.raises(t0mi.T0miError):
        t0mi.GptqWeight.from_bytes(struct.pack("<3I", 16, 16, 0) + bytes(128))


def test_flags_zero_range_and_bf16_exact_scales():
    base = dict(rows=8, cols=32, group=32, packed=[0x11] * 128)
    ok = t0mi.GptqWeight.from_bytes(container(*base.values(), [0.5] * 8, list(range(8))))
    assert ok.info.zeros_in_range == 1 and ok.info.scales_bf16_exact == 1
    for z in (16, -1):
        bad = t0mi.GptqWeight.from_bytes(container(*base.values(), [0.5] * 8, [0] * 7 + [z]))
        assert bad.info.zeros_in_range == 0
    inexact = t0mi.GptqWeight.from_bytes(container(*base.values(), [0.5] * 7 + [0.1], [8] * 8))
    assert inexact.info.scales_bf16_exact == 0


@pytest.fixture(scope="module")
def null_rt():
    r = t0mi.Runtime(null=True)
    yield r
    r.close()


def test_matmul_argument_checks(null_rt):
    a = 1 << 20
    null_rt.matmul(a, a, a, 37, 100, 70)  # ragged shapes are accepted
    with pytest.raises(t0mi.T0miError):
        null_rt.matmul(a + 4, a, a, 16, 16, 16)  # f32 buffers must be 16-byte aligned
    with pytest.raises(t0mi.T0miError):
        null_rt.matmul(0, a, a, 16, 16, 16)
    with pytest.raises(t0mi.T0miError):
        null_rt.matmul_with_wt_bf16(a, a, a, 16, 12, 16)  # WT used in place: K % 8
    null_rt.matmul_backward_data(a, a, a, 5, 9, 13)
    null_rt.matmul_backward_weight(a, a, a, 5, 9, 13)


def test_gptq_convert_argument_checks(null_rt):
    a = 1 << 20
    null_rt.gptq_convert(a, a, a, 64, 256, 128, a, a, a)
    for rows, cols, group in ((64, 250, 125), (60, 256, 128), (64, 256, 96), (64, 256, 0)):
        with pytest.raises(t0mi.T0miError):
            null_rt.gptq_convert(a, a, a, rows, cols, group, a, a, a)
