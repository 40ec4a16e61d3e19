"""GPU parity of the quantized matmul (decode GEMV, tokens <= 16 per pass,
and multi-block token counts) through the C ABI against the oracle.

Bar: the int32 group sums are bit-exact; the fp32 outputs are bit-exact too,
because the kernel keeps Scalar.MatMulRows' epilogue order (the required
tolerance, max-abs-error <= 1e-4 * RMS(y), is asserted as well)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(12345.0)


def int8_case(orc, seed, rows, cols, tokens):
    st = orc.state(seed)
    w = orc.synth_int8(st, rows * cols).reshape(rows, cols)
    scales = orc.synth_half_uniform(st, rows * cols // 32, 0.002, 0.02).reshape(rows, cols // 32)
    x = orc.synth_normal(st, tokens * cols).reshape(tokens, cols)
    q, qs = orc.quantize_rows(x)
    return w, scales, x, q, qs


def run_i8(hip, weights, q, qs, tokens, ldy, r0, r1, fill=SENTINEL):
    N = hip
    dq = N.DeviceBuffer.from_array(q)
    ds = N.DeviceBuffer.from_array(qs)
    y = np.full(max(tokens, 1) * ldy, fill, dtype=np.float32)
    dy = N.DeviceBuffer.from_array(y)
    N.check(N.lib().nhip_matmul_i8_dev(weights.handle, dq.ptr, ds.ptr, tokens, dy.ptr, ldy, r0, r1, None))
    return dy.download(np.float32).reshape(max(tokens, 1), ldy)


def assert_tolerance(y, want):
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert np.max(np.abs(y.astype(np.float64) - want)) <= 1e-4 * rms


@pytest.mark.parametrize("tokens,rows,cols", [
    (1, 4096, 1024),      # single decode GEMV (M=1, K=1024, N=4096)
    (3, 2048, 2048),      # beam-3 rows
    (16, 2048, 2048),     # 16 packed rows
    (3, 8192, 2048),
    (16, 8192, 2048),
    (2, 37, 96),          # ragged rows, odd group count
    (5, 16, 32),          # one group
    (17, 48, 256),        # two token blocks
    (33, 80, 512),        # three token blocks
    (4, 1024, 4096),      # K = 4096 (two weight chunks)
    (3, 1024, 3072),      # K = 3072: not a narrow-kernel shape
    (1, 3072, 3072),
])
def test_int8_matmul_bit_exact(hip, orc, tokens, rows, cols):
    w, scales, x, q, qs = int8_case(orc, tokens * 1000 + rows + cols, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, tokens, rows, 0, rows)
    want = np.full((tokens, rows), SENTINEL, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    assert_tolerance(y, want.astype(np.float64))


@pytest.mark.parametrize("tokens,rows,cols", [(1, 4096, 1024), (3, 2048, 2048), (16, 256, 2048), (7, 37, 96)])
def test_int8_group_sums_bit_exact(hip, orc, tokens, rows, cols):
    w, scales, x, q, qs = int8_case(orc, 7 + tokens, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    r0, r1 = 0, rows
    dq = hip.DeviceBuffer.from_array(q)
    dd = hip.DeviceBuffer(tokens * (r1 - r0) * (cols // 32) * 4)
    dd.zero()
    hip.check(hip.lib().nhip_group_dots_i8_dev(weights.handle, dq.ptr, tokens, r0, r1, dd.ptr, None))
    got = dd.download(np.int32).reshape(tokens, r1 - r0, cols // 32)
    assert np.array_equal(got, orc.group_dots_i8(w, q, tokens, r0, r1))


@pytest.mark.parametrize("r0,r1,tokens", [(5, 29, 3), (16, 32, 1), (0, 1, 16), (31, 37, 5), (7, 7, 2)])
def test_int8_rows_outside_range_untouched(hip, orc, r0, r1, tokens):
    rows, cols = 37, 256
    w, scales, x, q, qs = int8_case(orc, 99, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    ldy = rows + 3
    y = run_i8(hip, weights, q, qs, tokens, ldy, r0, r1)
    want = np.full((tokens, ldy), SENTINEL, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, ldy, r0, r1)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_int8_zero_tokens_is_a_no_op(hip, orc):
    w, scales, x, q, qs = int8_case(orc, 5, 32, 64, 1)
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, 0, 32, 0, 32)
    assert np.all(y == SENTINEL)


def test_int8_rejects_bad_ranges(hip, orc):
    w, scales, x, q, qs = int8_case(orc, 6, 32, 64, 1)
    weights = hip.Weights.int8(w, scales)
    dq = hip.DeviceBuffer.from_array(q)
    ds = hip.DeviceBuffer.from_array(qs)
    dy = hip.DeviceBuffer(32 * 4)
    assert hip.lib().nhip_matmul_i8_dev(weights.handle, dq.ptr, ds.ptr, 1, dy.ptr, 32, 0, 33, None) != 0
    assert hip.lib().nhip_matmul_i8_dev(weights.handle, dq.ptr, ds.ptr, 1, dy.ptr, 16, 0, 32, None) != 0
    assert "row range" in hip.last_error() or "ldy" in hip.last_error()


@pytest.mark.parametrize("tokens,cols", [(1, 1024), (3, 2048), (16, 4096), (2, 96)])
def test_quantize_rows_bit_exact(hip, orc, tokens, cols):
    st = orc.state(tokens + cols)
    x = orc.synth_normal(st, tokens * cols).reshape(tokens, cols)
    x[:, ::9] = 0.0
    dx = hip.DeviceBuffer.from_array(x)
    dq = hip.DeviceBuffer(tokens * cols)
    ds = hip.DeviceBuffer(tokens * 4)
    hip.check(hip.lib().nhip_quantize_rows_dev(dx.ptr, tokens, cols, dq.ptr, ds.ptr, None))
    q, s = orc.quantize_rows(x)
    assert np.array_equal(dq.download(np.int8).reshape(tokens, cols), q)
    assert np.array_equal(ds.download(np.float32), s)


def test_quantize_then_matmul_on_device_matches_oracle_pipeline(hip, orc):
    tokens, rows, cols = 3, 1024, 2048
    w, scales, x, q, qs = int8_case(orc, 31337, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    dx = hip.DeviceBuffer.from_array(x)
    dq = hip.DeviceBuffer(tokens * cols)
    ds = hip.DeviceBuffer(tokens * 4)
    dy = hip.DeviceBuffer(tokens * rows * 4)
    hip.check(hip.lib().nhip_quantize_rows_dev(dx.ptr, tokens, cols, dq.ptr, ds.ptr, None))
    hip.check(hip.lib().nhip_matmul_i8_dev(weights.handle, dq.ptr, ds.ptr, tokens, dy.ptr, rows, 0, rows, None))
    want = np.zeros((tokens, rows), dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    assert np.array_equal(dy.download(np.float32).reshape(tokens, rows), want)


# ------------------------------------------------------ codebook (.cact) --

def cq_case(orc, seed, rows, cols, bits, tokens):
    """Synthetic Cq weights and prepared activations as the reference's
    MatMulTests build them (tests/Needle.Tests/MatMulTests.cs:182-208), from
    the conformance XorShift64 stream."""
    st = orc.state(seed)
    count = 4 if bits == 2 else 16
    lib = orc.lib()
    levels = np.array([(i - (count - 1) / 2) * 0.4 + (lib.or_synth_u53(C.byref(st)) - 0.5) * 0.1 for i in range(count)],
                      dtype=np.float32)
    book = orc.codebook(levels, count)
    indices = np.zeros(rows * cols * bits // 8, dtype=np.uint8)
    lib.or_fill_bytes(orc.p(indices), indices.size, C.byref(st), 1)
    g = cols // 128
    norms = np.array([lib.or_single_to_half_rne(0.2 + lib.or_synth_u53(C.byref(st)) * 1.8) for _ in range(rows * g)],
                     dtype=np.uint16)
    norms[::11] = 0
    norms[-1] = 0x7BFF
    x = np.zeros(tokens * cols, dtype=np.float32)
    lib.or_fill_edges(orc.p(x), x.size, C.byref(st), 3.0)
    act, values, sc, off = orc.prepare(x, tokens, cols, bits)
    cq = orc.Cq(orc.p(indices), orc.p(norms), C.pointer(book), rows, cols, bits)
    return dict(book=book, indices=indices, norms=norms, x=x, act=act, values=values, scales=sc, offsets=off, cq=cq)


def hip_book(hip, book):
    hb = hip.Codebook()
    C.memmove(C.byref(hb), C.byref(book), C.sizeof(hb))
    return hb


SHAPES = [(1, 128), (3, 128), (4, 256), (5, 768), (13, 768), (64, 1024), (97, 768), (576, 768), (24, 3072),
          (320, 3072)]


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_cq_matmul_bit_exact_one_to_nine_tokens(hip, orc, bits, rows, cols):
    """tests/Needle.Tests/MatMulTests.cs:15-39 (shapes, tokens 1..9)."""
    for tokens in (1, 2, 3, 4, 5, 9):
        c = cq_case(orc, rows * 31 + cols + bits + tokens, rows, cols, bits, tokens)
        weights = hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)
        stride = c["act"].stride
        dv = hip.DeviceBuffer.from_array(c["values"])
        ds = hip.DeviceBuffer.from_array(c["scales"])
        do = hip.DeviceBuffer.from_array(c["offsets"])
        dy = hip.DeviceBuffer.from_array(np.full(tokens * rows, SENTINEL, dtype=np.float32))
        hip.check(hip.lib().nhip_matmul_cq_dev(weights.handle, dv.ptr, ds.ptr, do.ptr, stride, tokens, dy.ptr, rows,
                                               0, rows, None))
        want = np.full(tokens * rows, SENTINEL, dtype=np.float32)
        orc.matmul_rows(c["cq"], c["act"], tokens, want, rows, 0, rows)
        got = dy.download(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (tokens, np.max(np.abs(got - want)))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("tokens", [10, 16, 17, 33, 64])
def test_cq_matmul_bit_exact_wide_tokens(hip, orc, bits, tokens):
    """tests/Needle.Tests/MatMulTests.cs:41-63."""
    rows, cols = 97, 768
    c = cq_case(orc, tokens + bits, rows, cols, bits, tokens)
    weights = hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)
    dv = hip.DeviceBuffer.from_array(c["values"])
    ds = hip.DeviceBuffer.from_array(c["scales"])
    do = hip.DeviceBuffer.from_array(c["offsets"])
    dy = hip.DeviceBuffer(tokens * rows * 4)
    hip.check(hip.lib().nhip_matmul_cq_dev(weights.handle, dv.ptr, ds.ptr, do.ptr, c["act"].stride, tokens, dy.ptr,
                                           rows, 0, rows, None))
    want = np.zeros(tokens * rows, dtype=np.float32)
    orc.matmul_rows(c["cq"], c["act"], tokens, want, rows, 0, rows)
    assert np.array_equal(dy.download(np.float32), want)


@pytest.mark.parametrize("bits", [2, 4])
def test_cq_group_sums_bit_exact(hip, orc, bits):
    rows, cols, tokens = 40, 768, 5
    c = cq_case(orc, 77 + bits, rows, cols, bits, tokens)
    weights = hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)
    dv = hip.DeviceBuffer.from_array(c["values"])
    dd = hip.DeviceBuffer(tokens * rows * (cols // 128) * 4)
    hip.check(hip.lib().nhip_group_dots_cq_dev(weights.handle, dv.ptr, tokens, 0, rows, dd.ptr, None))
    got = dd.download(np.int32).reshape(tokens, rows, cols // 128)
    assert np.array_equal(got, orc.group_dots_cq(c["cq"], c["act"], tokens, 0, rows))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("cols,tokens", [(128, 1), (128, 3), (768, 1), (768, 3), (3072, 9)])
def test_prepare_bit_exact(hip, orc, bits, cols, tokens):
    """KernelConformanceTests.cs:192-335 (the reference allows +-1 per value;
    the HIP path is exact)."""
    st = orc.state(0x2458 + cols + tokens)
    x = np.zeros(tokens * cols, dtype=np.float32)
    orc.lib().or_fill_edges(orc.p(x), x.size, C.byref(st), 2.0)
    act, values, sc, off = orc.prepare(x, tokens, cols, bits)
    dx = hip.DeviceBuffer.from_array(x)
    dv = hip.DeviceBuffer(tokens * cols)
    ds = hip.DeviceBuffer.from_array(np.zeros(tokens * act.stride, dtype=np.float32))
    do = hip.DeviceBuffer.from_array(np.zeros(tokens * act.stride, dtype=np.float32))
    hip.check(hip.lib().nhip_prepare_dev(dx.ptr, tokens, cols, bits, dv.ptr, ds.ptr, do.ptr, act.stride, None))
    assert np.array_equal(dv.download(np.int8), values)
    assert np.array_equal(ds.download(np.float32), sc)
    assert np.array_equal(do.download(np.float32), off)


def run_cq(hip, c, rows, cols, bits, tokens, ldy, r0, r1):
    weights = hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)
    dv = hip.DeviceBuffer.from_array(c["values"])
    ds = hip.DeviceBuffer.from_array(c["scales"])
    do = hip.DeviceBuffer.from_array(c["offsets"])
    dy = hip.DeviceBuffer.from_array(np.full(tokens * ldy, SENTINEL, dtype=np.float32))
    hip.check(hip.lib().nhip_matmul_cq_dev(weights.handle, dv.ptr, ds.ptr, do.ptr, c["act"].stride, tokens, dy.ptr,
                                           ldy, r0, r1, None))
    return dy.download(np.float32)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("r0,r1", [(0, 37), (5, 29), (16, 17)])
def test_cq_decode_path_row_ranges(hip, orc, bits, tokens, r0, r1):
    """1..4 tokens run the codebook decode kernel, 5..16 the general one: K =
    640 (5 groups, a partial set of four), 2048, 8192 (64 groups) and 16384
    (128 groups, 16 per wave, the most the decode kernel takes)."""
    rows = 37
    ldy = rows + 5
    for cols in (640, 2048, 8192, 16384):
        c = cq_case(orc, 6000 + tokens * 10 + r0 + cols + bits, rows, cols, bits, tokens)
        got = run_cq(hip, c, rows, cols, bits, tokens, ldy, r0, r1)
        want = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
        orc.matmul_rows(c["cq"], c["act"], tokens, want, ldy, r0, r1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), cols


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("tokens", [3, 9, 20])
def test_cq_special_norm_patterns(hip, orc, bits, tokens):
    """Zero, negative-zero, subnormal and exponent-31 fp16 norms decode as
    Scalar.HalfToSingle does (Scalar.cs:121-128), in the decode kernel (3
    tokens) and the general kernel (9 and 20: one and two token blocks)."""
    rows, cols = 64, 2048
    c = cq_case(orc, 777 + tokens + bits, rows, cols, bits, tokens)
    flat = c["norms"]
    flat[::7] = 0x8000
    flat[::11] = 0x0000
    flat[::13] = 0x0001
    flat[::17] = 0x83FF
    flat[::19] = 0x7C00
    flat[::23] = 0xFC01
    got = run_cq(hip, c, rows, cols, bits, tokens, rows, 0, rows)
    want = np.full(tokens * rows, SENTINEL, dtype=np.float32)
    orc.matmul_rows(c["cq"], c["act"], tokens, want, rows, 0, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("extra", [1, 4])
def test_cq_wide_tokens_any_stride(hip, orc, bits, extra):
    """Activation scale rows of any stride >= G (here G + 1, not a multiple
    of 4, and G + 4) give the reference's bits."""
    rows, cols, tokens = 48, 2048, 7
    g = cols // 128
    c = cq_case(orc, 313 + bits + extra, rows, cols, bits, tokens)
    stride = g + extra
    sc = np.zeros((tokens, stride), dtype=np.float32)
    of = np.zeros((tokens, stride), dtype=np.float32)
    sc[:, :g] = c["scales"].reshape(tokens, -1)[:, :g]
    of[:, :g] = c["offsets"].reshape(tokens, -1)[:, :g]
    weights = hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)
    dv = hip.DeviceBuffer.from_array(c["values"])
    ds = hip.DeviceBuffer.from_array(sc)
    do = hip.DeviceBuffer.from_array(of)
    dy = hip.DeviceBuffer.from_array(np.full(tokens * rows, SENTINEL, dtype=np.float32))
    hip.check(hip.lib().nhip_matmul_cq_dev(weights.handle, dv.ptr, ds.ptr, do.ptr, stride, tokens, dy.ptr, rows, 0,
                                           rows, None))
    want = np.full(tokens * rows, SENTINEL, dtype=np.float32)
    orc.matmul_rows(c["cq"], c["act"], tokens, want, rows, 0, rows)
    assert np.array_equal(dy.download(np.float32).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
def test_codebook_bytes_above_127_are_rejected(hip, orc, bits):
    """The kernels multiply codebook bytes as signed int8 MFMA operands, so
    a codebook byte of 128 or more (Codebook.Fill makes [0, 126]) is refused
    when the weights are created, before anything is uploaded; bytes the
    format never indexes (4..15 of a 2-bit book) are not checked."""
    rows, cols = 16, 256
    c = cq_case(orc, 991 + bits, rows, cols, bits, 1)
    c["book"].bytes[7] = 200
    if bits == 2:
        hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits).close()
        c["book"].bytes[3] = 128
    with pytest.raises(hip.NeedleHipError, match="codebook byte"):
        hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), rows, cols, bits)


# ------------------------------------------------- kernel-table entries --

@pytest.mark.parametrize("bits,rows,cols,tokens,r0,r1", [
    (2, 37, 768, 5, 29, 37), (2, 37, 768, 1, 2, 3), (4, 37, 768, 3, 36, 37), (4, 21, 256, 8, 0, 21),
    (2, 50, 384, 16, 0, 7)])
def test_kernel_table_matmul_rows_leaves_rows_untouched(hip, orc, bits, rows, cols, tokens, r0, r1):
    """tests/Needle.Tests/MatMulTests.cs:115-137 through the MatMulRows slot."""
    c = cq_case(orc, rows + r0, rows, cols, bits, tokens)
    book = hip_book(hip, c["book"])
    cq = hip.Cq(c["indices"].ctypes.data, c["norms"].ctypes.data, C.pointer(book), rows, cols, bits)
    a = c["act"]
    act = hip.Activations(a.values, a.scales, a.offsets, a.cols, a.groups, a.stride)
    ldy = rows + 3
    got = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
    hip.lib().nhip_matmul_rows(C.byref(cq), C.byref(act), tokens, got.ctypes.data, ldy, r0, r1)
    assert hip.last_error() == ""
    # the entry caches the weights' device copy by host address; drop it as
    # the reference's host does when it disposes of a model, so that a later
    # case whose arrays reuse these addresses uploads its own weights
    released = C.c_int32(0)
    hip.check(hip.lib().nhip_table_release(c["indices"].ctypes.data, c["indices"].nbytes, C.byref(released)))
    assert released.value == 1
    want = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
    orc.matmul_rows(c["cq"], c["act"], tokens, want, ldy, r0, r1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_kernel_table_prepare_and_quantize(hip, orc):
    tokens, cols, bits = 3, 768, 4
    st = orc.state(0x2458)
    x = np.zeros(tokens * cols, dtype=np.float32)
    orc.lib().or_fill_uniform(orc.p(x), x.size, C.byref(st), 2.0)
    want_act, want_v, want_s, want_o = orc.prepare(x, tokens, cols, bits)
    groups, stride = cols // 128, want_act.stride
    v = np.zeros(tokens * cols, dtype=np.int8)
    s = np.zeros(tokens * stride, dtype=np.float32)
    o = np.zeros(tokens * stride, dtype=np.float32)
    act = hip.Activations(v.ctypes.data, s.ctypes.data, o.ctypes.data, cols, groups, stride)
    hip.lib().nhip_prepare(x.ctypes.data, tokens, cols, bits, C.byref(act))
    assert np.array_equal(v, want_v) and np.array_equal(s, want_s) and np.array_equal(o, want_o)
    g = np.array([-4, 0, 4, 0, 0, 0, 0, 0], dtype=np.float32)
    q = np.zeros(8, dtype=np.int8)
    scale = hip.lib().nhip_quantize_int8(g.ctypes.data, 8, q.ctypes.data)
    assert abs(scale - 0.03149606) <= 1e-6 and list(q) == [-127, 0, 127, 0, 0, 0, 0, 0]


# ----------------------------------------- decode kernel (M <= 16) edges --

@pytest.mark.parametrize("tokens", [1, 2, 3, 4])
@pytest.mark.parametrize("r0,r1", [(0, 37), (5, 29), (16, 17)])
def test_int8_decode_path_row_ranges(hip, orc, tokens, r0, r1):
    """M <= 4 with K = 1024 and K = 4096 runs the chained decode kernel."""
    for cols in (1024, 4096):
        rows = 37
        w, scales, x, q, qs = int8_case(orc, 4000 + tokens * 10 + r0 + cols, rows, cols, tokens)
        weights = hip.Weights.int8(w, scales)
        ldy = rows + 5
        y = run_i8(hip, weights, q, qs, tokens, ldy, r0, r1)
        want = np.full((tokens, ldy), SENTINEL, dtype=np.float32)
        orc.matmul_rows_i8(w, scales, q, qs, tokens, want, ldy, r0, r1)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("tokens", [5, 8, 13, 16])
@pytest.mark.parametrize("r0,r1", [(0, 64), (5, 29), (16, 17)])
def test_int8_wide_decode_path_row_ranges(hip, orc, tokens, r0, r1):
    """5..16 rows: lanes hold four tokens each and the swizzled products
    overwrite the staged activations (K = 1024 and 2048; K = 4096 up to 8
    rows, beyond which the general kernel runs)."""
    for cols in (1024, 2048, 4096):
        rows = 64
        w, scales, x, q, qs = int8_case(orc, 5000 + tokens * 10 + r0 + cols, rows, cols, tokens)
        weights = hip.Weights.int8(w, scales)
        ldy = rows + 3
        y = run_i8(hip, weights, q, qs, tokens, ldy, r0, r1)
        want = np.full((tokens, ldy), SENTINEL, dtype=np.float32)
        orc.matmul_rows_i8(w, scales, q, qs, tokens, want, ldy, r0, r1)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), cols


@pytest.mark.parametrize("tokens", [3, 7])
def test_int8_special_scale_patterns(hip, orc, tokens):
    """Zero, negative-zero, subnormal and exponent-31 fp16 scales decode as
    Scalar.HalfToSingle does (Scalar.cs:121-128), in both kernels."""
    rows, cols = 64, 2048
    w, scales, x, q, qs = int8_case(orc, 555 + tokens, rows, cols, tokens)
    scales = scales.copy()
    flat = scales.reshape(-1)
    flat[::7] = 0x8000
    flat[::11] = 0x0000
    flat[::13] = 0x0001
    flat[::17] = 0x83FF
    flat[::19] = 0x7C00
    flat[::23] = 0xFC01
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, tokens, rows, 0, rows)
    want = np.zeros((tokens, rows), dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("nbytes,off", [(1 << 20, 0), (4096 + 7, 0), (3000, 3), (16, 0), (1, 0)])
def test_copy_dev(hip, nbytes, off):
    src = np.random.default_rng(nbytes).integers(0, 256, nbytes + 32, dtype=np.uint8)
    ds = hip.DeviceBuffer.from_array(src)
    dd = hip.DeviceBuffer(nbytes + 32)
    dd.zero()
    hip.check(hip.lib().nhip_copy_dev(dd.ptr + off, ds.ptr + off, nbytes, None))
    hip.check(hip.lib().nhip_device_sync())
    got = dd.download(np.uint8)
    want = np.zeros(nbytes + 32, dtype=np.uint8)
    want[off:off + nbytes] = src[off:off + nbytes]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("tokens", [1, 2, 3, 4])
@pytest.mark.parametrize("rows,cols,r0,r1", [
    (1024, 4096, 0, 1024),   # the decoder's down matmul: 4-row workgroups, K = 4096
    (1000, 1024, 0, 1000),   # 4-row workgroups, rows not a multiple of 4
    (2048, 2048, 5, 1999),   # a row range cutting workgroups at both ends
    (3000, 2048, 0, 3000),   # 8-row workgroups, ragged last workgroup
    (4096, 1024, 1234, 4001),
    (3072, 4096, 0, 3072),
])
def test_int8_narrow_decode_bit_exact(hip, orc, tokens, rows, cols, r0, r1):
    """Matrices of at most 4096 rows with K a multiple of 1024 and at most 4
    tokens take the narrow kernel (4 or 8 whole rows per workgroup, from the
    row-major copy): bit-exact with the oracle, rows outside [r0, r1)
    untouched."""
    w, scales, x, q, qs = int8_case(orc, 31 * tokens + rows + 7 * cols, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, tokens, rows + 3, r0, r1)
    want = np.full((tokens, rows + 3), SENTINEL, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows + 3, r0, r1)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
