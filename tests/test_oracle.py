"""Pins the oracle (CPU restatement of the reference) before it is trusted as
the parity checker: the reference's own known answers, independent numpy /
scipy computations, and invariants chosen so that a plausible mistake (a
dropped term, a wrong index or sign, a transposed operand) fails."""
import ctypes as C
import json
import os

import numpy as np
import pytest
import scipy.linalg

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
MASK64 = (1 << 64) - 1


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------- RNG --

def _xs(state):
    x = state
    x ^= (x << 13) & MASK64
    x ^= x >> 7
    x ^= (x << 17) & MASK64
    return x


def test_xorshift_stream_matches_recurrence(orc):
    st = orc.state(0x1234)
    ref = 0x1234
    for _ in range(2000):
        ref = _xs(ref)
        assert orc.lib().or_xs_next(C.byref(st)) == ref
    assert orc.lib().or_xs_seed(0) == 0x9E3779B97F4A7C15


def test_next_int_and_float_follow_conformance_definitions(orc):
    st, ref = orc.state(99), 99
    for _ in range(500):
        ref = _xs(ref)
        assert orc.lib().or_xs_next_int(C.byref(st), -127, 128) == -127 + ref % 255
    st, ref = orc.state(7), 7
    for _ in range(500):
        ref = _xs(ref)
        u = np.float32(ref >> 11) * np.float32(1.0 / 9007199254740992.0)
        want = ((u - np.float32(0.5)) * np.float32(2.0)) * np.float32(3.0)
        assert orc.lib().or_xs_next_float(C.byref(st), 3.0) == want


def test_half_bits_known_values(orc):
    hb = orc.lib().or_half_bits
    assert hb(1.0) == 0x3C00 and hb(0.5) == 0x3800 and hb(-2.0) == 0xC000
    assert hb(65504.0) == 0x7BFF and hb(1e6) == 0x7BFF and hb(-1e6) == 0xFBFF
    assert hb(1e-8) == 0 and hb(-1e-8) == 0x8000


# ------------------------------------------------------------ fp16 ----

def test_half_to_single_all_patterns(orc):
    """tests/Needle.Tests/MatMulTests.cs:88-101: every finite pattern decodes
    per IEEE 754 (numpy's binary16 is the independent decoder); zeros give
    +0; exponent-31 patterns follow the reference's integer formula."""
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([orc.lib().or_half_to_single(int(b)) for b in bits], dtype=np.float32)
    ieee = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    mag = bits & 0x7FFF
    finite = mag < 0x7C00
    assert np.array_equal(got[finite].view(np.uint32)[mag[finite] != 0], ieee[finite].view(np.uint32)[mag[finite] != 0])
    assert np.all(got[mag == 0].view(np.uint32) == 0)
    quirk = (((mag << 13) + 0x38000000) | ((bits & 0x8000) << 16)).astype(np.uint32).view(np.float32)
    assert np.array_equal(got[~finite].view(np.uint32), quirk[~finite].view(np.uint32))


def test_half_to_single_upstream_subnormals(orc):
    """tests/Needle.Tests/MatMulTests.cs:103-113."""
    for b in range(1, 0x400):
        for sign in (0, 0x8000):
            want = np.float32((-1.0 if sign else 1.0) * (0x0400 + b)) * np.float32(2.9802322e-8)
            assert orc.lib().or_half_to_single_upstream(b | sign) == want


def test_single_to_half_rne_matches_numpy(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 3000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.9, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, np.inf, -np.inf],
                 dtype=np.float32)])
    got = np.array([orc.lib().or_single_to_half_rne(float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------- codebook --

@pytest.mark.parametrize("count", [4, 16])
def test_codebook_fill_closed_form(orc, count):
    rng = np.random.default_rng(count)
    levels = ((np.arange(count) - (count - 1) / 2) * 0.4 + (rng.random(count) - 0.5) * 0.1).astype(np.float32)
    book = orc.codebook(levels, count)
    bs = np.float32(np.max(np.abs(levels))) / np.float32(63.0)
    assert book.byte_scale == bs
    want = np.zeros(32, dtype=np.uint8)
    for i in range(32):
        if i % 16 < count:
            want[i] = int(np.rint(np.float32(levels[i % 16]) / bs) + np.float32(63))
    assert list(book.bytes) == list(want)
    assert max(book.bytes) <= 126
    assert list(book.levels) == [float(levels[i % count]) for i in range(16)]


def test_codebook_bytes_in_range_known_answer(orc):
    levels = ((np.arange(16) - 7.5) * 0.4).astype(np.float32)
    book = orc.codebook(levels, 16)
    spec = GOLDEN["codebook_bytes_range"]
    assert min(book.bytes) >= spec["min"] and max(book.bytes) <= spec["max"]


# ---------------------------------------------------------- hadamard --

def test_hadamard_is_the_sylvester_transform(orc):
    rng = np.random.default_rng(7)
    x = (rng.random(128) - 0.5).astype(np.float32)
    out = np.zeros(128, dtype=np.float32)
    orc.lib().or_hadamard(orc.p(x), orc.p(out))
    ref = scipy.linalg.hadamard(128) @ x.astype(np.float64) / np.sqrt(128.0)
    assert np.max(np.abs(out - ref)) < 1e-6
    back = np.zeros(128, dtype=np.float32)
    orc.lib().or_hadamard(orc.p(out), orc.p(back))
    assert np.max(np.abs(back - x)) < 1e-5
    assert abs(np.sum(out.astype(np.float64) ** 2) - np.sum(x.astype(np.float64) ** 2)) < 1e-4


# ---------------------------------------------------------- quantize --

def test_quantize_int8_golden(orc):
    g = GOLDEN["quantize_int8_neg4_0_4"]
    x = np.array(g["input"], dtype=np.float32)
    q = np.zeros(8, dtype=np.int8)
    s = orc.lib().or_quantize_int8(orc.p(x), 8, orc.p(q))
    assert abs(s - g["expected_scale"]) <= g["scale_tolerance"]
    assert list(q) == g["expected_values"]


def test_round_trip_ties(orc):
    g = GOLDEN["round_trip_ties"]
    x = np.array(g["input"], dtype=np.float32)
    orc.lib().or_round_trip(orc.p(x), len(x), 1.0, 1.0)
    assert list(x) == g["expected"]
    f = GOLDEN["fake_a8_ties"]
    x = np.array(f["input"], dtype=np.float32)
    orc.lib().or_round_trip(orc.p(x), 2, 1.0, 1.0)
    assert list(x) == f["expected"]


def test_quantize_int8_matches_numpy_rule(orc):
    rng = np.random.default_rng(3)
    for n in (8, 48, 64, 128, 1024):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        x[::7] = 0
        q = np.zeros(n, dtype=np.int8)
        s = orc.lib().or_quantize_int8(orc.p(x), n, orc.p(q))
        peak = np.max(np.abs(x))
        want_s = peak / np.float32(127.0)
        assert s == want_s
        inv = np.float32(1.0) / want_s
        want = np.clip(np.rint(x * inv), -128, 127).astype(np.int8)
        assert np.array_equal(q, want)
    z = np.zeros(16, dtype=np.float32)
    q = np.ones(16, dtype=np.int8)
    assert orc.lib().or_quantize_int8(orc.p(z), 16, orc.p(q)) == 1.0 and not q.any()


def test_prepare_zero_input_golden(orc):
    g = GOLDEN["prepare_zero_input"]
    x = np.zeros(g["tokens"] * g["cols"], dtype=np.float32)
    act, values, scales, offsets = orc.prepare(x, g["tokens"], g["cols"], g["bits"])
    stride = act.stride
    for t in range(g["tokens"]):
        assert scales[t * stride] == g["expected_scale"] and offsets[t * stride] == g["expected_offset"]
    assert not values.any()


def _natural_q(orc, x, tokens, cols):
    """Hadamard + QuantizeInt8 per group in natural element order."""
    q = np.zeros((tokens, cols), dtype=np.int8)
    rot = np.zeros(128, dtype=np.float32)
    for t in range(tokens):
        for g in range(cols // 128):
            src = np.ascontiguousarray(x[t, g * 128:(g + 1) * 128])
            orc.lib().or_hadamard(orc.p(src), orc.p(rot))
            dst = np.zeros(128, dtype=np.int8)
            orc.lib().or_quantize_int8(orc.p(rot), 128, orc.p(dst))
            q[t, g * 128:(g + 1) * 128] = dst
    return q


def _natural_indices(indices, rows, cols, bits):
    """Per element index of Scalar.DecodeRow (Scalar.cs:130-144), natural order."""
    rb = cols * bits // 8
    ind = indices.reshape(rows, rb).astype(np.int64)
    i = np.arange(cols)
    g, e = i // 128, i % 128
    if bits == 2:
        return (ind[:, g * 32 + e // 4] >> (2 * (e % 4))) & 3
    return (ind[:, g * 64 + e // 2] >> (4 * (e % 2))) & 15


def _cq_case(orc, seed, rows, cols, bits, tokens):
    rng = np.random.default_rng(seed)
    count = 4 if bits == 2 else 16
    levels = ((np.arange(count) - (count - 1) / 2) * 0.4 + (rng.random(count) - 0.5) * 0.1).astype(np.float32)
    book = orc.codebook(levels, count)
    indices = rng.integers(0, 256, rows * cols * bits // 8, dtype=np.uint8)
    norms = np.array([orc.lib().or_single_to_half_rne(float(v)) for v in 0.2 + rng.random(rows * cols // 128) * 1.8],
                     dtype=np.uint16)
    norms[::11] = 0
    cq = orc.Cq(orc.p(indices), orc.p(norms), C.pointer(book), rows, cols, bits)
    x = ((rng.random((tokens, cols)) - 0.5) * (1 + np.arange(tokens * cols).reshape(tokens, cols) % 7)).astype(np.float32)
    act, values, scales, offsets = orc.prepare(x, tokens, cols, bits)
    return cq, book, indices, norms, x, act, values, scales, offsets


@pytest.mark.parametrize("bits", [2, 4])
def test_prepare_planes_and_group_dots_against_decode_row_order(orc, bits):
    """Planes (Scalar.cs:91-111) + the MatMulRows dot (Scalar.cs:162-184) must
    equal sum_i Bytes[idx(i)] * q_i with idx(i) in DecodeRow's natural order
    (Scalar.cs:140-142) and q from Hadamard + QuantizeInt8 in natural order;
    offsets are 63 * sum(q)."""
    rows, cols, tokens = 7, 384, 3
    cq, book, indices, norms, x, act, values, scales, offsets = _cq_case(orc, bits, rows, cols, bits, tokens)
    qn = _natural_q(orc, x, tokens, cols).astype(np.int64)
    table = np.array(list(book.bytes), dtype=np.int64)
    wbytes = table[_natural_indices(indices, rows, cols, bits)]  # [rows][cols]
    want = np.einsum("nge,tge->tng", wbytes.reshape(rows, cols // 128, 128), qn.reshape(tokens, cols // 128, 128))
    got = orc.group_dots_cq(cq, act, tokens, 0, rows)
    assert np.array_equal(got, want)
    assert np.all(np.abs(got) <= 126 * 128 * 128)
    for t in range(tokens):
        for g in range(cols // 128):
            assert offsets[t * act.stride + g] == np.float32(63.0) * np.float32(qn[t, g * 128:(g + 1) * 128].sum())


@pytest.mark.parametrize("bits", [2, 4])
def test_matmul_rows_cq_epilogue_and_untouched_rows(orc, bits):
    rows, cols, tokens = 13, 768, 5
    cq, book, indices, norms, x, act, values, scales, offsets = _cq_case(orc, 10 + bits, rows, cols, bits, tokens)
    ldy = rows + 3
    y = np.full(tokens * ldy, 12345.0, dtype=np.float32)
    orc.matmul_rows(cq, act, tokens, y, ldy, 2, 11)
    y = y.reshape(tokens, ldy)
    assert np.all(y[:, :2] == 12345.0) and np.all(y[:, 11:] == 12345.0)
    dots = orc.group_dots_cq(cq, act, tokens, 0, rows).astype(np.float64)
    hs = orc.half_to_single_array(norms.reshape(rows, cols // 128)).astype(np.float64)
    sc = scales.reshape(tokens, act.stride)[:, :cols // 128].astype(np.float64)
    off = offsets.reshape(tokens, act.stride)[:, :cols // 128].astype(np.float64)
    scaled = hs[None, :, :] * book.byte_scale * sc[:, None, :]
    want = (scaled * dots).sum(-1) - (scaled * off[:, None, :]).sum(-1)
    mag = max(1.0, np.max(np.abs(want)))
    assert np.max(np.abs(y[:, 2:11] - want[:, 2:11])) < 1e-5 * mag


@pytest.mark.parametrize("tokens,rows,cols", [(1, 64, 1024), (3, 40, 2048), (16, 17, 256)])
def test_matmul_rows_i8_against_int64_and_float64(orc, tokens, rows, cols):
    rng = np.random.default_rng(tokens * 100 + rows)
    w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    scales = np.array([orc.lib().or_single_to_half_rne(float(v)) for v in rng.uniform(0.002, 0.02, rows * cols // 32)],
                      dtype=np.uint16).reshape(rows, cols // 32)
    x = rng.standard_normal((tokens, cols)).astype(np.float32)
    q, qs = orc.quantize_rows(x)
    dots = orc.group_dots_i8(w, q, tokens, 0, rows)
    want_dots = np.einsum("ngk,tgk->tng", w.astype(np.int64).reshape(rows, cols // 32, 32),
                          q.astype(np.int64).reshape(tokens, cols // 32, 32))
    assert np.array_equal(dots, want_dots)
    y = np.full((tokens, rows), 7.0, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, y, rows, 0, rows)
    hs = scales.astype(np.uint16).view(np.float16).astype(np.float64)
    want = np.einsum("ng,tng->tn", hs, want_dots.astype(np.float64)) * qs.astype(np.float64)[:, None]
    rms = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(y - want)) <= 1e-5 * rms
    # dequantised cross-check: y ~ (w * scale) @ (q * qscale)
    deq = (w.astype(np.float64).reshape(rows, cols // 32, 32) * hs[:, :, None]).reshape(rows, cols)
    assert np.max(np.abs(y - (q.astype(np.float64) * qs[:, None]) @ deq.T)) <= 1e-5 * rms


# ----------------------------------------------------------- softmax --

def test_softmax_goldens(orc):
    for key in ("softmax_0_0_0", "softmax_1_2_3"):
        g = GOLDEN[key]
        for poly in (0, 1):
            s = np.array(g["input"], dtype=np.float32)
            orc.lib().or_softmax(orc.p(s), len(s), poly)
            assert np.max(np.abs(s - np.array(g["expected"], dtype=np.float32))) <= g["tolerance"]


def test_exp_poly_against_exp(orc):
    xs = np.linspace(-87.0, 0.0, 20001, dtype=np.float32)
    got = np.array([orc.lib().or_exp_poly(float(v)) for v in xs], dtype=np.float64)
    ref = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 3e-7
    assert orc.lib().or_exp_poly(0.0) == 1.0


def test_exp_poly_clamps_like_avx_max_min(orc):
    """Ops.Exp clamps with Avx.Min(Avx.Max(x, -87.3), 88.7) (src/Needle/Ops.cs:18):
    MAXPS returns its second operand when the first is NaN, so a NaN argument
    (e.g. -inf - -inf) is exp(-87.3), and +-inf land on the clamp bounds.  At
    88.7 the power-of-two scale 2^128 overflows to +inf, as in the reference."""
    e = orc.lib().or_exp_poly
    lo, hi = e(-87.3), e(88.7)
    assert 1.17e-38 < lo < 1.3e-38 and hi == float("inf")
    assert e(float("nan")) == lo
    assert e(float("-inf")) == lo and e(-1e30) == lo
    assert e(float("inf")) == hi and e(1e30) == hi


# --------------------------------------------------------- attention --

def _attention_inputs(seed, positions, kv_heads, heads, qk):
    rng = np.random.default_rng(seed)
    queries = rng.integers(-128, 128, heads * qk, dtype=np.int8)
    keys = rng.integers(-128, 128, positions * kv_heads * qk, dtype=np.int8)
    values = rng.integers(-128, 128, positions * kv_heads * 64, dtype=np.int8)
    qs = (0.4 + 0.1 * np.arange(heads)).astype(np.float32)
    ks = (0.0004 * (1 + rng.integers(0, 4, positions * kv_heads))).astype(np.float32)
    vs = (0.003 * (1 + rng.integers(0, 4, positions * kv_heads))).astype(np.float32)
    return queries, keys, values, qs, ks, vs


@pytest.mark.parametrize("qk", [48, 64])
def test_attention_head_against_float64(orc, qk):
    positions, kv = 45, 2
    queries, keys, values, qs, ks, vs = _attention_inputs(qk, positions, kv, 1, qk)
    k = kv - 1
    first, count = 3, 40
    scores = np.zeros(count + 8, dtype=np.float32)
    out = np.zeros(64, dtype=np.float32)
    probs = np.zeros(positions, dtype=np.float32)
    orc.lib().or_attention_head(orc.p(queries), float(qs[0]), orc.p(keys[k * qk:]), orc.p(ks[k:]),
                                orc.p(values[k * 64:]), orc.p(vs[k:]), kv * qk, kv * 64, kv, first,
                                first + count - 1, orc.p(scores), orc.p(out), orc.p(probs), qk, 0)
    K = keys.reshape(positions, kv, qk)[first:first + count, k].astype(np.float64)
    V = values.reshape(positions, kv, 64)[first:first + count, k].astype(np.float64)
    ksv = ks.reshape(positions, kv)[first:first + count, k].astype(np.float64)
    vsv = vs.reshape(positions, kv)[first:first + count, k].astype(np.float64)
    sc = (K @ queries.astype(np.float64)) * ksv * float(qs[0]) / np.sqrt(qk)
    p = np.exp(sc - sc.max())
    p /= p.sum()
    want = (p * vsv) @ V
    peak = np.max(np.abs(want))
    assert np.max(np.abs(out - want)) <= 1e-5 * peak
    assert np.max(np.abs(probs[first:first + count] - p)) <= 1e-6


@pytest.mark.parametrize("pieces", [2, 3])
def test_split_partials_merge_to_whole(orc, pieces):
    """tests/Needle.Tests/KernelTests.cs:242-282."""
    g = GOLDEN["attention_split_merge_tolerance"]
    positions, heads = g["positions"], g["heads"]
    queries, keys, values, qs, ks, vs = _attention_inputs(pieces, positions, 1, heads, 48)
    PF = 6 * 64 + 16
    whole = np.zeros(heads * 64, dtype=np.float32)
    scores = np.zeros(positions + 8, dtype=np.float32)
    for h in range(heads):
        o = np.zeros(64, dtype=np.float32)
        orc.lib().or_attention_head(orc.p(np.ascontiguousarray(queries[h * 48:(h + 1) * 48])), float(qs[h]),
                                    orc.p(keys), orc.p(ks), orc.p(values), orc.p(vs), 48, 64, 1, 0, positions - 1,
                                    orc.p(scores), orc.p(o), None, 48, 1)
        whole[h * 64:(h + 1) * 64] = o
    partials = np.zeros(pieces * PF, dtype=np.float32)
    length = (positions + pieces - 1) // pieces
    for piece in range(pieces):
        begin = piece * length
        count = min(length, positions - begin)
        for h in range(heads):
            o = np.zeros(64, dtype=np.float32)
            pk, sm = C.c_float(), C.c_float()
            orc.lib().or_attention_partial(orc.p(np.ascontiguousarray(queries[h * 48:(h + 1) * 48])), float(qs[h]),
                                           orc.p(keys), orc.p(ks), orc.p(values), orc.p(vs), 48, 64, 1, begin, count,
                                           48, 1, orc.p(o), C.byref(pk), C.byref(sm))
            partials[piece * PF + h * 64: piece * PF + (h + 1) * 64] = o
            partials[piece * PF + 384 + h] = pk.value
            partials[piece * PF + 392 + h] = sm.value
    merged = np.zeros(heads * 64, dtype=np.float32)
    orc.lib().or_merge_partials(orc.p(partials), pieces, heads, orc.p(merged), 1)
    peak = np.max(np.abs(whole))
    assert np.max(np.abs(merged - whole)) <= g["relative_to_peak"] * peak
    ref = np.zeros(heads * 64, dtype=np.float32)
    orc.lib().or_merge_partials_double(orc.p(partials), pieces, heads, orc.p(ref))
    merged_libm = np.zeros(heads * 64, dtype=np.float32)
    orc.lib().or_merge_partials(orc.p(partials), pieces, heads, orc.p(merged_libm), 0)
    assert np.max(np.abs(merged_libm - ref)) <= 1e-6 * max(1.0, np.max(np.abs(ref)))


def test_attention_plan_known_values_and_invariants(orc):
    """AttentionBatch.ExecuteChunk's split (src/Needle/Blocks.cs:934-938)."""
    assert orc.attention_plan(2048, 8) == (8, 256)
    assert orc.attention_plan(40, 8) == (2, 20)
    assert orc.attention_plan(17, 8) == (1, 20)
    assert orc.attention_plan(33, 8) == (2, 20)
    assert orc.attention_plan(1, 8) == (1, 4)
    for count in range(1, 3000, 7):
        for cap in (1, 8, 64):
            chunks, length = orc.attention_plan(count, cap)
            assert length % 4 == 0 and 1 <= chunks <= cap
            assert (chunks - 1) * length < count <= chunks * length


@pytest.mark.parametrize("count", [1, 2, 3, 5, 8])
def test_merge_head_equals_merge_partials(orc, count):
    """The any-count merge keeps MergePartials' arithmetic for counts <= 8."""
    st = orc.state(77 + count)
    PF, heads = 6 * 64 + 16, 3
    partials = np.zeros(count * PF, dtype=np.float32)
    for c in range(count):
        partials[c * PF:c * PF + heads * 64] = orc.synth_normal(st, heads * 64)
        partials[c * PF + 384:c * PF + 384 + heads] = orc.synth_normal(st, heads) * 3
        partials[c * PF + 392:c * PF + 392 + heads] = np.abs(orc.synth_normal(st, heads)) * 10 + 1
    want = np.zeros(heads * 64, dtype=np.float32)
    orc.lib().or_merge_partials(orc.p(partials), count, heads, orc.p(want), 1)
    for h in range(heads):
        got = np.zeros(64, dtype=np.float32)
        orc.lib().or_merge_head(orc.p(partials[h * 64:]), PF, orc.p(partials[384 + h:]), orc.p(partials[392 + h:]),
                                PF, count, orc.p(got), 1)
        assert np.array_equal(got.view(np.uint32), want[h * 64:(h + 1) * 64].view(np.uint32))


@pytest.mark.parametrize("heads,kv_heads,qk,max_chunks", [(4, 4, 64, 8), (6, 2, 48, 64), (4, 1, 64, 1)])
def test_attention_decode_against_float64(orc, heads, kv_heads, qk, max_chunks):
    """Ragged decode attention: softmax((q.k) * scales / sqrt(qk)) . v in
    float64 from the same int8 values, per row of a pooled cache."""
    st = orc.state(heads * 100 + qk + max_chunks)
    slots, capacity = 3, 300
    keys, ks, values, vs = orc.kv_cache(st, slots, capacity, kv_heads, qk)
    rows = 5
    row_slot = np.array([0, 2, 1, 2, 0], dtype=np.int32)
    row_first = np.array([0, 10, 0, 250, 3], dtype=np.int32)
    row_count = np.array([1, 37, 300, 50, 129], dtype=np.int32)
    qf = orc.synth_normal(st, rows * heads * qk).reshape(rows * heads, qk)
    q, qs = orc.quantize_rows(qf)
    out = orc.attention_decode(q, qs, heads, kv_heads, qk, keys, ks, values, vs, capacity, row_slot, row_first,
                               row_count, max_chunks)
    group = heads // kv_heads
    for r in range(rows):
        sl, f, n = row_slot[r], row_first[r], row_count[r]
        for h in range(heads):
            kv = h // group
            K = keys[sl, f:f + n, kv * qk:(kv + 1) * qk].astype(np.float64)
            V = values[sl, f:f + n, kv * 64:(kv + 1) * 64].astype(np.float64)
            dots = K @ q[r * heads + h].astype(np.float64)
            sc = dots * ks[sl, f:f + n, kv] * qs[r * heads + h] / np.sqrt(qk)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            want = (p * vs[sl, f:f + n, kv]) @ V
            assert np.max(np.abs(out[r, h] - want)) <= 2e-5 * max(1e-3, np.max(np.abs(want)))


def test_attention_span(orc):
    f, c = C.c_int(), C.c_int()
    for pos, window, frames, want in [(10, 0, 0, (0, 11)), (10, 4, 0, (7, 4)), (2, 4, 0, (0, 3)),
                                      (5, 0, 9, (0, 9)), (0, 0, 0, (0, 1))]:
        orc.lib().or_attention_span(pos, window, frames, C.byref(f), C.byref(c))
        assert (f.value, c.value) == want


# --------------------------------------------------------- selection --

def test_argmax_first_index(orc):
    x = np.array([1, 5, 3, 5, -2], dtype=np.float32)
    assert orc.lib().or_argmax(orc.p(x), 5) == 1
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = rng.integers(-5, 5, 300).astype(np.float32)
        assert orc.lib().or_argmax(orc.p(x), 300) == int(np.argmax(x))


def test_argmax_special_values(orc):
    """Ops.ArgMax's scalar loop (src/Needle/Ops.cs:1086-1089): NaN-free rows
    give numpy's argmax (first index of the maximum; +0 and -0 equal; all
    -inf gives 0); a NaN at id 0 gives 0, NaN elsewhere is skipped
    (np.nanargmax)."""
    f = orc.lib().or_argmax
    inf, nan = np.inf, np.nan
    cases = [([-inf, -inf, -inf], 0), ([-0.0, 0.0, -0.0], 0), ([0.0, -0.0, 1e-45], 2), ([nan, 5.0, 7.0], 0),
             ([1.0, nan, 3.0, 3.0], 2), ([-inf, nan, -inf], 0), ([2.0, inf, inf, nan], 1), ([7.0], 0)]
    for vals, want in cases:
        x = np.array(vals, dtype=np.float32)
        assert f(orc.p(x), len(x)) == want, vals
    rng = np.random.default_rng(6)
    for _ in range(50):
        n = int(rng.integers(1, 3000))
        x = rng.integers(-4, 4, n).astype(np.float32)
        x[rng.random(n) < 0.05] = -inf
        assert f(orc.p(x), n) == int(np.argmax(x))
        x[1 + rng.integers(0, n, 3) % max(n - 1, 1)] = nan
        if n > 1:
            assert f(orc.p(x), n) == int(np.nanargmax(x))


def topk_select(orc, vals, k, mask=1):
    x = np.array(vals, dtype=np.float32)
    idx = np.zeros(k, dtype=np.int32)
    val = np.zeros(k, dtype=np.float32)
    orc.lib().or_topk_select(orc.p(x), len(x), k, mask, orc.p(idx), orc.p(val))
    return list(idx), list(val)


def test_topk_select_fewer_values_than_k(orc):
    """Known answers traced by hand through Ops.TopKLogSoftmax's selection
    loop (src/Needle/Ops.cs:1094-1166): slots start (-inf, -1), min = (-inf,
    INT_MAX); with the mask id 1 is put in slot 0 (and becomes the minimum
    only when k == 1) and the scan starts at id 4; a value enters when v >
    min or (v == min and id < min id), then min = the last slot."""
    inf = np.inf
    # x[4] = -inf enters first (-inf == min, 4 < INT_MAX) into the last slot;
    # 5 and 6 (-inf, ids above 4) never enter
    assert topk_select(orc, [0, 1, 0, 0, -inf, -inf, -inf], 3)[0] == [1, -1, 4]
    # the finite x[5] enters after x[4] and pushes it out of the last slot
    assert topk_select(orc, [0, 1, 0, 0, -inf, 2, -inf], 3)[0] == [5, 1, -1]
    # x[1] = -inf stays in slot 0 until a larger value moves it down
    assert topk_select(orc, [0, -inf, 0, 0, -inf, -inf], 2)[0] == [1, 4]
    assert topk_select(orc, [0, -inf, 0, 0, 3, -inf], 3)[0] == [4, 1, -1]
    # k == 1: min starts at (x[1], 1): -inf ids never enter
    assert topk_select(orc, [0, -inf, 0, 0, -inf, -inf], 1)[0] == [1]
    # n == 1 with the mask: id 0 is masked, nothing is selected
    assert topk_select(orc, [5.0], 2)[0] == [-1, -1]
    # without the mask the first value enters at -inf, later ones do not
    assert topk_select(orc, [-inf, -inf, -inf], 2, mask=0)[0] == [-1, 0]
    assert topk_select(orc, [-inf, 4.0, -inf], 3, mask=0)[0] == [1, -1, -1]


def test_topk_select_against_brute_force(orc):
    """With at least k values above -inf among the allowed ids, the
    selection is the k first allowed ids by (larger value, then lower id)."""
    rng = np.random.default_rng(17)
    for trial in range(200):
        n = int(rng.integers(12, 400))
        k = int(rng.integers(1, 9))
        mask = trial % 2
        x = rng.integers(-6, 6, n).astype(np.float32)
        x[rng.random(n) < 0.3] = -np.inf
        allowed = [i for i in range(n) if not (mask and i in (0, 2, 3))]
        finite = [i for i in allowed if x[i] > -np.inf]
        if len(finite) < k:
            continue
        want = sorted(finite, key=lambda i: (-float(x[i]), i))[:k]
        assert topk_select(orc, x, k, mask)[0] == want, trial


def test_zero_centered_rms_against_float64(orc):
    """Ops.ZeroCenteredRms (src/Needle/Ops.cs:209, 233-244): (1 + scale) * x /
    sqrt(mean(x^2) + 1e-6), within a few float32 roundings of float64."""
    rng = np.random.default_rng(21)
    for n in (48, 64, 7):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        sc = (rng.standard_normal(n) * 0.2).astype(np.float32)
        out = np.zeros(n, np.float32)
        orc.lib().or_zero_centered_rms(orc.p(x), orc.p(sc), n, orc.p(out))
        x64 = x.astype(np.float64)
        want = (1 + sc.astype(np.float64)) * x64 / np.sqrt(np.mean(x64 * x64) + 1e-6)
        assert np.max(np.abs(out - want)) <= 4e-7 * np.max(np.abs(want))


def test_rope_rotate_is_a_rotation(orc):
    """Scalar.Rope (src/Needle/Scalar.cs:233-248): pairs (i, i + n/2) rotate by
    the table's angle (float64 check), and the pair norms are kept."""
    rng = np.random.default_rng(22)
    n = 48
    x = rng.standard_normal(n).astype(np.float32)
    ang = rng.uniform(0, 6.3, n // 2)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = x.copy()
    orc.lib().or_rope_rotate(orc.p(y), n, orc.p(cs), orc.p(sn))
    z = (x[:24] + 1j * x[24:]).astype(np.complex128) * (cs.astype(np.float64) + 1j * sn.astype(np.float64))
    assert np.allclose(y[:24], z.real, atol=1e-6) and np.allclose(y[24:], z.imag, atol=1e-6)
    assert np.allclose(np.hypot(y[:24], y[24:]), np.hypot(x[:24], x[24:]), rtol=1e-5)


def test_needle3_attention_inputs_against_float64(orc):
    """The row step (src/Needle/Engine.cs:1302-1387): taps over the history,
    norm, rotation and per-head quantization match a float64 computation to
    one int8 step, and the history moves on one frame."""
    rng = np.random.default_rng(23)
    heads, kv, qk, vd, slots, cap = 4, 2, 48, 64, 2, 8
    qw, kw, vw = heads * qk, kv * qk, kv * vd
    allw = qw + kw + vw
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    taps = [f(3, qw), f(3, kw), f(3, vw)]
    qn, kn = f(qk) * 0.1, f(qk) * 0.1
    ang = rng.uniform(0, 6.3, (cap, qk // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    hist = f(slots, 2 * allw)
    raw = f(1, allw)
    q = np.zeros((1, qw), np.int8)
    qs = np.zeros((1, heads), np.float32)
    keys, values = np.zeros((slots, cap, kw), np.int8), np.zeros((slots, cap, vw), np.int8)
    ks, vs = np.zeros((slots, cap, kv), np.float32), np.zeros((slots, cap, kv), np.float32)
    h0 = hist.copy()
    rsl, rps = np.array([1], np.int32), np.array([3], np.int32)
    orc.lib().or_needle3_attention_inputs(orc.p(raw), 1, heads, kv, qk, vd, orc.p(taps[0]), orc.p(taps[1]),
                                          orc.p(taps[2]), orc.p(qn), orc.p(kn), orc.p(cs), orc.p(sn), orc.p(hist),
                                          orc.p(rsl), orc.p(rps), slots, cap, orc.p(q), orc.p(qs), orc.p(keys),
                                          orc.p(ks), orc.p(values), orc.p(vs))
    d = lambda a: a.astype(np.float64)
    hs = d(h0[1])
    def conv(part_base, W, t):
        f0, f1 = hs[2 * part_base:2 * part_base + W], hs[2 * part_base + W:2 * part_base + 2 * W]
        cur = d(raw[0, part_base:part_base + W])
        return d(t[0]) * cur + d(t[1]) * f1 + d(t[2]) * f0
    def norm_rope(x, sc):
        y = (1 + d(sc)) * x / np.sqrt(np.mean(x * x) + 1e-6)
        a, b = y[:qk // 2], y[qk // 2:]
        c_, s_ = d(cs[3]), d(sn[3])
        return np.concatenate([a * c_ - b * s_, b * c_ + a * s_])
    def check(x, qv, scale):
        want = np.clip(np.round(x / (np.max(np.abs(x)) / 127)), -128, 127)
        assert np.max(np.abs(qv.astype(np.int32) - want)) <= 1
        assert abs(scale - np.max(np.abs(x)) / 127) <= 1e-5 * abs(scale)
    cq = conv(0, qw, taps[0])
    for h in range(heads):
        check(norm_rope(cq[h * qk:(h + 1) * qk], qn), q[0, h * qk:(h + 1) * qk], qs[0, h])
    ck = conv(qw, kw, taps[1])
    for h in range(kv):
        check(norm_rope(ck[h * qk:(h + 1) * qk], kn), keys[1, 3, h * qk:(h + 1) * qk], ks[1, 3, h])
    cv = conv(qw + kw, vw, taps[2])
    for h in range(kv):
        check(cv[h * vd:(h + 1) * vd], values[1, 3, h * vd:(h + 1) * vd], vs[1, 3, h])
    new = hist[1]
    for base, W in ((0, qw), (qw, kw), (qw + kw, vw)):
        assert np.array_equal(new[2 * base:2 * base + W], h0[1, 2 * base + W:2 * base + 2 * W])
        assert np.array_equal(new[2 * base + W:2 * base + 2 * W], raw[0, base:base + W])
    assert np.array_equal(hist[0], h0[0])


def masked_argmax_brute(x, mask, words, length):
    """The largest allowed value that exceeds -inf (NaN never does), then its
    lowest id: the closed form of Ops.ArgMaxMaskedScalar's ascending scan."""
    ids = [w * 32 + b for w in range(words) for b in range(32) if (int(mask[w]) >> b) & 1]
    ids = [i for i in ids if i < length and x[i] > -np.inf]
    if not ids:
        return -1
    peak = max(x[i] for i in ids)
    return min(i for i in ids if x[i] == peak)


def test_argmax_masked_cases(orc):
    """src/Needle/Ops.cs:1236-1266: ties to the first id, +0 and -0 tie, NaN
    and -inf never win, ids past length and cleared bits are skipped, an
    empty selection gives -1."""
    f = orc.lib().or_argmax_masked
    x = np.array([1, 7, 7, 3, -0.0, 0.0, np.nan, -np.inf] + [0] * 56, dtype=np.float32)
    m = np.array([0xFFFFFFFF, 0xFFFFFFFF], dtype=np.uint32)
    assert f(orc.p(x), orc.p(m), 2, 8) == 1
    m = np.array([0b11110000, 0], dtype=np.uint32)   # -0, +0, NaN, -inf
    assert f(orc.p(x), orc.p(m), 2, 8) == 4
    m = np.array([0b11000000, 0], dtype=np.uint32)   # NaN, -inf only
    assert f(orc.p(x), orc.p(m), 2, 8) == -1
    m = np.array([0b1000, 0], dtype=np.uint32)
    assert f(orc.p(x), orc.p(m), 2, 3) == -1           # id 3 >= length
    assert f(orc.p(x), orc.p(np.zeros(2, dtype=np.uint32)), 2, 64) == -1
    y = np.full(64, -np.inf, dtype=np.float32)
    y[40] = np.inf
    m = np.array([0, 1 << 8], dtype=np.uint32)
    assert f(orc.p(y), orc.p(m), 2, 64) == 40


def test_argmax_masked_against_brute_force(orc):
    rng = np.random.default_rng(77)
    for trial in range(200):
        n = int(rng.integers(1, 300))
        words = (n + 31) // 32 + int(rng.integers(0, 2))
        x = rng.integers(-4, 4, words * 32).astype(np.float32)
        x[rng.random(x.size) < 0.05] = np.nan
        x[rng.random(x.size) < 0.05] = -np.inf
        density = [0.0, 0.01, 0.2, 1.0][trial % 4]
        bits = rng.random(words * 32) < density
        mask = np.packbits(bits.reshape(words, 32)[:, ::-1], axis=1).view(">u4").reshape(words).astype(np.uint32)
        got = orc.lib().or_argmax_masked(orc.p(x), orc.p(mask), words, n)
        assert got == masked_argmax_brute(x, mask, words, n), trial


@pytest.mark.parametrize("mask", [0, 1])
def test_topk_log_softmax_against_numpy(orc, mask):
    rng = np.random.default_rng(11 + mask)
    for n in (5, 40, 1000):
        x = rng.integers(-20, 20, n).astype(np.float32) * np.float32(0.25)
        k = 3
        idx = np.zeros(k, dtype=np.int32)
        lp = np.zeros(k, dtype=np.float32)
        pr = np.zeros(k, dtype=np.float32)
        orc.lib().or_topk_log_softmax(orc.p(x), n, k, orc.p(idx), orc.p(lp), orc.p(pr), mask)
        xm = x.astype(np.float64).copy()
        if mask:
            xm[[0, 2, 3]] = -1e30
        # masked ids 0, 2, 3 are never candidates (Ops.cs:1101-1107,1167); a
        # short candidate list keeps index -1 in the tail slots
        cand = [i for i in range(n) if not (mask and i in (0, 2, 3))]
        order = sorted(cand, key=lambda i: (-xm[i], i))[:k]
        order += [-1] * (k - len(order))
        assert list(idx) == order
        valid = [j for j, i in enumerate(order) if i >= 0]
        lse = np.log(np.sum(np.exp(xm - xm.max()))) + xm.max()
        sel = np.array([order[j] for j in valid])
        assert np.max(np.abs(lp[valid] - (xm[sel] - lse))) <= 2e-6
        assert np.max(np.abs(pr[valid] - np.exp(xm[sel] - lse))) <= 2e-6
