"""GPU parity of the AttentionTile / MergePartials kernel-table entries
against the oracle, at the reference's own conformance bounds
(tests/Needle.Tests/Conformance/KernelConformanceTests.cs:399-565)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

POSITIONS = 45
PF = 6 * 64 + 16


def tile_inputs(orc, kv_heads, heads, first, count, extremes):
    """KernelConformanceTests.cs:415-436."""
    st = orc.state(kv_heads * 1000 + heads * 100 + first * 7 + count * 13 + 0xBEEF)
    lib = orc.lib()
    q = np.zeros(heads * 48, dtype=np.int8)
    k = np.zeros(POSITIONS * kv_heads * 48, dtype=np.int8)
    v = np.zeros(POSITIONS * kv_heads * 64, dtype=np.int8)
    lib.or_fill_sbyte(orc.p(q), q.size, C.byref(st), int(extremes))
    lib.or_fill_sbyte(orc.p(k), k.size, C.byref(st), int(extremes))
    lib.or_fill_sbyte(orc.p(v), v.size, C.byref(st), int(extremes))
    qs = np.array([0.4 + 0.1 * i for i in range(heads)], dtype=np.float32)
    ks = np.zeros(POSITIONS * kv_heads, dtype=np.float32)
    vs = np.zeros(POSITIONS * kv_heads, dtype=np.float32)
    for i in range(POSITIONS * kv_heads):
        ks[i] = np.float32(0.0004) * np.float32(1 + lib.or_xs_next_int(C.byref(st), 0, 4))
        vs[i] = np.float32(0.003) * np.float32(1 + lib.or_xs_next_int(C.byref(st), 0, 4))
    return q, qs, k, ks, v, vs


def make_tile(mod, kv_heads, heads, first, count, arrays, out, probs, peaks=None, sums=None):
    q, qs, k, ks, v, vs = arrays
    kv = kv_heads - 1
    return mod.AttnTile(q.ctypes.data, qs.ctypes.data, heads, k.ctypes.data + kv * 48, ks.ctypes.data + kv * 4,
                        v.ctypes.data + kv * 64, vs.ctypes.data + kv * 4, kv_heads * 48, kv_heads * 64, kv_heads,
                        first, count, None, out.ctypes.data, probs.ctypes.data if probs is not None else None,
                        POSITIONS, peaks.ctypes.data if peaks is not None else None,
                        sums.ctypes.data if sums is not None else None)


@pytest.mark.parametrize("kv_heads,heads,first,count,capture,extremes", [
    (2, 6, 0, 45, True, False), (2, 6, 13, 32, True, False), (2, 6, 41, 4, True, False),
    (8, 1, 0, 45, True, False), (1, 6, 0, 1, False, False), (2, 6, 7, 2, False, False),
    (2, 6, 0, 45, True, True)])
def test_attention_tile_matches_scalar(hip, orc, kv_heads, heads, first, count, capture, extremes):
    arrays = tile_inputs(orc, kv_heads, heads, first, count, extremes)
    want = np.zeros(heads * 64, dtype=np.float32)
    want_p = np.zeros(heads * POSITIONS, dtype=np.float32) if capture else None
    scores = np.zeros(count + 8, dtype=np.float32)
    t = make_tile(orc, kv_heads, heads, first, count, arrays, want, want_p)
    t.scores = scores.ctypes.data
    orc.lib().or_attention_tile_run(C.byref(t), 0)
    got = np.zeros(heads * 64, dtype=np.float32)
    got_p = np.zeros(heads * POSITIONS, dtype=np.float32) if capture else None
    ht = make_tile(hip, kv_heads, heads, first, count, arrays, got, got_p)
    hip.lib().nhip_attention_tile(C.byref(ht))
    assert hip.last_error() == ""
    peak = np.max(np.abs(want))
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) <= 5e-5 * peak
    if capture:
        assert np.max(np.abs(got_p - want_p)) <= 1e-5


def test_attention_tile_partials_merge_to_whole(hip, orc):
    """Position-split partials from the tile entry merged by the merge entry
    equal the whole tile (tests/Needle.Tests/KernelTests.cs:242-282)."""
    kv_heads, heads = 2, 6
    arrays = tile_inputs(orc, kv_heads, heads, 0, POSITIONS, False)
    whole = np.zeros(heads * 64, dtype=np.float32)
    hip.lib().nhip_attention_tile(C.byref(make_tile(hip, kv_heads, heads, 0, POSITIONS, arrays, whole, None)))
    pieces = 3
    length = (POSITIONS + pieces - 1) // pieces
    partials = np.zeros(pieces * PF, dtype=np.float32)
    for piece in range(pieces):
        begin = piece * length
        cnt = min(length, POSITIONS - begin)
        out = np.zeros(heads * 64, dtype=np.float32)
        pk = np.zeros(8, dtype=np.float32)
        sm = np.zeros(8, dtype=np.float32)
        hip.lib().nhip_attention_tile(C.byref(make_tile(hip, kv_heads, heads, begin, cnt, arrays, out, None, pk, sm)))
        partials[piece * PF: piece * PF + heads * 64] = out
        partials[piece * PF + 384: piece * PF + 384 + heads] = pk[:heads]
        partials[piece * PF + 392: piece * PF + 392 + heads] = sm[:heads]
    merged = np.zeros(heads * 64, dtype=np.float32)
    hip.lib().nhip_merge_partials(partials.ctypes.data, pieces, heads, merged.ctypes.data)
    peak = np.max(np.abs(whole))
    assert np.max(np.abs(merged - whole)) <= 3e-5 * peak


@pytest.mark.parametrize("count,heads", [(1, 1), (1, 6), (2, 1), (2, 6), (3, 6)])
def test_merge_partials_matches_double_reference(hip, orc, count, heads):
    """KernelConformanceTests.cs:527-559."""
    st = orc.state(count * 31 + heads * 7 + 0xF001)
    lib = orc.lib()
    partials = np.zeros(count * PF, dtype=np.float32)
    for c in range(count):
        chunk = np.zeros(heads * 64, dtype=np.float32)
        lib.or_fill_edges(orc.p(chunk), heads * 64, C.byref(st), 2.0)
        partials[c * PF: c * PF + heads * 64] = chunk
        for h in range(heads):
            partials[c * PF + 384 + h] = lib.or_xs_next_float(C.byref(st), 2.0)
            partials[c * PF + 392 + h] = np.float32(0.5) + abs(np.float32(lib.or_xs_next_float(C.byref(st), 2.0)))
    want = np.zeros(heads * 64, dtype=np.float32)
    lib.or_merge_partials_double(orc.p(partials), count, heads, orc.p(want))
    got = np.zeros(heads * 64, dtype=np.float32)
    hip.lib().nhip_merge_partials(partials.ctypes.data, count, heads, got.ctypes.data)
    assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, float(np.max(np.abs(want))))
