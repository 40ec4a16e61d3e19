"""The kernel-table provider under the reference's calling patterns:
MatMulBatch's pool members calling the MatMulRows slot at once on disjoint
row ranges of one weight view (src/Needle/Quant.cs:725-771), bit-identical
with the oracle; and a model disposed and another mapped at the same host
addresses (nhip_table_release drops the cached device weights, so the new
contents are uploaded instead of reusing the old copy)."""
import ctypes as C
import threading

import numpy as np
import pytest

from test_matmul_gpu import SENTINEL, cq_case, hip_book

pytestmark = pytest.mark.gpu


def views(hip, c, rows, cols, bits):
    book = hip_book(hip, c["book"])
    cq = hip.Cq(c["indices"].ctypes.data, c["norms"].ctypes.data, C.pointer(book), rows, cols, bits)
    a = c["act"]
    act = hip.Activations(a.values, a.scales, a.offsets, a.cols, a.groups, a.stride)
    return book, cq, act


@pytest.mark.parametrize("bits", [2, 4])
def test_concurrent_members_on_disjoint_rows(hip, orc, bits):
    rows, cols, tokens, members = 1000, 768, 3, 8
    c = cq_case(orc, 4400 + bits, rows, cols, bits, tokens)
    book, cq, act = views(hip, c, rows, cols, bits)
    ldy = rows + 1
    got = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
    blocks = (rows + 3) // 4
    errors = []

    def member(m):  # MatMulBatch.RunShard: blocks [m*B/M, (m+1)*B/M) of 4 rows
        r0 = min(rows, (m * blocks // members) * 4)
        r1 = min(rows, ((m + 1) * blocks // members) * 4)
        for _ in range(5):  # several rounds, every member at once
            hip.lib().nhip_matmul_rows(C.byref(cq), C.byref(act), tokens, got.ctypes.data, ldy, r0, r1)
            if hip.last_error():
                errors.append(hip.last_error())

    threads = [threading.Thread(target=member, args=(m,)) for m in range(members)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    want = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
    orc.matmul_rows(c["cq"], c["act"], tokens, want, ldy, 0, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_release_drops_a_disposed_models_weights(hip, orc):
    rows, cols, tokens, bits = 64, 256, 2, 4
    a = cq_case(orc, 4501, rows, cols, bits, tokens)
    b = cq_case(orc, 4502, rows, cols, bits, tokens)
    # one "mapping" whose bytes hold model a's indices, then model b's
    mapping = a["indices"].copy()
    c = dict(a, indices=mapping)
    book, cq, act = views(hip, c, rows, cols, bits)
    ldy = rows

    def run():
        y = np.zeros(tokens * ldy, dtype=np.float32)
        hip.lib().nhip_matmul_rows(C.byref(cq), C.byref(act), tokens, y.ctypes.data, ldy, 0, rows)
        assert hip.last_error() == ""
        return y

    def want():  # the oracle over the mapping's current bytes
        cqo = orc.Cq(orc.p(mapping), orc.p(a["norms"]), C.pointer(a["book"]), rows, cols, bits)
        y = np.zeros(tokens * ldy, dtype=np.float32)
        orc.matmul_rows(cqo, a["act"], tokens, y, ldy, 0, rows)
        return y

    first = want()
    assert np.array_equal(run(), first)
    entries = C.c_int32()
    hip.check(hip.lib().nhip_table_cached(C.byref(entries), None))
    assert entries.value >= 1
    mapping[:] = b["indices"]  # the same addresses, new contents
    released = C.c_int32()
    hip.check(hip.lib().nhip_table_release(mapping.ctypes.data, mapping.nbytes, C.byref(released)))
    assert released.value == 1
    second = want()
    assert not np.array_equal(first, second)
    assert np.array_equal(run(), second)  # uploaded afresh from the new bytes
    hip.check(hip.lib().nhip_table_release(None, 0, None))
    hip.check(hip.lib().nhip_table_cached(C.byref(entries), None))
    assert entries.value == 0


def test_void_entry_failure_sets_last_error(hip, orc):
    """A failed call leaves the output untouched and reports through
    nhip_last_error (the probe a host runs before installing the table)."""
    rows, cols, tokens, bits = 16, 256, 1, 2
    c = cq_case(orc, 4601, rows, cols, bits, tokens)
    book, cq, act = views(hip, c, rows, cols, bits)
    y = np.full(tokens * rows, SENTINEL, dtype=np.float32)
    hip.lib().nhip_matmul_rows(C.byref(cq), C.byref(act), tokens, y.ctypes.data, rows, 0, rows + 5)  # past the rows
    assert "row range" in hip.last_error()
    assert np.all(y == SENTINEL)
    hip.lib().nhip_matmul_rows(C.byref(cq), C.byref(act), tokens, y.ctypes.data, rows, 0, rows)
    assert hip.last_error() == ""
