"""GPU Quant.MatMulBatch (nhip_matmul_batch_dev; src/Needle/Quant.cs:679-816):
up to four weight matrices sharing one activation set, every job's rows in
one launch at decode sizes, each job bit-identical with the oracle's
MatMulRows over all its rows and with the single-matrix entries; columns
past a job's rows (ldy > rows) untouched.  Shapes: Needle 3's Q / K / V /
Gate projections (576, 96, 128, 768 rows x 768, codebook 2- and 4-bit) and
the literal int8 format at K = 2048 (one launch) and K = 768 (the jobs in
turn)."""
import ctypes as C

import numpy as np
import pytest

from test_matmul_gpu import SENTINEL, cq_case, hip_book, int8_case

pytestmark = pytest.mark.gpu

NEEDLE3_QKVG = (576, 96, 128, 768)


def run_batch(hip, handles, rows, q, scales, offsets, stride, tokens, pad=3):
    n = len(handles)
    outs = [hip.DeviceBuffer.from_array(np.full(tokens * (r + pad), SENTINEL, dtype=np.float32)) for r in rows]
    W = (C.c_void_p * n)(*handles)
    Y = (C.c_void_p * n)(*[o.ptr for o in outs])
    L = (C.c_int32 * n)(*[r + pad for r in rows])
    dq = hip.DeviceBuffer.from_array(q)
    ds = hip.DeviceBuffer.from_array(scales)
    do = hip.DeviceBuffer.from_array(offsets) if offsets is not None else None
    hip.check(hip.lib().nhip_matmul_batch_dev(W, n, dq.ptr, ds.ptr, do.ptr if do else None, stride, tokens, Y, L,
                                              None))
    return [o.download(np.float32).reshape(tokens, r + pad) for o, r in zip(outs, rows)]


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("tokens", [1, 3, 4, 7, 12, 16, 40])
@pytest.mark.parametrize("jobs", [4, 1, 3])
def test_codebook_batch_bit_exact(hip, orc, bits, tokens, jobs):
    rows = NEEDLE3_QKVG[:jobs]
    cases = [cq_case(orc, 900 + 10 * j + bits, r, 768, bits, tokens) for j, r in enumerate(rows)]
    act = cases[0]  # one activation set shared by every job
    weights = [hip.Weights.codebook(c["indices"], c["norms"], hip_book(hip, c["book"]), r, 768, bits)
               for c, r in zip(cases, rows)]
    got = run_batch(hip, [w.handle for w in weights], rows, act["values"], act["scales"], act["offsets"],
                    act["act"].stride, tokens)
    for j, (c, r) in enumerate(zip(cases, rows)):
        ldy = r + 3
        want = np.full(tokens * ldy, SENTINEL, dtype=np.float32)
        orc.matmul_rows(c["cq"], act["act"], tokens, want, ldy, 0, r)
        assert np.array_equal(got[j].reshape(-1).view(np.uint32), want.view(np.uint32)), j


@pytest.mark.parametrize("tokens", [1, 3, 16, 20])
@pytest.mark.parametrize("cols,rows", [(2048, (3072, 1024, 8192, 16)), (768, (576, 96, 128, 768))])
def test_int8_batch_bit_exact(hip, orc, tokens, cols, rows):
    cases = [int8_case(orc, 300 + j + cols, r, cols, tokens) for j, r in enumerate(rows)]
    _, _, _, q, qs = cases[0]
    weights = [hip.Weights.int8(w, s) for w, s, _, _, _ in cases]
    got = run_batch(hip, [w.handle for w in weights], rows, q, qs, None, 0, tokens)
    for j, ((w, s, _, _, _), r) in enumerate(zip(cases, rows)):
        ldy = r + 3
        want = np.full((tokens, ldy), SENTINEL, dtype=np.float32)
        orc.matmul_rows_i8(w, s, q, qs, tokens, want, ldy, 0, r)
        assert np.array_equal(got[j].view(np.uint32), want.view(np.uint32)), j


def test_batch_rejects_mismatched_jobs(hip, orc):
    a = int8_case(orc, 1, 64, 256, 2)
    b = int8_case(orc, 2, 64, 512, 2)
    wa, wb = hip.Weights.int8(a[0], a[1]), hip.Weights.int8(b[0], b[1])
    with pytest.raises(RuntimeError, match="K of job 0"):
        run_batch(hip, [wa.handle, wb.handle], (64, 64), a[3], a[4], None, 0, 2)
    with pytest.raises(RuntimeError, match="outside"):
        run_batch(hip, [wa.handle] * 5, (64,) * 5, a[3], a[4], None, 0, 2)
    W = (C.c_void_p * 1)(wa.handle)
    Y = (C.c_void_p * 1)(0)
    L = (C.c_int32 * 1)(10)  # below the 64 rows
    buf = hip.DeviceBuffer(4096)
    assert hip.lib().nhip_matmul_batch_dev(W, 1, buf.ptr, buf.ptr, None, 0, 2, Y, L, None) != 0
