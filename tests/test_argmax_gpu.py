"""GPU Ops.ArgMax (nhip_argmax_dev; src/Needle/Ops.cs:1052-1090) against the
oracle's restatement of the scalar loop (or_argmax, pinned in
tests/test_oracle.py against numpy's argmax / nanargmax): the same id for
every row, including ties, +0 / -0, -inf rows, NaN at id 0 and elsewhere,
and rows that are not a multiple of the kernel's batch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run(hip, x, ldx=None):
    rows, n = x.shape
    ldx = ldx or n
    buf = np.zeros((rows, ldx), dtype=np.float32)
    buf[:, :n] = x
    dx = hip.DeviceBuffer.from_array(buf)
    di, dv = hip.DeviceBuffer(rows * 4), hip.DeviceBuffer(rows * 4)
    hip.check(hip.lib().nhip_argmax_dev(dx.ptr, ldx, n, rows, di.ptr, dv.ptr, None))
    return di.download(np.int32), dv.download(np.float32)


def oracle(orc, x):
    return np.array([orc.lib().or_argmax(orc.p(np.ascontiguousarray(r)), x.shape[1]) for r in x], dtype=np.int32)


@pytest.mark.parametrize("n", [1, 5, 1023, 1024, 1025, 8192, 32000, 100003])
def test_argmax_matches_oracle(hip, orc, n):
    rng = np.random.default_rng(n)
    rows = 12
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[1] = rng.integers(-3, 3, n).astype(np.float32)  # ties: the lowest id wins
    x[2] = -np.inf
    x[3, 0] = np.nan
    x[4, rng.integers(0, n, 7)] = np.nan
    x[5] = 0.0
    x[5, ::2] = -0.0
    x[6, n // 2] = np.inf
    x[6, n - 1] = np.inf
    x[7, n - 1] = 1e30  # the maximum at the very end
    x[8] = np.float32(3.0)
    x[9, rng.integers(0, n, 3)] = -np.inf
    idx, val = run(hip, x)
    want = oracle(orc, x)
    assert np.array_equal(idx, want)
    picked = x[np.arange(rows), want]
    assert np.array_equal(np.isnan(val), np.isnan(picked))
    ok = ~np.isnan(picked)
    assert np.array_equal(val[ok].view(np.uint32), picked[ok].view(np.uint32))


def test_argmax_row_stride(hip, orc):
    rng = np.random.default_rng(3)
    x = rng.integers(-9, 9, (5, 3000)).astype(np.float32)
    idx, _ = run(hip, x, ldx=3072)
    assert np.array_equal(idx, oracle(orc, x))


def test_argmax_rejects_bad_arguments(hip):
    lib = hip.lib()
    buf = hip.DeviceBuffer(4096)
    assert lib.nhip_argmax_dev(buf.ptr, 10, 0, 1, buf.ptr, None, None) != 0  # n < 1
    assert lib.nhip_argmax_dev(buf.ptr, 10, 20, 2, buf.ptr, None, None) != 0  # stride shorter than a row
    assert lib.nhip_argmax_dev(None, 10, 10, 1, buf.ptr, None, None) != 0
    assert lib.nhip_argmax_dev(buf.ptr, 10, 10, 0, buf.ptr, None, None) == 0  # no rows: nothing to do
