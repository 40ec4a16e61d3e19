"""GPU TopKLogSoftmax as the decoder's head runs it (nhip_topk_lse_dev;
Ops.TopKLogSoftmax, src/Needle/Ops.cs:1092-1221) against the oracle's
restatement (or_topk_lse): ids and log-probabilities bit-identical, also
with ties across and within the 2048-id blocks, -inf logits, masked ids
and fewer allowed ids than k."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def oracle(orc, x, k):
    rows = x.shape[0]
    idx = np.zeros((rows, k), dtype=np.int32)
    lp = np.zeros((rows, k), dtype=np.float32)
    for r in range(rows):
        xr = np.ascontiguousarray(x[r])
        orc.lib().or_topk_lse(orc.p(xr), x.shape[1], k, 1, orc.p(idx[r]), orc.p(lp[r]))
    return idx, lp


def run(hip, x, k):
    rows, n = x.shape
    lib = hip.lib()
    dx = hip.DeviceBuffer.from_array(np.ascontiguousarray(x))
    ws = hip.DeviceBuffer(lib.nhip_topk_lse_workspace(rows, n))
    di, dl = hip.DeviceBuffer(rows * k * 4), hip.DeviceBuffer(rows * k * 4)
    hip.check(lib.nhip_topk_lse_dev(dx.ptr, rows, n, k, ws.ptr, ws.nbytes, di.ptr, dl.ptr, None))
    return di.download(np.int32).reshape(rows, k), dl.download(np.float32).reshape(rows, k)


@pytest.mark.parametrize("n", [5, 7, 300, 2048, 2051, 32000, 20000 + 3])
@pytest.mark.parametrize("k", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_topk_lse_matches_oracle(hip, orc, n, k, kind):
    rng = np.random.default_rng(n * 16 + k + (kind == "ties"))
    rows = 4
    if kind == "ties":  # few distinct values: ties inside and across blocks
        x = rng.integers(-6, 3, (rows, n)).astype(np.float32)
    else:
        x = rng.standard_normal((rows, n)).astype(np.float32) * 3.0
    x[1, : n // 2] = -np.inf
    x[2, 1] = 50.0  # the row's top allowed value
    x[2, 2] = 60.0  # larger values on the masked ids 2 and 3: never chosen
    x[2, 3] = 70.0
    got = run(hip, x, k)
    want = oracle(orc, x, k)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))


def test_topk_lse_fewer_allowed_ids_than_k(hip, orc):
    """n = 5: ids 1 and 4 are the only allowed ones; the remaining slots are
    the (-inf, INT_MAX) placeholders of both restatements."""
    x = np.array([[3.0, 1.0, 9.0, 9.0, 2.0], [-1.0, -np.inf, 4.0, 4.0, 2.0]], dtype=np.float32)
    for k in (2, 3, 4):
        got = run(hip, x, k)
        want = oracle(orc, x, k)
        assert np.array_equal(got[0], want[0]), k
        assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), k


def test_topk_lse_rejects_bad_arguments(hip, orc):
    lib = hip.lib()
    buf = hip.DeviceBuffer(1 << 16)
    p = buf.ptr
    assert lib.nhip_topk_lse_dev(p, 1, 100, 9, p, buf.nbytes, p, p, None) != 0  # k above 8
    assert lib.nhip_topk_lse_dev(p, 1, 100, 0, p, buf.nbytes, p, p, None) != 0
    assert lib.nhip_topk_lse_dev(p, 1, 600000, 3, p, buf.nbytes, p, p, None) != 0  # above 256 blocks
    assert lib.nhip_topk_lse_dev(p, 4, 32000, 3, p, 64, p, p, None) != 0  # workspace too small
    assert "workspace" in hip.last_error()
