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
    the reference's (-inf, -1) (Ops.cs:1096)."""
    x = np.array([[3.0, 1.0, 9.0, 9.0, 2.0], [-1.0, -np.inf, 4.0, 4.0, 2.0]], dtype=np.float32)
    for k in (2, 3, 4):
        got = run(hip, x, k)
        want = oracle(orc, x, k)
        assert np.array_equal(got[0], want[0]), k
        assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), k
        assert np.all(got[0][:, 2:] == -1)


@pytest.mark.parametrize("n", [6, 300, 4100])
def test_topk_lse_few_values_above_minus_inf(hip, orc, n):
    """Rows with fewer than k values above -inf: the reference's selection
    admits its first scanned id (4) at -inf and drops it at the next entry,
    never admits a later -inf, and leaves (-inf, -1) in the slots left over
    (tests/test_oracle.py traces these cases by hand).  Ids equal; the
    log-probabilities bit-identical, or NaN on both sides for rows whose
    peak is -inf."""
    inf = np.inf
    rows = np.full((8, n), -inf, dtype=np.float32)
    rows[1, 1] = 2.5                      # only id 1 (x[4] = -inf stays in the last slot for k >= 2)
    rows[2, 5] = 1.0                      # one finite id after x[4] = -inf
    rows[3, n - 1] = 0.5                  # the last id only
    rows[4, [1, 4]] = [3.0, 3.0]          # a tie of id 1 and id 4
    rows[5, 4] = 7.0                      # x[4] finite
    rows[6, [1, n - 2, n - 1]] = [1.0, 1.0, 0.0]
    # row 0 and row 7: all -inf (peak -inf: NaN log-probabilities)
    rows[7, 0] = 9.0  # a masked id only
    for k in (1, 2, 3, 8):
        got = run(hip, rows, k)
        want = oracle(orc, rows, k)
        assert np.array_equal(got[0], want[0]), k
        g, w = got[1], want[1]
        assert np.array_equal(np.isnan(g), np.isnan(w)), k
        ok = ~np.isnan(w)
        assert np.array_equal(g[ok].view(np.uint32), w[ok].view(np.uint32)), k
        for r in range(rows.shape[0]):
            ref_idx = np.zeros(k, dtype=np.int32)
            ref_lp = np.zeros(k, dtype=np.float32)
            xr = np.ascontiguousarray(rows[r])
            orc.lib().or_topk_log_softmax(orc.p(xr), n, k, orc.p(ref_idx), orc.p(ref_lp), None, 1)
            assert np.array_equal(got[0][r], ref_idx), (k, r)


def test_topk_lse_rejects_bad_arguments(hip, orc):
    lib = hip.lib()
    buf = hip.DeviceBuffer(1 << 16)
    p = buf.ptr
    assert lib.nhip_topk_lse_dev(p, 1, 100, 9, p, buf.nbytes, p, p, None) != 0  # k above 8
    assert lib.nhip_topk_lse_dev(p, 1, 100, 0, p, buf.nbytes, p, p, None) != 0
    assert lib.nhip_topk_lse_dev(p, 1, 600000, 3, p, buf.nbytes, p, p, None) != 0  # above 256 blocks
    assert lib.nhip_topk_lse_dev(p, 4, 32000, 3, p, 64, p, p, None) != 0  # workspace too small
    assert "workspace" in hip.last_error()
