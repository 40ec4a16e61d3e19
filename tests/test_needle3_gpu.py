"""Needle 3 attention inputs (nhip_needle3_attention_inputs_dev): taps,
ZeroCenteredRms, Rope and QuantizeInt8 from raw Q/K/V rows to the int8
queries and the KV-cache rows, against the oracle's row-by-row restatement of
EngineCore.TapsAndAttentionHeadsSingle (src/Needle/Engine.cs:1302-1387):
bit-identical queries, scales, cache rows and slot histories."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def avx2_row_tier(orc):
    """The GPU engine sums its rows in the AVX2 tier's order
    (or_n3_set_tier(1)); the oracle runs the same order here."""
    orc.lib().or_n3_set_tier(1)
    yield
    orc.lib().or_n3_set_tier(0)


class Case:
    def __init__(self, seed, heads, kv, qk, vd, slots, capacity):
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.g = (heads, kv, qk, vd)
        self.slots, self.capacity = slots, capacity
        qw, kw, vw = heads * qk, kv * qk, kv * vd
        self.all = qw + kw + vw
        f = lambda *s: rng.standard_normal(s).astype(np.float32)
        self.taps = [f(3, qw) * 0.5, f(3, kw) * 0.5, f(3, vw) * 0.5]
        self.qn, self.kn = f(qk) * 0.1, f(qk) * 0.1
        ang = rng.uniform(0, 6.28, (capacity, qk // 2))
        self.cos, self.sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        self.history = f(slots, 2 * self.all)
        self.keys = rng.integers(-128, 128, (slots, capacity, kw)).astype(np.int8)
        self.values = rng.integers(-128, 128, (slots, capacity, vw)).astype(np.int8)
        self.ks, self.vs = f(slots, capacity, kv), f(slots, capacity, kv)

    def oracle(self, orc, raw, row_slot, row_pos):
        heads, kv, qk, vd = self.g
        rows = len(row_slot)
        out = dict(q=np.zeros((rows, heads * qk), np.int8), qs=np.zeros((rows, heads), np.float32),
                   keys=self.keys.copy(), values=self.values.copy(), ks=self.ks.copy(), vs=self.vs.copy(),
                   history=self.history.copy())
        rs, rp = np.asarray(row_slot, np.int32), np.asarray(row_pos, np.int32)
        orc.lib().or_needle3_attention_inputs(
            orc.p(raw), rows, heads, kv, qk, vd, orc.p(self.taps[0]), orc.p(self.taps[1]), orc.p(self.taps[2]),
            orc.p(self.qn), orc.p(self.kn), orc.p(self.cos), orc.p(self.sin), orc.p(out["history"]), orc.p(rs),
            orc.p(rp), self.slots, self.capacity, orc.p(out["q"]), orc.p(out["qs"]), orc.p(out["keys"]),
            orc.p(out["ks"]), orc.p(out["values"]), orc.p(out["vs"]))
        return out

    def gpu(self, hip, raw, row_slot, row_pos, state=None):
        heads, kv, qk, vd = self.g
        rows = len(row_slot)
        D = hip.DeviceBuffer.from_array
        st = state or dict(keys=D(self.keys), values=D(self.values), ks=D(self.ks), vs=D(self.vs),
                           history=D(self.history))
        dq, dqs = hip.DeviceBuffer(rows * heads * qk), hip.DeviceBuffer(rows * heads * 4)
        args = [D(raw), D(self.taps[0]), D(self.taps[1]), D(self.taps[2]), D(self.qn), D(self.kn), D(self.cos),
                D(self.sin), D(np.asarray(row_slot, np.int32)), D(np.asarray(row_pos, np.int32))]
        hip.check(hip.lib().nhip_needle3_attention_inputs_dev(
            args[0].ptr, rows, heads, kv, qk, vd, args[1].ptr, args[2].ptr, args[3].ptr, args[4].ptr, args[5].ptr,
            args[6].ptr, args[7].ptr, st["history"].ptr, args[8].ptr, args[9].ptr, self.slots, self.capacity,
            dq.ptr, dqs.ptr, st["keys"].ptr, st["ks"].ptr, st["values"].ptr, st["vs"].ptr, None))
        out = dict(q=dq.download(np.int8).reshape(rows, -1), qs=dqs.download(np.float32).reshape(rows, -1),
                   keys=st["keys"].download(np.int8).reshape(self.keys.shape),
                   values=st["values"].download(np.int8).reshape(self.values.shape),
                   ks=st["ks"].download(np.float32).reshape(self.ks.shape),
                   vs=st["vs"].download(np.float32).reshape(self.vs.shape),
                   history=st["history"].download(np.float32).reshape(self.history.shape))
        return out, st


def same(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@pytest.mark.parametrize("geom", [(12, 2, 48, 64), (16, 16, 64, 64), (4, 1, 48, 32)],
                         ids=["needle3-qk48", "mha-qk64", "gqa-small"])
def test_attention_inputs_match_row_by_row_oracle(hip, orc, geom):
    c = Case(sum(geom), *geom, slots=4, capacity=40)
    # runs: slot 2 positions 10..12, slot 0 position 5, an invalid row, slot 3 positions 0..1
    row_slot = [2, 2, 2, 0, 9, 3, 3]
    row_pos = [10, 11, 12, 5, 3, 0, 1]
    raw = c.rng.standard_normal((len(row_slot), c.all)).astype(np.float32)
    got, st = c.gpu(hip, raw, row_slot, row_pos)
    want = c.oracle(orc, raw, row_slot, row_pos)
    for k in ("q", "qs", "keys", "values", "ks", "vs", "history"):
        assert same(got[k], want[k]), k
    assert np.all(got["q"][4] == 0) and np.all(got["qs"][4] == 1.0)
    # the next step of every slot continues from the moved histories
    c.keys, c.values, c.ks, c.vs, c.history = (want[k] for k in ("keys", "values", "ks", "vs", "history"))
    row_slot2, row_pos2 = [0, 2, 3], [6, 13, 2]
    raw2 = c.rng.standard_normal((3, c.all)).astype(np.float32)
    got2, _ = c.gpu(hip, raw2, row_slot2, row_pos2, state=st)
    want2 = c.oracle(orc, raw2, row_slot2, row_pos2)
    for k in ("q", "qs", "keys", "values", "ks", "vs", "history"):
        assert same(got2[k], want2[k]), ("second step", k)


def test_attention_inputs_chunk_equals_single_rows(hip, orc):
    """A run of six rows in one call equals six one-row calls (the
    reference's chunk == sequential invariant)."""
    c = Case(99, 12, 2, 48, 64, slots=2, capacity=32)
    raw = c.rng.standard_normal((6, c.all)).astype(np.float32)
    whole, _ = c.gpu(hip, raw, [1] * 6, list(range(4, 10)))
    st = None
    qs = []
    for i in range(6):
        one, st = c.gpu(hip, raw[i:i + 1], [1], [4 + i], state=st)
        qs.append(one["q"][0])
    assert same(np.stack(qs), whole["q"])
    for k in ("keys", "values", "ks", "vs", "history"):
        assert same(one[k], whole[k]), k
