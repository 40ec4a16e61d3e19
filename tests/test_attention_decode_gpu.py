"""GPU parity of the ragged decode attention over a pooled int8 KV cache
(nhip_attention_decode_dev) against the oracle's restatement of
AttentionBatch.ExecuteChunk + MergePartials (src/Needle/Blocks.cs:927-966,
750-817): bit-exact, because the chunk plan, the per-chunk sums (ascending
positions), the merge order and the polynomial exp are the same."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class Cache:
    def __init__(self, orc, hip, seed, slots, capacity, kv_heads, qk):
        st = orc.state(seed)
        self.slots, self.capacity, self.kv_heads, self.qk = slots, capacity, kv_heads, qk
        self.keys, self.ks, self.values, self.vs = orc.kv_cache(st, slots, capacity, kv_heads, qk)
        self.st = st
        self.d = [hip.DeviceBuffer.from_array(a) for a in (self.keys, self.ks, self.values, self.vs)]


def run_decode(hip, cache, q, qs, heads, rows_spec, max_chunks, ws=None, out=None):
    slot, first, count = (np.array(x, dtype=np.int32) for x in zip(*rows_spec))
    rows = len(rows_spec)
    dq, dqs = hip.DeviceBuffer.from_array(q), hip.DeviceBuffer.from_array(qs)
    dsl, dfi, dco = (hip.DeviceBuffer.from_array(a) for a in (slot, first, count))
    if ws is None:
        nbytes = hip.lib().nhip_attention_decode_workspace(rows, heads, max_chunks)
        ws = hip.DeviceBuffer(nbytes)
        hip.check(hip.lib().nhip_attention_decode_workspace_init(ws.ptr, ws.nbytes, None))
    if out is None:
        out = hip.DeviceBuffer(rows * heads * 64 * 4)
    k, ks, v, vs = cache.d
    hip.check(hip.lib().nhip_attention_decode_dev(dq.ptr, dqs.ptr, rows, heads, cache.kv_heads, cache.qk, k.ptr, ks.ptr,
                                                  v.ptr, vs.ptr, cache.slots, cache.capacity, dsl.ptr, dfi.ptr,
                                                  dco.ptr, max_chunks, ws.ptr, ws.nbytes, out.ptr, None))
    return out.download(np.float32).reshape(rows, heads, 64), ws


def oracle_decode(orc, cache, q, qs, heads, rows_spec, max_chunks):
    slot, first, count = (np.array(x, dtype=np.int32) for x in zip(*rows_spec))
    return orc.attention_decode(q, qs, heads, cache.kv_heads, cache.qk, cache.keys, cache.ks, cache.values, cache.vs,
                                cache.capacity, slot, first, count, max_chunks)


def queries(orc, st, rows, heads, qk):
    qf = orc.synth_normal(st, rows * heads * qk).reshape(rows * heads, qk)
    q, qs = orc.quantize_rows(qf)
    return q, qs


def bit_equal(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("heads,kv_heads,qk", [(16, 16, 64), (12, 2, 48), (4, 1, 64), (8, 8, 48), (6, 2, 64)])
@pytest.mark.parametrize("max_chunks", [8, 64])
def test_decode_attention_bit_exact(hip, orc, heads, kv_heads, qk, max_chunks):
    cache = Cache(orc, hip, 1000 + heads + kv_heads + qk, 4, 2048, kv_heads, qk)
    spec = [(0, 0, 1), (1, 0, 2), (2, 5, 3), (3, 0, 16), (0, 7, 17), (1, 100, 31), (2, 0, 32), (3, 0, 33),
            (0, 1000, 100), (1, 0, 257), (2, 1048, 1000), (3, 0, 2048), (1, 2047, 1), (0, 64, 64)]
    q, qs = queries(orc, cache.st, len(spec), heads, qk)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
    want = oracle_decode(orc, cache, q, qs, heads, spec, max_chunks)
    assert bit_equal(got, want)


@pytest.mark.parametrize("capacity", [256, 600])
@pytest.mark.parametrize("heads,kv_heads,qk", [(16, 16, 64), (6, 2, 48)])
def test_decode_attention_single_chunk_plan(hip, orc, heads, kv_heads, qk, capacity):
    """max_chunks 1: every row is one chunk, finished with the merge of one
    partial, no merge launch (capacity 256: the whole-row kernel; 600: the
    chunk kernel)."""
    cache = Cache(orc, hip, 31 + heads, 3, capacity, kv_heads, qk)
    spec = [(0, 0, 1), (1, 3, 17), (2, 0, 256), (0, 100, 99), (1, 0, 192)]
    q, qs = queries(orc, cache.st, len(spec), heads, qk)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, 1)
    assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, 1))


@pytest.mark.parametrize("heads,kv_heads,qk", [(16, 16, 64), (12, 2, 48), (4, 1, 64), (8, 8, 48)])
@pytest.mark.parametrize("capacity,max_chunks", [(512, 1), (512, 2), (512, 8), (512, 64), (192, 64), (513, 64)])
def test_decode_attention_short_cache_bit_exact(hip, orc, heads, kv_heads, qk, capacity, max_chunks):
    """Caches of at most 512 positions take the whole-row kernel (one
    workgroup per (row, head) runs every chunk and the merge); 513 takes the
    chunk kernel and its merge launch.  Counts cover one chunk, the two-chunk
    merge branch, uneven last chunks and the full cache."""
    cache = Cache(orc, hip, 77 + heads + qk + capacity + max_chunks, 3, capacity, kv_heads, qk)
    spec = [(0, 0, 1), (1, 0, 2), (2, 5, 15), (0, 0, 16), (1, 7, 17), (2, 0, 31), (0, 1, 32), (1, 0, 33),
            (2, 0, 47), (0, 10, 48), (1, 0, 100), (2, 3, 129), (0, 0, 160), (1, 0, 191), (2, 0, capacity),
            (0, capacity - 1, 1), (1, capacity // 2, capacity - capacity // 2)]
    q, qs = queries(orc, cache.st, len(spec), heads, qk)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
    assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, max_chunks))


@pytest.mark.parametrize("heads,kv_heads,qk,rows", [(16, 16, 64, 17), (32, 4, 64, 9), (16, 2, 48, 16)])
@pytest.mark.parametrize("capacity,max_chunks", [(2048, 64), (2048, 8), (4096, 64), (600, 2), (1024, 4)])
def test_decode_attention_long_rows_bit_exact(hip, orc, heads, kv_heads, qk, rows, capacity, max_chunks):
    """Caches of 600..4096 positions and at least 256 (row, head) pairs, in
    groups of 1, 8 and 8 query heads per kv head: the chunk kernel and its
    merge, bit-exact, with full-cache, single-position and random spans."""
    cache = Cache(orc, hip, 500 + heads + qk + capacity + max_chunks, 4, capacity, kv_heads, qk)
    rng = np.random.default_rng(capacity + max_chunks + heads)
    fixed = [(0, 0, capacity), (1, capacity - 1, 1), (2, 0, 2), (3, 5, 33), (0, 100, 17), (1, 0, capacity // 2 + 3)]
    spec = fixed + [(int(rng.integers(0, 4)), 0, int(rng.integers(1, capacity + 1))) for _ in range(rows - len(fixed))]
    assert len(spec) * heads >= 256
    q, qs = queries(orc, cache.st, len(spec), heads, qk)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
    assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, max_chunks))


def test_decode_attention_several_head_blocks(hip, orc):
    """Chunks of up to 1024 positions (capacity 8192, max_chunks 8) leave LDS
    for 5 of 16 kv heads per workgroup: 4 head blocks per row."""
    heads = 16
    cache = Cache(orc, hip, 4242, 2, 8192, heads, 64)
    spec = [(0, 0, 8192), (1, 17, 5000), (0, 3, 40), (1, 0, 1), (1, 4000, 2049), (0, 8000, 192)]
    q, qs = queries(orc, cache.st, len(spec), heads, 64)
    assert hip.lib().nhip_attention_decode_workspace(len(spec), heads, 8) > 0
    for rep in range(2):
        got, _ = run_decode(hip, cache, q, qs, heads, spec, 8)
        assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, 8)), rep


def test_decode_attention_invalid_rows_are_zero(hip, orc):
    cache = Cache(orc, hip, 42, 2, 256, 2, 64)
    heads = 4
    spec = [(0, 0, 10), (5, 0, 10), (1, 250, 10), (1, -1, 5), (0, 0, 0), (1, 0, 256)]
    q, qs = queries(orc, cache.st, len(spec), heads, 64)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, 64)
    want = oracle_decode(orc, cache, q, qs, heads, [(0, 0, 10), (0, 0, 0), (0, 0, 0), (0, 0, 0), (0, 0, 0),
                                                    (1, 0, 256)], 64)
    assert bit_equal(got[[0, 5]], want[[0, 5]])
    assert np.all(got[1:5] == 0.0)


@pytest.mark.parametrize("rows", [6, 20, 64, 70])
def test_decode_attention_chunk_kernel_invalid_and_many_rows(hip, orc, rows):
    """The chunk kernel (capacity 1024) with invalid spans among valid ones:
    up to 64 rows the units are placed in length order over the compute
    units (20 rows x 16 chunks: a second, backward round of 256 workgroups,
    partly used), beyond that one workgroup per (chunk, row); either way the
    valid rows are bit-exact and the invalid ones zero."""
    heads, kv_heads, capacity, max_chunks = 8, 4, 1024, 16
    cache = Cache(orc, hip, 7000 + rows, 3, capacity, kv_heads, 64)
    rng = np.random.default_rng(rows)
    spec = [(int(rng.integers(0, 3)), 0, int(rng.integers(1, capacity + 1))) for _ in range(rows)]
    bad = {1: (3, 0, 10), 2: (1, -1, 5), 3: (0, 0, 0), 4: (2, 1000, 25)}
    for k, v in bad.items():
        spec[k] = v
    q, qs = queries(orc, cache.st, rows, heads, 64)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
    good = [k for k in range(rows) if k not in bad]
    want = oracle_decode(orc, cache, q, qs, heads, [spec[k] if k not in bad else (0, 0, 0) for k in range(rows)],
                         max_chunks)
    assert bit_equal(got[good], want[good])
    assert np.all(got[list(bad)] == 0.0)


@pytest.mark.parametrize("max_chunks", [100, 256])
def test_decode_attention_merge_of_many_chunks(hip, orc, max_chunks):
    """Rows of up to 8192 positions in up to 256 chunks: the merge walks its
    chunks in batches of 64 (the last one partly filled), bit-exact."""
    heads = 8
    cache = Cache(orc, hip, 9100 + max_chunks, 2, 8192, heads, 64)
    spec = [(0, 0, 8192), (1, 5, 4100), (0, 100, 1700), (1, 0, 1040), (0, 7000, 1190), (1, 3, 33)]
    q, qs = queries(orc, cache.st, len(spec), heads, 64)
    got, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
    assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, max_chunks))


def test_decode_attention_workspace_reuse(hip, orc):
    """Repeated calls on one workspace stay exact, also with new spans."""
    cache = Cache(orc, hip, 7, 3, 1024, 4, 64)
    heads = 8
    rng = np.random.default_rng(5)
    ws = out = None
    for it in range(4):
        spec = [(int(rng.integers(0, 3)), 0, int(rng.integers(1, 1025))) for _ in range(9)]
        q, qs = queries(orc, cache.st, len(spec), heads, 64)
        got, ws = run_decode(hip, cache, q, qs, heads, spec, 64, ws=ws)
        assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, 64)), it


def test_decode_attention_graph_replays(hip, orc):
    """Captured once, replayed with new spans written to the device arrays
    between replays (the decode loop's pattern); every replay is exact."""
    cache = Cache(orc, hip, 99, 4, 512, 2, 48)
    heads, rows, mc = 12, 6, 64
    q, qs = queries(orc, cache.st, rows, heads, 48)
    dq, dqs = hip.DeviceBuffer.from_array(q), hip.DeviceBuffer.from_array(qs)
    dsl, dfi, dco = (hip.DeviceBuffer(rows * 4) for _ in range(3))
    ws = hip.DeviceBuffer(hip.lib().nhip_attention_decode_workspace(rows, heads, mc))
    hip.check(hip.lib().nhip_attention_decode_workspace_init(ws.ptr, ws.nbytes, None))
    out = hip.DeviceBuffer(rows * heads * 64 * 4)
    k, ks, v, vs = cache.d
    stream = hip.Stream()
    with hip.Graph.capture(stream) as g:
        hip.check(hip.lib().nhip_attention_decode_dev(dq.ptr, dqs.ptr, rows, heads, 2, 48, k.ptr, ks.ptr, v.ptr, vs.ptr,
                                                      4, 512, dsl.ptr, dfi.ptr, dco.ptr, mc, ws.ptr, ws.nbytes,
                                                      out.ptr, stream.ptr))
    for rep in range(4):
        spec = [(r % 4, 0, 20 + 83 * rep + 37 * r) for r in range(rows)]
        for buf, col in zip((dsl, dfi, dco), zip(*spec)):
            buf.upload(np.array(col, dtype=np.int32))
        g.launch()
        stream.sync()
        got = out.download(np.float32).reshape(rows, heads, 64)
        assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, mc)), rep
    g.close()


def test_decode_attention_rejects_bad_shapes(hip, orc):
    lib = hip.lib()
    buf = hip.DeviceBuffer(1 << 16)
    p = buf.ptr
    assert lib.nhip_attention_decode_dev(p, p, 1, 6, 4, 64, p, p, p, p, 1, 16, p, p, p, 8, p, buf.nbytes, p, None) != 0
    assert lib.nhip_attention_decode_dev(p, p, 1, 4, 4, 32, p, p, p, p, 1, 16, p, p, p, 8, p, buf.nbytes, p, None) != 0
    # chunks of 8192 positions: even one kv head per workgroup exceeds LDS,
    # so the call is rejected before any launch
    assert lib.nhip_attention_decode_dev(p, p, 1, 4, 4, 64, p, p, p, p, 1, 65536, p, p, p, 8, p, buf.nbytes, p,
                                         None) != 0
    assert "max_chunks" in hip.last_error()
