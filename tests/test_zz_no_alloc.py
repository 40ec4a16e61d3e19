"""The no-allocation attention entry (nhip_attention_decode_noalloc_dev,
no counterpart in the reference: for callers that cannot allocate) against
the workspace entry it mirrors (nhip_attention_decode_dev) on the same
inputs: bit-identical outputs on two calls in a row, the second with a
smaller input (the shared scratch keeps the first call's partials, which
the second must not read), on caches above 512 positions so that the chunk
kernel and the merge (the paths that use the scratch) run; sizes above the
8 MiB scratch are refused.  Also checked against the oracle."""
import numpy as np
import pytest

from test_attention_decode_gpu import Cache, bit_equal, oracle_decode, queries, run_decode

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20


def run_noalloc(hip, cache, q, qs, heads, rows_spec, max_chunks):
    slot, first, count = (np.array(x, dtype=np.int32) for x in zip(*rows_spec))
    rows = len(rows_spec)
    dq, dqs = hip.DeviceBuffer.from_array(q), hip.DeviceBuffer.from_array(qs)
    dsl, dfi, dco = (hip.DeviceBuffer.from_array(a) for a in (slot, first, count))
    out = hip.DeviceBuffer.from_array(np.full(rows * heads * 64, np.nan, dtype=np.float32))
    k, ks, v, vs = cache.d
    hip.check(hip.lib().nhip_attention_decode_noalloc_dev(dq.ptr, dqs.ptr, rows, heads, cache.kv_heads, cache.qk,
                                                          k.ptr, ks.ptr, v.ptr, vs.ptr, cache.slots, cache.capacity,
                                                          dsl.ptr, dfi.ptr, dco.ptr, max_chunks, out.ptr, None))
    return out.download(np.float32).reshape(rows, heads, 64)


@pytest.mark.parametrize("heads,kv_heads,qk", [(16, 16, 64), (12, 2, 48)])
def test_noalloc_matches_workspace_entry_twice(hip, orc, heads, kv_heads, qk):
    cache = Cache(orc, hip, 4100 + heads, 16, 2048, kv_heads, qk)
    rng = np.random.default_rng(heads)
    big = [(s, 0, int(c)) for s, c in zip(range(16), rng.integers(32, 2049, 16))]
    small = [(3, 7, 900), (0, 0, 600), (5, 100, 1)]
    for spec, max_chunks in ((big, 64), (small, 8)):
        q, qs = queries(orc, cache.st, len(spec), heads, qk)
        got = run_noalloc(hip, cache, q, qs, heads, spec, max_chunks)
        want, _ = run_decode(hip, cache, q, qs, heads, spec, max_chunks)
        assert bit_equal(got, want)
        assert bit_equal(got, oracle_decode(orc, cache, q, qs, heads, spec, max_chunks))


def test_noalloc_refuses_partials_above_the_scratch(hip, orc):
    cache = Cache(orc, hip, 4200, 2, 1024, 4, 64)
    rows, heads, chunks = 64, 16, 256
    assert hip.lib().nhip_attention_decode_workspace(rows, heads, chunks) > SCRATCH_BYTES
    spec = [(r % 2, 0, 1000) for r in range(rows)]
    q, qs = queries(orc, cache.st, rows, heads, 64)
    with pytest.raises(RuntimeError, match="scratch"):
        run_noalloc(hip, cache, q, qs, heads, spec, chunks)
