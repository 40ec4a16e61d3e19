"""The Needle 3 batched engine on the GPU (nhip_ctx_* / nhip_step /
nhip_slot_*) against the oracle's ForwardBatch restatement, bit for bit.

A random-init archive of Needle 3's layer program (needle_cs_amd/archive.py:
4-lane hyper-connections, an engram site, a global layer among windowed
ones, the Kronecker-Hadamard MLP) is opened with nhip_open and stepped like
BatchedEngine (src/Needle/BatchEngine.cs:5-50, Engine.cs:2285-2350); the
oracle engine steps the same rows.  Beyond equality with the oracle, the
engine's own structure is checked on the GPU: batched == single slots, one
chunk == row-by-row, rewind + re-feed == the first feed, slot copy == the
source, and head_rows subsets == rows of the full head.
"""
import ctypes as C

import numpy as np
import pytest

from needle_cs_amd.archive import NEEDLE3, SMALL, needle3_archive
from oracle.needle3 import OracleEngine, OracleModel

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def avx2_row_tier(orc):
    """The GPU engine sums its rows in the AVX2 tier's order
    (or_n3_set_tier(1)); the oracle runs the same order here."""
    orc.lib().or_n3_set_tier(1)
    yield
    orc.lib().or_n3_set_tier(0)

GEOM = SMALL
SEED = 3
MAX_CHUNKS = 8


@pytest.fixture(scope="module")
def archive():
    return needle3_archive(GEOM, SEED)


@pytest.fixture(scope="module")
def model(hip, archive):
    from needle_cs_amd.engine import Model
    m = Model(archive)
    yield m
    m.close()


@pytest.fixture(scope="module")
def omodel(orc, archive):
    return OracleModel(orc, archive)


def gpu_engine(model, slots=3, capacity=96, chunk=16):
    from needle_cs_amd.engine import BatchedEngine
    return BatchedEngine(model, context_length=capacity, chunk_size=chunk, slots=slots, max_chunks=MAX_CHUNKS)


def cpu_engine(orc, omodel, slots=3, capacity=96):
    return OracleEngine(orc, omodel, slots=slots, capacity=capacity, max_chunks=MAX_CHUNKS)


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def tokens(seed, n):
    return np.random.default_rng(seed).integers(0, GEOM["vocab"], n).astype(np.int32)


def test_steps_match_the_oracle(hip, orc, model, omodel):
    """Mixed prefill chunks over three slots, then decode steps past the
    sliding window (6) with every row a head row: logits, top-4 and ArgMax."""
    print("needle3 step parity", flush=True)
    g, o = gpu_engine(model), cpu_engine(orc, omodel)
    try:
        rounds = [
            (np.r_[tokens(1, 7), tokens(2, 5)], [0] * 7 + [1] * 5, [6, 11]),
            (tokens(3, 9), [2] * 9, [8]),
            (np.r_[tokens(4, 3), tokens(5, 1), tokens(6, 2)], [1, 1, 1, 0, 2, 2], [0, 2, 3, 5]),
        ]
        for step in range(12):
            t = tokens(100 + step, 3)
            rounds.append((t, [0, 1, 2], [0, 1, 2]))
        for i, (t, s, h) in enumerate(rounds):
            lg, idx, lp, am = g.forward_batch(t, s, h, k=4, argmax=True)
            want = o.step(t, s, h)
            assert np.isfinite(want).all()
            assert same_bits(lg, want), f"round {i}: max |diff| {np.abs(lg - want).max()}"
            for r in range(len(h)):
                assert am[r] == orc.lib().or_argmax(orc.p(want[r]), want.shape[1])
                ridx = np.zeros(4, dtype=np.int32)
                rlp = np.zeros(4, dtype=np.float32)
                orc.lib().or_topk_log_softmax(orc.p(np.ascontiguousarray(want[r])), want.shape[1], 4, orc.p(ridx),
                                              orc.p(rlp), None, 1)
                assert np.array_equal(idx[r], ridx)
                assert np.allclose(lp[r], rlp, rtol=0, atol=2e-5)
        for slot in range(3):
            assert g.slot_length(slot) == o.length(slot)
    finally:
        g.close()
        o.close()


def test_decode_of_many_slots_matches_the_oracle(hip, orc, model, omodel):
    """Steps of 2 to 16 rows, one per slot: up to 4 rows the gate and the
    output matmul run in one launch; from 5 rows the attention launch forms
    the Q/K/V/Gate projections itself and the gate runs apart from the output
    matmul.  Logits bit for bit."""
    print("needle3 many-slot decode parity", flush=True)
    n = 16
    g, o = gpu_engine(model, slots=n), cpu_engine(orc, omodel, slots=n)
    try:
        rounds = [(np.r_[tokens(200, 8), tokens(201, 8)], [0] * 8 + [1] * 8, [7, 15])]
        for base in range(2, n, 2):  # two slots a round: runs of rows
            rounds.append((np.r_[tokens(200 + base, 3), tokens(201 + base, 4)], [base] * 3 + [base + 1] * 4, [2, 6]))
        for step, live in enumerate([n, 4, 5, n, 2, 9, 12, n]):
            slots = list(range(n))[step % 3::1][:live] if live < n else list(range(n))
            t = tokens(300 + step, len(slots))
            rounds.append((t, slots, list(range(len(slots)))))
        for i, (t, s, h) in enumerate(rounds):
            lg, _, _, _ = g.forward_batch(t, s, h, argmax=True)
            want = o.step(t, s, h)
            assert np.isfinite(want).all()
            assert same_bits(lg, want), f"round {i} ({len(s)} rows): max |diff| {np.abs(lg - want).max()}"
        for slot in range(n):
            assert g.slot_length(slot) == o.length(slot)
    finally:
        g.close()
        o.close()


def test_head_rows_subset_equals_rows_of_the_full_head(hip, model):
    t = tokens(11, 10)
    s = [0] * 4 + [1] * 6
    a, b = gpu_engine(model), gpu_engine(model)
    try:
        full, _, _, _ = a.forward_batch(t, s, list(range(10)))
        sub, _, _, _ = b.forward_batch(t, s, [9, 2, 5])
        assert same_bits(sub, full[[9, 2, 5]])
        none, _, _, _ = b.forward_batch(tokens(12, 2), [0, 1], [])
        assert none.shape == (0, GEOM["vocab"])
    finally:
        a.close()
        b.close()


def test_batched_equals_single(hip, model):
    """Two slots stepped together give each slot's logits of stepping alone."""
    p0, p1 = tokens(21, 9), tokens(22, 7)
    both, alone = gpu_engine(model), gpu_engine(model)
    try:
        lg, _, _, _ = both.forward_batch(np.r_[p0, p1], [0] * 9 + [1] * 7, [8, 15])
        a0, _, _, _ = alone.forward_batch(p0, [0] * 9, [8])
        a1, _, _, _ = alone.forward_batch(p1, [1] * 7, [6])
        assert same_bits(lg, np.r_[a0, a1])
        for step in range(8):
            t = tokens(300 + step, 2)
            lg, _, _, _ = both.forward_batch(t, [0, 1], [0, 1])
            a1, _, _, _ = alone.forward_batch(t[1:], [1], [0])
            a0, _, _, _ = alone.forward_batch(t[:1], [0], [0])
            assert same_bits(lg, np.r_[a0, a1]), f"decode step {step}"
    finally:
        both.close()
        alone.close()


def test_chunk_equals_sequential(hip, model):
    """A prompt in one chunk and row by row reach the same logits."""
    p = tokens(31, 14)
    chunk, seq = gpu_engine(model), gpu_engine(model)
    try:
        lc, _, _, _ = chunk.forward_batch(p, [0] * 14, list(range(14)))
        rows = []
        for i in range(14):
            r, _, _, _ = seq.forward_batch(p[i:i + 1], [0], [0])
            rows.append(r[0])
        assert same_bits(lc, np.stack(rows))
        for step in range(6):
            t = tokens(400 + step, 1)
            a, _, _, _ = chunk.forward_batch(t, [0], [0])
            b, _, _, _ = seq.forward_batch(t, [0], [0])
            assert same_bits(a, b)
    finally:
        chunk.close()
        seq.close()


def test_feed_slot_matches_the_oracle_in_chunks(hip, orc, model, omodel):
    """FeedSlot over 40 tokens in chunks of 16 (three steps, logits of the last)."""
    p = tokens(41, 40)
    g, o = gpu_engine(model, slots=2), cpu_engine(orc, omodel, slots=2)
    try:
        got = g.feed_slot(1, p)
        want = None
        for start in range(0, 40, 16):
            part = p[start:start + 16]
            last = start + len(part) == 40
            want = o.step(part, [1] * len(part), [len(part) - 1] if last else [])
        assert same_bits(got, want[0])
        assert g.slot_length(1) == 40 and g.feed_slot(1, [], compute_logits=False) is None
    finally:
        g.close()
        o.close()


def test_rewind_refeed_equals_first_feed_and_fresh_prefill(hip, model):
    p, more = tokens(51, 11), tokens(52, 5)
    g, fresh = gpu_engine(model), gpu_engine(model)
    try:
        g.feed_slot(0, p)
        g.mark_slot(0)
        first = [g.forward_batch(more[i:i + 1], [0], [0])[0] for i in range(5)]
        g.forward_batch(tokens(53, 4), [0] * 4, [3])  # a detour to rewind over
        g.rewind_slot(0)
        assert g.slot_length(0) == 11
        again = [g.forward_batch(more[i:i + 1], [0], [0])[0] for i in range(5)]
        fresh.feed_slot(2, p)
        ref = [fresh.forward_batch(more[i:i + 1], [2], [0])[0] for i in range(5)]
        for a, b, c in zip(first, again, ref):
            assert same_bits(a, b) and same_bits(a, c)
        g.reset_slot(0)
        assert g.slot_length(0) == 0
        lg_reset = g.feed_slot(0, p)
        lg_fresh = fresh.feed_slot(1, p)
        assert same_bits(lg_reset, lg_fresh)
    finally:
        g.close()
        fresh.close()


def test_slot_copy_clones_the_source(hip, model):
    p = tokens(61, 12)
    g = gpu_engine(model)
    try:
        g.feed_slot(0, p)
        g.mark_slot(0)
        g.forward_batch(tokens(62, 2), [0, 0], [1])
        g.copy_slot(2, 0)
        assert g.slot_length(2) == 14
        for step in range(5):
            t = tokens(500 + step, 1)
            lg, _, _, _ = g.forward_batch(np.r_[t, t], [0, 2], [0, 1])
            assert same_bits(lg[0:1], lg[1:2]), f"step {step}"
        g.rewind_slot(2)  # the copied mark
        assert g.slot_length(2) == 12
    finally:
        g.close()


def test_errors_leave_the_slots_untouched(hip, model):
    from needle_cs_amd import NeedleHipError
    g = gpu_engine(model, slots=2, capacity=20, chunk=8)
    try:
        g.feed_slot(0, tokens(71, 18))
        with pytest.raises(NeedleHipError, match="capacity"):
            g.forward_batch(tokens(72, 3), [0, 0, 0], [2])
        with pytest.raises(NeedleHipError, match="capacity"):
            g.feed_slot(0, tokens(73, 5))
        assert g.slot_length(0) == 18
        with pytest.raises(NeedleHipError, match="contiguous"):
            g.forward_batch(tokens(74, 3), [1, 0, 1], [0])
        with pytest.raises(NeedleHipError, match="rows"):
            g.forward_batch(tokens(75, 9), [1] * 9, [0])
        with pytest.raises(NeedleHipError, match="token"):
            g.forward_batch(np.array([GEOM["vocab"]], dtype=np.int32), [1], [0])
        with pytest.raises(NeedleHipError, match="slot"):
            g.forward_batch(tokens(76, 1), [2], [0])
        assert g.slot_length(1) == 0
        lg, _, _, _ = g.forward_batch(tokens(77, 2), [0, 0], [1])  # still usable: 20 of 20
        assert np.isfinite(lg).all() and g.slot_length(0) == 20
    finally:
        g.close()


def test_needle3_geometry_matches_the_oracle(hip, orc):
    """Needle 3's own geometry (768 hidden, 20 layers, 12/2 heads, 5 engram
    sites, 1024-wide MLP, 8192 vocab): a mixed prefill step and decode steps
    of three slots, bit for bit."""
    from needle_cs_amd.engine import BatchedEngine, Model
    print("needle3 full geometry parity", flush=True)
    archive = needle3_archive(NEEDLE3, 7)
    om = OracleModel(orc, archive)
    o = OracleEngine(orc, om, slots=3, capacity=64, max_chunks=MAX_CHUNKS)
    with Model(archive) as model, BatchedEngine(model, context_length=64, chunk_size=16, slots=3,
                                                max_chunks=MAX_CHUNKS) as g:
        rng = np.random.default_rng(8)
        t = rng.integers(0, NEEDLE3["vocab"], 16).astype(np.int32)
        s = [0] * 8 + [1] * 5 + [2] * 3
        lg, _, _, am = g.forward_batch(t, s, [7, 12, 15], argmax=True)
        want = o.step(t, s, [7, 12, 15])
        assert same_bits(lg, want)
        for step in range(3):
            t = am.astype(np.int32)
            lg, _, _, am = g.forward_batch(t, [0, 1, 2], [0, 1, 2], argmax=True)
            want = o.step(t, [0, 1, 2], [0, 1, 2])
            assert same_bits(lg, want), f"decode step {step}"
            assert np.array_equal(am, np.argmax(want, axis=1))
    o.close()


def test_needle3_window_past_1024_positions(hip, orc):
    """Needle 3's geometry with the cache past its 1024-position window
    (windowed layers attend max(0, pos - 1023)..pos, Blocks.cs:973-978;
    global layers every position, Model.cs:89-90): 1088 prompt tokens fed in
    128-row chunks, then 12 decode steps to position 1099.  Every decode
    step's logits equal the oracle's bit for bit, and the last one meets the
    reference's own numpy forward (tools/golden.py, the `window` vectors of
    tests/golden/needle3_golden.npz) at cosine >= 0.9995 with the same argmax."""
    import hashlib
    import os

    from needle_cs_amd.engine import BatchedEngine, Model
    fix = np.load(os.path.join(os.path.dirname(__file__), "golden", "needle3_golden.npz"))
    archive = needle3_archive(NEEDLE3, int(fix["window_seed"]))
    assert hashlib.sha256(archive).hexdigest() == str(fix["window_sha256"])
    toks = np.ascontiguousarray(fix["window_tokens"], dtype=np.int32)
    prompt, cap, chunks = 1088, 1152, 64
    orc.lib().or_n3_set_threads(min(16, os.cpu_count() or 1))
    om = OracleModel(orc, archive)
    o = OracleEngine(orc, om, slots=1, capacity=cap, max_chunks=chunks)
    try:
        with Model(archive) as model, BatchedEngine(model, context_length=cap, chunk_size=128, slots=1,
                                                    max_chunks=chunks) as g:
            print("needle3 window: GPU prefill of 1088 tokens", flush=True)
            g.feed_slot(0, toks[:prompt], compute_logits=False)
            for s in range(0, prompt, 128):
                part = toks[s:min(s + 128, prompt)]
                o.step(part, [0] * len(part), [])
                print(f"needle3 window: oracle prefill {s + len(part)}/{prompt}", flush=True)
            for pos in range(prompt, len(toks)):
                lg, _, _, _ = g.forward_batch(toks[pos:pos + 1], [0], [0])
                want = o.step(toks[pos:pos + 1], [0], [0])
                assert same_bits(lg, want), f"position {pos}"
            assert g.slot_length(0) == len(toks)
        ref = fix["window_logits"].astype(np.float64)
        last = lg[0].astype(np.float64)
        assert int(np.argmax(last)) == int(np.argmax(ref))
        assert last @ ref / np.linalg.norm(last) / np.linalg.norm(ref) >= 0.9995
    finally:
        o.close()
        orc.lib().or_n3_set_threads(1)
