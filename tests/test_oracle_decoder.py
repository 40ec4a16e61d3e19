"""CPU checks of the oracle's synthetic decoder (the CPU path the GPU decode
loop is compared against): each canonical element-wise operation against
float64 mathematics, top-k against the reference restatement of
TopKLogSoftmax, and the decoder's structural invariants -- batched == single
(tests/Needle.Tests/BatchedDecodeTests.cs:61-132), chunked prefill ==
sequential feeding (tests/Needle.Tests/ChunkParityTests.cs:22-39) and a beam
search that re-prefills every hypothesis from scratch (no slot reuse or KV
copies) giving the same winner as the slot-tracking driver."""
import ctypes as C
import math

import numpy as np
import pytest

from needle_cs_amd.decoder import random_prompt, synthetic_model

TINY = dict(layers=2, d=128, heads=2, kv_heads=2, head_dim=64, ffn=256, vocab=300, theta=10000.0, eps=1e-5)
GQA = dict(layers=2, d=256, heads=6, kv_heads=2, head_dim=64, ffn=512, vocab=1000, theta=10000.0, eps=1e-5)


def test_log_poly_against_log(orc):
    xs = np.concatenate([np.linspace(1.0, 4.0, 3001), np.geomspace(1.0, 1e30, 3001), np.geomspace(1e-30, 1.0, 3001)])
    for x in xs.astype(np.float32):
        got = orc.lib().or_log_poly(float(x))
        want = math.log(float(x))
        assert abs(got - want) <= 3e-7 * max(1.0, abs(want)), (x, got, want)


def test_add_rmsnorm_quant_against_float64(orc):
    st = orc.state(21)
    d = 1024
    x = orc.synth_normal(st, d) * 37.0
    delta = orc.synth_normal(st, d)
    gain = (orc.synth_normal(st, d) * 0.1 + 1.0).astype(np.float32)
    xs = x.copy()
    h = np.zeros(d, dtype=np.float32)
    q = np.zeros(d, dtype=np.int8)
    s = orc.lib().or_add_rmsnorm_quant(orc.p(xs), orc.p(delta), orc.p(gain), d, 1e-5, orc.p(h), orc.p(q))
    x64 = x.astype(np.float64) + delta.astype(np.float64)
    assert np.array_equal(xs, (x + delta).astype(np.float32))
    want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-5) * gain
    assert np.max(np.abs(h - want)) <= 2e-6 * np.max(np.abs(want))
    q2 = np.zeros(d, dtype=np.int8)
    assert orc.lib().or_quantize_int8(orc.p(h), d, orc.p(q2)) == s and np.array_equal(q, q2)


def test_rope_table_and_rotation(orc):
    pos, dim = 300, 64
    c = np.zeros(pos * 32, dtype=np.float32)
    s = np.zeros(pos * 32, dtype=np.float32)
    orc.lib().or_rope_table(pos, dim, 10000.0, orc.p(c), orc.p(s))
    ang = np.arange(pos)[:, None] * 10000.0 ** (-2.0 * np.arange(32)[None, :] / dim)
    assert np.max(np.abs(c.reshape(pos, 32) - np.cos(ang))) <= 6e-8
    assert np.max(np.abs(s.reshape(pos, 32) - np.sin(ang))) <= 6e-8
    st = orc.state(5)
    v = orc.synth_normal(st, 64)
    p = 123
    out = v.copy()
    orc.lib().or_rope_head(orc.p(out), orc.p(c[p * 32:]), orc.p(s[p * 32:]))
    z = (v[:32] + 1j * v[32:]).astype(np.complex128) * np.exp(1j * ang[p])
    assert np.max(np.abs(out[:32] - z.real)) <= 1e-6 and np.max(np.abs(out[32:] - z.imag)) <= 1e-6


def test_swiglu_against_float64(orc):
    st = orc.state(8)
    n = 4096
    g = orc.synth_normal(st, n) * 20
    u = orc.synth_normal(st, n) * 20
    a = np.zeros(n, dtype=np.float32)
    q = np.zeros(n, dtype=np.int8)
    orc.lib().or_swiglu_quant(orc.p(g), orc.p(u), n, orc.p(a), orc.p(q))
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1.0 + np.exp(-np.clip(g64, -88, 88))) * u64
    assert np.max(np.abs(a - want) / np.maximum(1.0, np.abs(want))) <= 2e-6


@pytest.mark.parametrize("k", [1, 3, 5])
def test_topk_lse_against_reference_restatement(orc, k):
    st = orc.state(90 + k)
    n = 32000
    for trial in range(3):
        x = orc.synth_normal(st, n) * (3 + 10 * trial)
        x[7] = x[11] = np.max(x)  # a tie: lower id first
        idx = np.zeros(k, dtype=np.int32)
        lp = np.zeros(k, dtype=np.float32)
        orc.lib().or_topk_lse(orc.p(x), n, k, 1, orc.p(idx), orc.p(lp))
        ridx = np.zeros(k, dtype=np.int32)
        rlp = np.zeros(k, dtype=np.float32)
        orc.lib().or_topk_log_softmax(orc.p(x), n, k, orc.p(ridx), orc.p(rlp), None, 1)
        assert np.array_equal(idx, ridx)
        assert np.max(np.abs(lp - rlp)) <= 2e-5


@pytest.fixture(scope="module")
def tiny(orc):
    model = synthetic_model(TINY, 4242)
    dec = orc.CpuDecoder(model, slots=4, capacity=64)
    yield model, dec
    dec.close()


@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_decoder_batched_equals_single(orc, dims):
    model = synthetic_model(dims, 4243)
    a = orc.CpuDecoder(model, slots=3, capacity=32)
    b = orc.CpuDecoder(model, slots=3, capacity=32)
    prompts = [random_prompt(s, 6, dims["vocab"]) for s in (1, 2, 3)]
    for i, pr in enumerate(prompts):  # prefill each slot alone in both
        for dec in (a, b):
            dec.forward(pr, [i] * 6, np.arange(6))
    toks = [p[-1] for p in prompts]
    lg_batch, _, _ = a.forward(toks, [0, 1, 2], [6, 6, 6])
    for i in range(3):
        lg_one, _, _ = b.forward([toks[i]], [i], [6])
        assert np.array_equal(lg_one[0].view(np.uint32), lg_batch[i].view(np.uint32))
    a.close()
    b.close()


def test_decoder_chunked_prefill_equals_sequential(orc, tiny):
    model, _ = tiny
    a = orc.CpuDecoder(model, slots=1, capacity=32)
    b = orc.CpuDecoder(model, slots=1, capacity=32)
    pr = random_prompt(9, 10, TINY["vocab"])
    lg_chunk, _, _ = a.forward(pr, [0] * 10, np.arange(10))
    for i in range(10):
        lg_i, _, _ = b.forward([pr[i]], [0], [i])
        assert np.array_equal(lg_i[0].view(np.uint32), lg_chunk[i].view(np.uint32))
    a.close()
    b.close()


def _beam_from_scratch(orc, model, prompt, width, max_new, eos):
    """Whistle.BeamSearch (Whistle.Decode.cs:226-350) restated over full
    re-prefills: every hypothesis' logits come from prefilling prompt +
    tokens into a fresh cache."""
    def step_topk(tokens):
        dec = orc.CpuDecoder(model, slots=1, capacity=len(prompt) + max_new + 2)
        seq = np.concatenate([prompt, np.array(tokens, dtype=np.int32)])
        lg, _, _ = dec.forward(seq, [0] * len(seq), np.arange(len(seq)))
        dec.close()
        idx = np.zeros(width, dtype=np.int32)
        lp = np.zeros(width, dtype=np.float32)
        row = np.ascontiguousarray(lg[-1])
        orc.lib().or_topk_lse(orc.p(row), len(row), width, 1, orc.p(idx), orc.p(lp))
        return idx, lp
    live = [([], np.float32(0.0))]
    finished = []
    tops = [step_topk([])]
    for _ in range(max_new):
        cands = []
        for i, (toks, sc) in enumerate(live):
            idx, lp = tops[i]
            for k in range(width):
                cands.append((np.float32(sc + lp[k]), i, int(idx[k])))
        cands.sort(key=lambda c: -c[0])  # stable: ties keep insertion order
        kept = []
        for sc, parent, tok in cands:
            if tok == eos:
                finished.append((sc, list(live[parent][0])))
            else:
                kept.append((sc, parent, tok))
            if len(kept) >= width:
                break
        if not kept:
            break
        if len(finished) >= width:
            bf = max(np.float32(f[0]) / np.float32(len(f[1]) + 1) for f in finished)
            bl = max(np.float32(sc) / np.float32(len(live[p][0]) + 1) for sc, p, _ in kept)
            if bf >= bl:
                break
        live = [(live[p][0] + [tok], sc) for sc, p, tok in kept]
        tops = [step_topk(t) for t, _ in live]
    best, best_sc = None, -np.inf
    for sc, toks in finished:
        v = np.float32(sc) / np.float32(len(toks) + 1)
        if v > best_sc:
            best, best_sc = toks, v
    if best is None:
        for toks, sc in live:
            v = np.float32(sc) / np.float32(len(toks))
            if v > best_sc:
                best, best_sc = toks, v
    return np.array(best, dtype=np.int32), float(best_sc)


@pytest.mark.parametrize("eos", [1, 299])
def test_beam_search_matches_from_scratch_restatement(orc, tiny, eos):
    model, _ = tiny
    prompt = random_prompt(77, 7, TINY["vocab"])
    dec = orc.CpuDecoder(model, slots=3, capacity=32)
    toks, score, fed = dec.beam_search(prompt, 3, 8, eos)
    dec.close()
    want, want_score = _beam_from_scratch(orc, model, prompt, 3, 8, eos)
    assert np.array_equal(toks, want)
    assert np.float32(score) == np.float32(want_score)
    assert fed >= len(toks)
