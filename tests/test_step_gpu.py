"""The batched engine's step API on the GPU (nhip_decoder_step and the slot
operations; BatchedEngine.ForwardBatch / ResetSlot / MarkSlot / RewindSlot,
src/Needle/BatchEngine.cs:25-39, src/Needle/Engine.cs:2227-2350) and greedy
decoding (nhip_decoder_greedy; ToolCaller.Complete, src/Needle/ToolCaller.cs:
59-77) against the oracle's CPU path on the same synthetic weights: head-row
logits, top-k and Ops.ArgMax bit-identical with the same rows of a full
forward, rewind + re-feed equal to a fresh prefill, and greedy token streams
identical."""
import numpy as np
import pytest

from needle_cs_amd.decoder import GpuDecoder, random_prompt, synthetic_model

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, d=128, heads=2, kv_heads=2, head_dim=64, ffn=256, vocab=300, theta=10000.0, eps=1e-5)
GQA = dict(layers=2, d=256, heads=6, kv_heads=2, head_dim=64, ffn=512, vocab=1000, theta=10000.0, eps=1e-5)
WIDE = dict(layers=2, d=1024, heads=16, kv_heads=16, head_dim=64, ffn=4096, vocab=32000, theta=10000.0, eps=1e-5)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def argmax_rows(orc, lg):
    return np.array([orc.lib().or_argmax(orc.p(np.ascontiguousarray(r)), lg.shape[1]) for r in lg], dtype=np.int32)


@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_head_rows_equal_the_same_rows_of_a_full_forward(hip, orc, dims):
    model = synthetic_model(dims, 7301)
    gpu = GpuDecoder(model, slots=3, capacity=64, max_rows=24)
    cpu = orc.CpuDecoder(model, slots=3, capacity=64)
    prompts = [random_prompt(40 + s, n, dims["vocab"]) for s, n in zip(range(3), (9, 4, 20))]
    for slot, pr in enumerate(prompts):
        lg, idx, lp, am = gpu.step(pr, [slot] * len(pr), [len(pr) - 1], k=3, argmax=True)
        want, widx, wlp = cpu.forward(pr, [slot] * len(pr), np.arange(len(pr)), k=3)
        assert np.array_equal(bits(lg[0]), bits(want[-1])), slot
        assert np.array_equal(idx[0], widx[-1]) and np.array_equal(bits(lp[0]), bits(wlp[-1]))
        assert am[0] == argmax_rows(orc, want[-1:])[0]
        assert gpu.slot_length(slot) == len(pr)
    # ragged rows: two of slot 0, one of slot 2, three of slot 1; heads in
    # any order, a row twice
    toks = np.array([11, 12, 13, 14, 15, 16], dtype=np.int32)
    row_slots = [0, 0, 2, 1, 1, 1]
    pos = [9, 10, 20, 4, 5, 6]
    heads = [5, 0, 2, 2]
    lg, idx, lp, am = gpu.step(toks, row_slots, heads, k=2, argmax=True)
    want, widx, wlp = cpu.forward(toks, row_slots, pos, k=2)
    assert np.array_equal(bits(lg), bits(want[heads]))
    assert np.array_equal(idx, widx[heads]) and np.array_equal(bits(lp), bits(wlp[heads]))
    assert np.array_equal(am, argmax_rows(orc, want[heads]))
    assert [gpu.slot_length(s) for s in range(3)] == [11, 7, 21]
    # no head rows: only the caches and lengths move
    lg, _, _, _ = gpu.step(toks[:1], [2], [])
    assert lg.shape == (0, dims["vocab"]) and gpu.slot_length(2) == 22
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_rewind_and_refeed_equals_fresh_prefill(hip, orc, dims):
    model = synthetic_model(dims, 7302)
    p = random_prompt(50, 10, dims["vocab"])
    q1 = random_prompt(51, 5, dims["vocab"])
    q2 = random_prompt(52, 5, dims["vocab"])
    gpu = GpuDecoder(model, slots=2, capacity=48, max_rows=16)
    gpu.step(p, [1] * 10, [9])
    gpu.slot_mark(1)
    for t in q1:  # decode steps past the mark
        gpu.step([t], [1], [0])
    assert gpu.slot_length(1) == 15
    gpu.slot_rewind(1)
    assert gpu.slot_length(1) == 10
    got = np.concatenate([gpu.step([t], [1], [0], k=2)[0] for t in q2])
    fresh = GpuDecoder(model, slots=1, capacity=48, max_rows=16)
    seq = np.concatenate([p, q2])
    want_gpu, _, _, _ = fresh.step(seq, [0] * 15, list(range(10, 15)))
    cpu = orc.CpuDecoder(model, slots=1, capacity=48)
    want, _, _ = cpu.forward(seq, [0] * 15, np.arange(15))
    assert np.array_equal(bits(got), bits(want[10:]))
    assert np.array_equal(bits(want_gpu), bits(want[10:]))
    # reset: the slot starts over at position 0
    gpu.slot_reset(1)
    lg, _, _, _ = gpu.step(seq, [1] * 15, [14])
    assert np.array_equal(bits(lg[0]), bits(want[14])) and gpu.slot_length(1) == 15
    # a copied slot takes the copied length (Engine.CopyFrom)
    gpu.copy_slot(0, 1, 12)
    assert gpu.slot_length(0) == 12
    gpu.close()
    fresh.close()
    cpu.close()


def test_step_rejects_bad_rows(hip):
    model = synthetic_model(TINY, 7303)
    gpu = GpuDecoder(model, slots=2, capacity=8, max_rows=8)
    with pytest.raises(RuntimeError, match="contiguous run"):
        gpu.step([5, 6, 7], [0, 1, 0], [2])
    with pytest.raises(RuntimeError, match="head row"):
        gpu.step([5, 6], [0, 0], [2])
    with pytest.raises(RuntimeError, match="capacity"):
        gpu.step([5] * 6, [1] * 6, [5])
        gpu.step([5] * 3, [1] * 3, [2])
    assert gpu.slot_length(0) == 0  # rejected steps change nothing
    gpu.close()


def test_greedy_stream_wide_64_tokens(hip, orc):
    """64 greedy tokens at the benchmark decoder's widths (two layers):
    Ops.ArgMax on the device every step, the same stream as the CPU path."""
    model = synthetic_model(WIDE, 7304)
    prompt = random_prompt(9, 16, WIDE["vocab"])
    gpu = GpuDecoder(model, slots=1, capacity=96, max_rows=16)
    cpu = orc.CpuDecoder(model, slots=1, capacity=96, threads=8)
    toks, stats = gpu.greedy(prompt, 64)
    want = cpu.greedy(prompt, 64)
    assert len(toks) == 64 and np.array_equal(toks, want)
    assert stats.steps == 64
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_greedy_chunked_prompt_and_stop(hip, orc, dims):
    """A 40-token prompt fed in chunks of 16 rows; the stream stops before
    the stop token."""
    model = synthetic_model(dims, 7305)
    prompt = random_prompt(10, 40, dims["vocab"])
    gpu = GpuDecoder(model, slots=2, capacity=80, max_rows=16)
    cpu = orc.CpuDecoder(model, slots=1, capacity=80)
    toks, _ = gpu.greedy(prompt, 24)
    want = cpu.greedy(prompt, 24)
    assert np.array_equal(toks, want)
    stop = int(want[6])
    first = int(np.argmax(want == stop))
    toks, _ = gpu.greedy(prompt, 24, stop=stop)
    assert np.array_equal(toks, want[:first])
    assert np.array_equal(cpu.greedy(prompt, 24, stop=stop), want[:first])
    gpu.close()
    cpu.close()
