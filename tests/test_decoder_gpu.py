"""GPU decode loop (nhip_decoder_*) against the oracle's CPU path on the same
synthetic weights: logits and top-k bit-identical per forward, and beam
search producing identical token streams and scores."""
import numpy as np
import pytest

from needle_cs_amd.decoder import GpuDecoder, random_prompt, synthetic_model

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, d=128, heads=2, kv_heads=2, head_dim=64, ffn=256, vocab=300, theta=10000.0, eps=1e-5)
GQA = dict(layers=2, d=256, heads=6, kv_heads=2, head_dim=64, ffn=512, vocab=1000, theta=10000.0, eps=1e-5)
ODD = dict(layers=1, d=96, heads=1, kv_heads=1, head_dim=64, ffn=160, vocab=301, theta=10000.0, eps=1e-5)
WIDE = dict(layers=2, d=1024, heads=16, kv_heads=16, head_dim=64, ffn=4096, vocab=32000, theta=10000.0, eps=1e-5)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("capacity", [64, 600])
@pytest.mark.parametrize("max_chunks", [1, 64])
@pytest.mark.parametrize("dims", [TINY, GQA, ODD], ids=["tiny", "gqa", "odd"])
def test_forward_bit_identical(hip, orc, dims, max_chunks, capacity):
    """Capacity 64: decode steps run the whole-row attention with the
    RoPE/quantize/KV write folded in; 600 (over 512 positions): the separate
    post-processing kernel, the chunk kernel and the merge."""
    model = synthetic_model(dims, 7001)
    gpu = GpuDecoder(model, slots=4, capacity=capacity, max_rows=40, max_chunks=max_chunks)
    cpu = orc.CpuDecoder(model, slots=4, capacity=capacity, max_chunks=max_chunks)
    prompts = [random_prompt(10 + s, n, dims["vocab"]) for s, n in zip(range(3), (33, 5, 12))]
    for slot, pr in enumerate(prompts):  # prefill (32+ rows use the prefill matmul)
        pos = np.arange(len(pr))
        lg_g, ig, lpg = gpu.forward(pr, [slot] * len(pr), pos, k=3)
        lg_c, ic, lpc = cpu.forward(pr, [slot] * len(pr), pos, k=3)
        assert np.array_equal(bits(lg_g), bits(lg_c)), slot
        assert np.array_equal(ig, ic) and np.array_equal(bits(lpg), bits(lpc))
    gpu.copy_slot(3, 1, 5)
    cpu.copy_slot(3, 1, 5)
    toks = np.array([17, 29, 41, 53], dtype=np.int32)
    slots = [0, 1, 2, 3]
    pos = [33, 5, 12, 5]
    for step in range(3):  # ragged decode rows from four slots
        lg_g, ig, lpg = gpu.forward(toks, slots, pos, k=3)
        lg_c, ic, lpc = cpu.forward(toks, slots, pos, k=3)
        assert np.array_equal(bits(lg_g), bits(lg_c)), step
        assert np.array_equal(ig, ic) and np.array_equal(bits(lpg), bits(lpc))
        toks = ic[:, 0].copy()
        pos = [p + 1 for p in pos]
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("max_chunks", [8, 64])
@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_small_batches_sharing_slots(hip, orc, dims, max_chunks):
    """Forwards of at most 4 rows write their key/value rows inside the
    attention launch; rows of one slot at consecutive positions attend to
    each other's new positions, which the launch takes from its own results.
    Chunked prefills of 4, 3, 4 and 2 rows, then mixed batches of two slots."""
    model = synthetic_model(dims, 7004)
    gpu = GpuDecoder(model, slots=3, capacity=64, max_rows=8, max_chunks=max_chunks)
    cpu = orc.CpuDecoder(model, slots=3, capacity=64, max_chunks=max_chunks)
    prompt = random_prompt(12, 13, dims["vocab"])
    start = 0
    for n in (4, 3, 4, 2):
        for slot in (0, 1):
            toks = prompt[start:start + n]
            pos = np.arange(start, start + n)
            lg_g, ig, lpg = gpu.forward(toks, [slot] * n, pos, k=2)
            lg_c, ic, lpc = cpu.forward(toks, [slot] * n, pos, k=2)
            assert np.array_equal(bits(lg_g), bits(lg_c)), (start, slot)
            assert np.array_equal(ig, ic) and np.array_equal(bits(lpg), bits(lpc))
        start += n
    toks = np.array([5, 9, 11, 13], dtype=np.int32)
    for step in range(3):  # [slot 0, slot 0, slot 1, slot 2] and the reverse order
        p0 = 13 + 2 * step
        spec = [(0, p0), (0, p0 + 1), (1, 13 + step), (2, step)]
        if step == 1:
            spec = spec[::-1]
        slots, pos = [x[0] for x in spec], [x[1] for x in spec]
        lg_g, ig, lpg = gpu.forward(toks, slots, pos, k=2)
        lg_c, ic, lpc = cpu.forward(toks, slots, pos, k=2)
        assert np.array_equal(bits(lg_g), bits(lg_c)), step
        assert np.array_equal(ig, ic) and np.array_equal(bits(lpg), bits(lpc))
        toks = ic[:, 0].copy()
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("max_chunks", [1, 64])
@pytest.mark.parametrize("eos", [1, 7])
def test_beam_search_identical_tokens(hip, orc, eos, max_chunks):
    model = synthetic_model(TINY, 7002)
    prompt = random_prompt(5, 20, TINY["vocab"])
    gpu = GpuDecoder(model, slots=3, capacity=64, max_rows=20, max_chunks=max_chunks)
    cpu = orc.CpuDecoder(model, slots=3, capacity=64, max_chunks=max_chunks)
    tg, sg, stats = gpu.beam_search(prompt, 3, 24, eos)
    tc, sc, fed = cpu.beam_search(prompt, 3, 24, eos)
    assert np.array_equal(tg, tc)
    assert np.float32(sg) == np.float32(sc)
    assert stats.fed_rows == fed
    gpu.close()
    cpu.close()


def test_wide_layers_prefill_and_beam(hip, orc):
    """d_model 1024, 16 heads, SwiGLU 4096, vocab 32000 (two layers)."""
    model = synthetic_model(WIDE, 7003)
    prompt = random_prompt(6, 16, WIDE["vocab"])
    gpu = GpuDecoder(model, slots=3, capacity=32, max_rows=16)
    cpu = orc.CpuDecoder(model, slots=3, capacity=32, threads=8)
    lg_g, ig, lpg = gpu.forward(prompt, [0] * 16, np.arange(16), k=3)
    lg_c, ic, lpc = cpu.forward(prompt, [0] * 16, np.arange(16), k=3)
    assert np.array_equal(bits(lg_g), bits(lg_c))
    assert np.array_equal(ig, ic)
    # three decode rows: the QKV, output and down matmuls take the narrow
    # kernel with their prologues, the gate/up matmul the 16-row kernel with
    # its norm prologue and SwiGLU chain epilogue, the head (2000 tiles) the
    # separate norm launch and the plain kernel
    gpu.copy_slot(1, 0, 16)
    cpu.copy_slot(1, 0, 16)
    gpu.copy_slot(2, 0, 16)
    cpu.copy_slot(2, 0, 16)
    toks = np.array([ig[-1, 0], ig[-1, 1], ig[-1, 2]], dtype=np.int32)
    for step in range(2):
        lg_g, ig2, lpg = gpu.forward(toks, [0, 1, 2], [16 + step] * 3, k=3)
        lg_c, ic2, lpc = cpu.forward(toks, [0, 1, 2], [16 + step] * 3, k=3)
        assert np.array_equal(bits(lg_g), bits(lg_c)), step
        assert np.array_equal(ig2, ic2) and np.array_equal(bits(lpg), bits(lpc))
        toks = ic2[:, 0].copy()
    gpu.close()
    cpu.close()
    gpu = GpuDecoder(model, slots=3, capacity=32, max_rows=16)
    cpu = orc.CpuDecoder(model, slots=3, capacity=32, threads=8)
    tg, sg, _ = gpu.beam_search(prompt, 3, 4, 1)
    tc, sc, _ = cpu.beam_search(prompt, 3, 4, 1)
    assert np.array_equal(tg, tc) and np.float32(sg) == np.float32(sc)
    gpu.close()
    cpu.close()


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
def test_wide_decode_rows(hip, orc, rows):
    """Decode steps of 1-4 rows (one per slot) at d_model 1024: every token
    count of the narrow kernel's norm and quantize prologues and of the fused
    gate/up kernel, bit for bit against the oracle."""
    model = synthetic_model(WIDE, 7004)
    prompt = random_prompt(9, 8, WIDE["vocab"])
    gpu = GpuDecoder(model, slots=4, capacity=16, max_rows=8)
    cpu = orc.CpuDecoder(model, slots=4, capacity=16, threads=8)
    _, ig, _ = gpu.forward(prompt, [0] * 8, np.arange(8), k=4)
    _, ic, _ = cpu.forward(prompt, [0] * 8, np.arange(8), k=4)
    assert np.array_equal(ig, ic)
    for s in range(1, rows):
        gpu.copy_slot(s, 0, 8)
        cpu.copy_slot(s, 0, 8)
    toks = ig[-1, :rows].astype(np.int32)
    lanes = list(range(rows))
    for step in range(2):
        lg_g, ig2, lpg = gpu.forward(toks, lanes, [8 + step] * rows, k=4)
        lg_c, ic2, lpc = cpu.forward(toks, lanes, [8 + step] * rows, k=4)
        assert np.array_equal(bits(lg_g), bits(lg_c)), step
        assert np.array_equal(ig2, ic2) and np.array_equal(bits(lpg), bits(lpc))
        toks = ic2[:, 0].copy()
    gpu.close()
    cpu.close()


def test_replacing_weights_after_graph_capture(hip, orc):
    """Beam-search decode steps replay a captured graph per row count;
    weights replaced afterwards (set_layer / set_head) must be the ones the
    next search reads (the graphs holding the old pointers are dropped)."""
    model_a = synthetic_model(TINY, 7101)
    model_b = synthetic_model(TINY, 7102)
    prompt = random_prompt(8, 12, TINY["vocab"])
    gpu = GpuDecoder(model_a, slots=3, capacity=64, max_rows=16)
    gpu.beam_search(prompt, 3, 10, 1)  # captures the 1..3-row graphs
    gpu.set_model(model_b)
    cpu = orc.CpuDecoder(model_b, slots=3, capacity=64)
    tg, sg, _ = gpu.beam_search(prompt, 3, 10, 1)
    tc, sc, _ = cpu.beam_search(prompt, 3, 10, 1)
    assert np.array_equal(tg, tc) and np.float32(sg) == np.float32(sc)
    gpu.close()
    cpu.close()


def test_config4_beam3_decode_loop_as_specified(hip, orc):
    """The benchmark decode loop as specified: 12 layers, d_model 1024, 16
    heads x 64, SwiGLU 4096, vocab 32000, int8 g32 linears, a 128-token
    prompt, beam width 3, 64 new tokens (Whistle.BeamSearch,
    src/Needle/Whistle.Decode.cs:226-350) - the same model, prompt and search
    bench.py times.  Token stream and score identical to the oracle's scalar
    order; then 64 greedy tokens from the same prompt (Engine.Greedy)."""
    from needle_cs_amd.decoder import CONFIG4
    assert CONFIG4["layers"] == 12 and CONFIG4["d"] == 1024 and CONFIG4["vocab"] == 32000
    print("config 4: model", flush=True)
    model = synthetic_model(CONFIG4, 0x5005)
    prompt = random_prompt(0x6006, 128, CONFIG4["vocab"])
    gpu = GpuDecoder(model, slots=3, capacity=256, max_rows=128)
    cpu = orc.CpuDecoder(model, slots=3, capacity=256, threads=16)
    try:
        print("config 4: beam search", flush=True)
        tg, sg, stats = gpu.beam_search(prompt, 3, 64, 1)
        tc, sc, fed = cpu.beam_search(prompt, 3, 64, 1)
        assert len(tg) == 64
        assert np.array_equal(tg, tc) and np.float32(sg) == np.float32(sc)
        assert stats.fed_rows == fed
        print("config 4: greedy", flush=True)
        g1, gs = gpu.greedy(prompt, 64)
        c1 = cpu.greedy(prompt, 64)
        assert len(g1) == 64 and np.array_equal(g1, c1) and gs.steps == 64
    finally:
        gpu.close()
        cpu.close()
