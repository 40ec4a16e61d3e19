"""GPU masked head: nhip_argmax_masked_dev (Ops.ArgMaxMasked,
src/Needle/Ops.cs:1223-1266) against the oracle's restatement, and the
decoder's grammar-constrained step (sparse LM head over the allowed vocab
tiles, then the masked argmax) against the CPU path's full logits."""
import numpy as np
import pytest

from needle_cs_amd.decoder import GpuDecoder, random_prompt, synthetic_model
from test_decoder_gpu import GQA, TINY, WIDE

pytestmark = pytest.mark.gpu


def random_masks(rng, rows, words, density):
    bits = rng.random((rows, words * 32)) < density
    return np.packbits(bits.reshape(rows, words, 32)[:, :, ::-1], axis=2).view(">u4").reshape(rows, words).astype(
        np.uint32)


def oracle_rows(orc, x, masks, words, length):
    return [orc.lib().or_argmax_masked(orc.p(np.ascontiguousarray(x[r])), orc.p(np.ascontiguousarray(masks[r])),
                                       words, length) for r in range(x.shape[0])]


@pytest.mark.parametrize("length", [1, 31, 300, 32000, 32003])
@pytest.mark.parametrize("density", [0.0, 0.0005, 0.05, 1.0])
def test_argmax_masked_dev_matches_oracle(hip, orc, length, density):
    rng = np.random.default_rng(length + int(density * 1e4))
    rows, words = 6, (length + 31) // 32 + 1
    x = rng.integers(-40, 40, (rows, words * 32)).astype(np.float32)  # many ties
    x[rng.random(x.shape) < 0.03] = np.nan
    x[rng.random(x.shape) < 0.03] = -np.inf
    x[1, :] = -np.inf                           # a row with nothing above -inf
    x[2, 5] = np.inf
    masks = random_masks(rng, rows, words, density)
    masks[3, :] = 0                             # a row with nothing allowed
    dx, dm = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(masks)
    di, dv = hip.DeviceBuffer(rows * 4), hip.DeviceBuffer(rows * 4)
    hip.check(hip.lib().nhip_argmax_masked_dev(dx.ptr, x.shape[1], dm.ptr, words, words, length, rows, di.ptr, dv.ptr,
                                               None))
    got = di.download(np.int32)
    want = oracle_rows(orc, x, masks, words, length)
    assert list(got) == want
    vals = dv.download(np.float32)
    for r, i in enumerate(want):
        assert (vals[r] == -np.inf) if i < 0 else (vals[r] == x[r, i])


@pytest.mark.parametrize("dims,density", [(TINY, 0.02), (TINY, 1.0), (GQA, 0.005), (WIDE, 0.0005), (WIDE, 0.3)],
                         ids=["tiny-sparse", "tiny-full", "gqa-sparse", "wide-sparse", "wide-dense"])
def test_decoder_masked_step_matches_cpu(hip, orc, dims, density):
    """Decode rows from three slots with per-row grammar masks: the chosen ids
    and logits equal ArgMaxMasked over the CPU path's full logits; a row with
    an empty mask gets -1; a dense forward afterwards is still exact."""
    model = synthetic_model(dims, 9100)
    vocab = dims["vocab"]
    gpu = GpuDecoder(model, slots=3, capacity=40, max_rows=16)
    cpu = orc.CpuDecoder(model, slots=3, capacity=40, threads=8)
    prompt = random_prompt(9, 12, vocab)
    for g in (gpu, cpu):
        g.forward(prompt, [0] * 12, np.arange(12), k=1)
        g.copy_slot(1, 0, 12)
        g.copy_slot(2, 0, 12)
    rng = np.random.default_rng(len(prompt) + vocab)
    words = (vocab + 31) // 32
    toks = np.array([5, 17, 29], dtype=np.int32)
    for step in range(3):
        pos = [12 + step] * 3
        masks = random_masks(rng, 3, words, density)
        if step == 1:
            masks[2, :] = 0
        best, val = gpu.forward_masked(toks, [0, 1, 2], pos, masks)
        lg, _, _ = cpu.forward(toks, [0, 1, 2], pos, k=1)
        want = oracle_rows(orc, lg, masks, words, vocab)
        assert list(best) == want, step
        for r, i in enumerate(want):
            if i >= 0:
                assert np.float32(val[r]).view(np.uint32) == np.float32(lg[r, i]).view(np.uint32)
        toks = np.array([b if b >= 0 else 7 for b in best], dtype=np.int32)
    lg_g, _, _ = gpu.forward(toks, [0, 1, 2], [15] * 3, k=1)
    lg_c, _, _ = cpu.forward(toks, [0, 1, 2], [15] * 3, k=1)
    assert np.array_equal(lg_g.view(np.uint32), lg_c.view(np.uint32))
    gpu.close()
    cpu.close()
