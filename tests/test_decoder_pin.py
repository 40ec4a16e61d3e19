"""Pins the composition of the oracle's decoder (or_decoder_forward, the CPU
path every GPU decoder test and the benchmark's token comparison are checked
against) with an independent float64 forward written from the model's
mathematics (tests/decoder_f64.py): same int8 weights times their fp16
scales, same activation-quantization points, float64 everywhere else.

Bound, over every row of a prefill and of ragged decode steps in two slots
(RMS = RMS of all float64 logits, row error = max |oracle - f64| of the row):
  * at least 60% of the rows within 1e-4 * RMS (measured: about 1e-6 * RMS,
    float32 roundings only);
  * every row within 0.15 * RMS: where float32 and float64 land on opposite
    sides of a rounding tie, one quantized activation differs by one step,
    which moves the rows that depend on it by up to about 0.07 * RMS at the
    1024 / 4096 widths (3 of 13 rows there, none at the small widths);
  * identical argmax on at least 95% of the rows (measured: all).

Negative controls: each composition mistake planted in the float64 forward
(swapped gate/up halves, a dropped residual, RoPE applied to the values, the
wrong kv head, no final norm, RoPE one position off, no 1/sqrt(d) score
scale) must break the bound, so the comparison would see the same mistake in the
oracle.  The random-weight model saturates the softmax and RoPE is
shift-invariant, so a few mistakes (no score scale, RoPE one position off)
move only some rows; every planted mistake still moves some row by more than
0.9 * RMS."""
import numpy as np
import pytest

from decoder_f64 import MISTAKES, Float64Decoder
from needle_cs_amd.decoder import random_prompt, synthetic_model

TINY = dict(layers=2, d=128, heads=2, kv_heads=2, head_dim=64, ffn=256, vocab=300, theta=10000.0, eps=1e-5)
GQA = dict(layers=2, d=256, heads=6, kv_heads=2, head_dim=64, ffn=512, vocab=1000, theta=10000.0, eps=1e-5)
# the benchmark decoder's widths (d 1024, 16 x 64 heads, SwiGLU 4096, vocab
# 32000), two layers
WIDE = dict(layers=2, d=1024, heads=16, kv_heads=16, head_dim=64, ffn=4096, vocab=32000, theta=10000.0, eps=1e-5)

CLEAN, CLEAN_SHARE, WORST, ARGMAX_SHARE = 1e-4, 0.6, 0.15, 0.95


def run_both(orc, dims, seed, mistake=None, prompts=(12, 5), steps=4, threads=1):
    """Prefills one prompt per slot, then `steps` ragged decode steps over
    both slots feeding the oracle's argmax; returns the stacked logits of
    both sides."""
    model = synthetic_model(dims, seed)
    cpu = orc.CpuDecoder(model, slots=len(prompts), capacity=48, threads=threads)
    ref = Float64Decoder(model, slots=len(prompts), mistake=mistake)
    got, want, toks, pos = [], [], [], []
    for slot, n in enumerate(prompts):
        pr = random_prompt(3 + slot, n, dims["vocab"])
        a, _, _ = cpu.forward(pr, [slot] * n, np.arange(n))
        got.append(a)
        want.append(ref.forward(pr, [slot] * n, np.arange(n)))
        toks.append(int(np.argmax(a[-1])))
        pos.append(n)
    slots = list(range(len(prompts)))
    for _ in range(steps):
        a, _, _ = cpu.forward(toks, slots, pos)
        got.append(a)
        want.append(ref.forward(toks, slots, pos))
        toks = [int(t) for t in np.argmax(a, axis=1)]
        pos = [p + 1 for p in pos]
    cpu.close()
    return np.concatenate(got).astype(np.float64), np.concatenate(want)


def row_errors(got, want):
    return np.max(np.abs(got - want), axis=1) / np.sqrt(np.mean(want ** 2))


def within_bound(got, want) -> bool:
    err = row_errors(got, want)
    argmax_share = np.mean(np.argmax(got, axis=1) == np.argmax(want, axis=1))
    return bool(np.mean(err <= CLEAN) >= CLEAN_SHARE and np.max(err) <= WORST and argmax_share >= ARGMAX_SHARE)


@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_oracle_decoder_matches_float64_forward(orc, dims):
    got, want = run_both(orc, dims, 4250)
    assert np.max(row_errors(got, want)) <= CLEAN  # no tie flips at these widths
    assert within_bound(got, want)


def test_oracle_decoder_matches_float64_forward_wide(orc):
    got, want = run_both(orc, WIDE, 4251, prompts=(6, 3), steps=2, threads=8)
    assert within_bound(got, want)


@pytest.mark.parametrize("mistake", MISTAKES)
@pytest.mark.parametrize("dims", [TINY, GQA], ids=["tiny", "gqa"])
def test_planted_composition_mistake_is_detected(orc, dims, mistake):
    got, want = run_both(orc, dims, 4250, mistake=mistake)
    assert not within_bound(got, want), mistake
    assert np.max(row_errors(got, want)) > 0.9, mistake
