"""The SIMD tier of the CPU matmul (oracle/cpu_simd.c: Quant.MatMulRows'
SIMD branch -- Gemv.Tile4 / Tile2 / Rows with the Avx2Dot or VnniDot group
dot, src/Needle/Gemv.cs:204-317, src/Needle/Tiers.cs:23-55), the timed CPU
baseline: its int32 group sums are exact and only the float association
differs from Scalar.MatMulRows, so every output is within 2e-6 * RMS of a
float64 evaluation of the exact integers (a wrong dot or a dropped group is
orders of magnitude above that) and within 1e-4 * RMS of the oracle's scalar
order; rows outside the range stay untouched.  Every tier this CPU runs is
checked, with token counts covering 4-token tiles, a 2-token tile and
single tokens."""
import numpy as np
import pytest

TIERS = {"avx2": 1, "avx_vnni": 2}


def available():
    from oracle import oracle as O
    best = O.lib().or_simd_tier()
    return [name for name, t in TIERS.items() if t <= best]


def exact64(w, scales, q, qs):
    rows, cols = w.shape
    tokens = q.shape[0]
    d = np.einsum("tgk,ngk->tng", q.reshape(tokens, -1, 32).astype(np.int64),
                  w.reshape(rows, -1, 32).astype(np.int64)).astype(np.float64)
    hs = scales.view(np.float16).astype(np.float64)
    return (d * hs[None]).sum(axis=2) * qs.astype(np.float64)[:, None]


@pytest.mark.parametrize("tier", ["avx2", "avx_vnni"])
@pytest.mark.parametrize("tokens,rows,cols", [(1, 4096, 1024), (3, 2048, 2048), (4, 64, 256), (7, 37, 512),
                                              (16, 130, 2048), (2, 5, 32), (9, 3, 8192)])
def test_simd_matmul_against_exact_integers(orc, tier, tokens, rows, cols):
    if tier not in available():
        pytest.skip(f"this CPU does not run the {tier} tier")
    st = orc.state(tokens * 31 + rows + cols)
    w = orc.synth_int8(st, rows * cols).reshape(rows, cols)
    scales = orc.synth_half_uniform(st, rows * cols // 32, 0.002, 0.02).reshape(rows, cols // 32)
    x = orc.synth_normal(st, tokens * cols).reshape(tokens, cols)
    q, qs = orc.quantize_rows(x)
    ldy = rows + 2
    y = np.full((tokens, ldy), 7.0, dtype=np.float32)
    orc.lib().or_simd_matmul_i8(TIERS[tier], orc.p(w), orc.p(scales), rows, cols, orc.p(q), orc.p(qs), tokens,
                                orc.p(y), ldy, 0, rows)
    want = exact64(w, scales, q, qs)
    rms = float(np.sqrt(np.mean(want ** 2)))
    assert np.max(np.abs(y[:, :rows] - want)) <= 2e-6 * rms
    assert np.all(y[:, rows:] == 7.0)
    ref = np.zeros((tokens, rows), dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, ref, rows, 0, rows)
    assert np.max(np.abs(y[:, :rows].astype(np.float64) - ref)) <= 1e-4 * rms


def test_simd_pool_row_split(orc):
    """The pool's 4-row-block split (MatMulBatch.RunShard) over 5 members
    gives the single-member result bit for bit on a range of whole blocks
    (a range ending inside a block runs its tail rows as Gemv.Single, whose
    sums associate differently), and leaves the other rows alone."""
    if not available():
        pytest.skip("no SIMD tier on this CPU")
    tier = orc.lib().or_simd_tier()
    st = orc.state(99)
    rows, cols, tokens = 203, 1024, 3
    w = orc.synth_int8(st, rows * cols).reshape(rows, cols)
    scales = orc.synth_half_uniform(st, rows * cols // 32, 0.002, 0.02).reshape(rows, cols // 32)
    q, qs = orc.quantize_rows(orc.synth_normal(st, tokens * cols).reshape(tokens, cols))
    one = np.zeros((tokens, rows), dtype=np.float32)
    orc.lib().or_simd_matmul_i8(tier, orc.p(w), orc.p(scales), rows, cols, orc.p(q), orc.p(qs), tokens, orc.p(one),
                                rows, 0, rows)
    assert orc.lib().or_baseline_start(5) == 5
    try:
        many = np.full((tokens, rows), 3.0, dtype=np.float32)
        orc.lib().or_baseline_simd_matmul_i8(tier, orc.p(w), orc.p(scales), rows, cols, orc.p(q), orc.p(qs), tokens,
                                             orc.p(many), rows, 8, 188)
    finally:
        orc.lib().or_baseline_stop()
    assert np.array_equal(many[:, 8:188], one[:, 8:188])
    assert np.all(many[:, :8] == 3.0) and np.all(many[:, 188:] == 3.0)
