"""The AVX2-tier row order of the oracle's Needle 3 ops (or_n3_set_tier(1):
the Vector256 sums of Ops.SumOfSquares / Ops.Dot, Ops.cs:123-205, with the
elementwise forms of the ops that own them), which the GPU engine runs,
held to the reference's own bar for a row-op tier against Scalar.cs.

The reference compares each tier's row ops with the scalar kernels on its
conformance inputs (tests/Needle.Tests/Conformance/KernelConformanceTests.cs
RowOpsConformance, :782-1000: XorShift64 seeds 0x0DD5.., FillEdges /
FillUniform, sizes 8, 24, 768) at cosine >= 0.99995 (ConformanceAssert.Parity,
Conformance.cs:197-202); the Hadamard MLP at 1e-5 of the largest magnitude
(ConformanceAssert.Close, Conformance.cs:149-161; HadamardMlpConformance,
:568-690).  The same inputs and bars are used here, tier 1 against tier 0,
and the tier-1 engine keeps the engine's structural invariants.  The
accumulation structure itself (lanes, the 16- and 8-blocks, the FMA tail,
Vector256.Sum's tree) is restated from Ops.cs by reading: without .NET its
bits cannot be compared with the reference's, only these bars.
"""
import ctypes as C
import math

import numpy as np
import pytest

from needle_cs_amd.archive import SMALL, needle3_archive
from oracle.needle3 import OracleEngine, OracleModel

F32 = np.float32


@pytest.fixture
def tiers(orc):
    yield orc
    orc.lib().or_n3_set_tier(0)


def conformance(orc, seed, n, scale, edges=True, st=None):
    st = st if st is not None else orc.state(seed)
    x = np.zeros(max(n, 1), F32)
    (orc.lib().or_fill_edges if edges else orc.lib().or_fill_uniform)(orc.p(x), max(n, 1), C.byref(st), scale)
    return x[:n], st


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def both(orc, fn):
    out = []
    for tier in (0, 1):
        orc.lib().or_n3_set_tier(tier)
        out.append(fn())
    orc.lib().or_n3_set_tier(0)
    return out


@pytest.mark.parametrize("n", [8, 24, 768, 3072])
def test_rms_fake_a8_tier_parity(tiers, n):
    orc = tiers
    x, _ = conformance(orc, 0x0DD5, n, 3.0)

    def run():
        d = np.zeros(n, F32)
        orc.lib().or_rms_fake_a8(orc.p(x), n, orc.p(d))
        return d
    scalar, tier = both(orc, run)
    assert cosine(scalar, tier) >= 0.99995


@pytest.mark.parametrize("n", [8, 24, 768])
def test_centered_rms_fake_a8_tier_parity(tiers, n):
    orc = tiers
    x, st = conformance(orc, 0x0DD6, n, 3.0)
    s, _ = conformance(orc, 0, n, 0.1, edges=False, st=st)

    def run():
        d = np.zeros(n, F32)
        orc.lib().or_centered_rms_fake_a8(orc.p(x), orc.p(s), n, orc.p(d))
        return d
    scalar, tier = both(orc, run)
    assert cosine(scalar, tier) >= 0.99995


@pytest.mark.parametrize("n", [8, 24, 768])
def test_post_norm_add_tier_parity(tiers, n):
    orc = tiers
    st = orc.state(0x0DD8)
    residual, st = conformance(orc, 0, n, 1.0, edges=False, st=st)
    x, st = conformance(orc, 0, n, 3.0, st=st)
    s, _ = conformance(orc, 0, n, 0.1, edges=False, st=st)

    def run():
        r = residual.copy()
        orc.lib().or_post_norm_add(orc.p(r), orc.p(x), orc.p(s), F32(0.7), n)
        return r
    scalar, tier = both(orc, run)
    assert cosine(scalar, tier) >= 0.99995


@pytest.mark.parametrize("n", [8, 24, 48, 768])
def test_zero_centered_rms_and_rms_unit_tier_parity(tiers, n):
    orc = tiers
    x, st = conformance(orc, 0x0DDC, n, 3.0)
    s, _ = conformance(orc, 0, n, 0.1, edges=False, st=st)

    def run():
        z = np.zeros(n, F32)
        u = np.zeros(n, F32)
        orc.lib().or_zero_centered_rms(orc.p(x), orc.p(s), n, orc.p(z))
        orc.lib().or_rms_unit(orc.p(x), n, orc.p(u))
        return z, u
    (z0, u0), (z1, u1) = both(orc, run)
    assert cosine(z0, z1) >= 0.99995
    assert cosine(u0, u1) >= 0.99995


@pytest.mark.parametrize("n", [1, 7, 8, 31, 32, 48, 768, 3072])
def test_dot_tier_within_float_rounding(tiers, n):
    """Dot of two rows: the two orders differ by rounding only (bounded by
    n ulps of the sum of |products|)."""
    orc = tiers
    a, st = conformance(orc, 0x0DDD, n, 2.0, edges=False)
    b, _ = conformance(orc, 0, n, 2.0, edges=False, st=st)
    s0, s1 = both(orc, lambda: orc.lib().or_dot(orc.p(a), orc.p(b), n))
    bound = n * float(np.finfo(F32).eps) * float(np.sum(np.abs(a.astype(np.float64) * b)))
    assert abs(s0 - s1) <= bound
    exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(s1 - exact) <= bound


def test_v256_sum_closed_forms(orc):
    """Exact cases: every partial sum representable, so the order cannot
    show; and one whose value the order fixes: 2^24 followed by 31 ones,
    which a sequential sum reduces to 2^24 and the lanes and tree to
    2^24 + 30."""
    x = np.ones(96, F32)
    assert orc.lib().or_v256_sum(orc.p(x), None, 96) == 96.0
    y = np.arange(1, 41, dtype=F32)
    assert orc.lib().or_v256_sum(orc.p(y), None, 40) == float(np.sum(y.astype(np.int64) ** 2))
    big = np.ones(32, F32)
    big[0] = F32(2.0 ** 24)
    seq = F32(0)
    for v in big:
        seq = F32(seq + v)
    assert seq == F32(2.0 ** 24)  # the sequential order loses every one (2^24 + 1 ties to 2^24)
    # each element is one lane's only term; v0 = (2^24 + 1) + (1 + 1) = 2^24 + 2
    # (the first sum ties to even), v1..v7 = 4; ((v0 + v1) + (v2 + v3)) +
    # ((v4 + v5) + (v6 + v7)) = (2^24 + 14) + 16, all exact
    t = orc.lib().or_v256_sum(orc.p(big), orc.p(np.ones(32, F32)), 32)
    assert t == 2.0 ** 24 + 30


def test_hadamard_mlp_tier_close(tiers):
    """HadamardMlpConformance's bar (1e-5 of the largest magnitude) between
    the tiers, on Needle 3's MLP shape (768 hidden, 32 x 32)."""
    orc = tiers
    rng = np.random.default_rng(0x1A5E)
    dim, rows, cols = 768, 32, 32
    width = rows * cols
    N = orc.N3
    keep = []

    def arr(a):
        a = np.ascontiguousarray(a, F32)
        keep.append(a)
        return a.ctypes.data
    w = N.Mlp()
    w.d1, w.d2, w.b2 = arr(rng.uniform(0.5, 1.5, width)), arr(rng.uniform(0.5, 1.5, width)), arr(rng.uniform(-.1, .1, width))
    w.d3, w.d4 = arr(rng.uniform(0.5, 1.5, width)), arr(rng.uniform(0.2, 0.8, width))
    for name, n in (("w1a", rows), ("w1b", cols), ("w2a", rows), ("w2b", cols), ("w3a", rows), ("w3b", cols)):
        setattr(w, name, arr(rng.standard_normal(n * n) / math.sqrt(n)))
    w.cond_v, w.cond_u = arr(rng.standard_normal(dim * 8) * 0.05), arr(rng.uniform(-0.2, 0.2, 8 * width))
    pre = np.ascontiguousarray(rng.uniform(-0.2, 0.2, dim), F32)
    pa = np.ascontiguousarray(rng.permutation(width), np.int32)
    pb = np.ascontiguousarray(rng.permutation(width), np.int32)
    resid = np.ascontiguousarray(rng.standard_normal(dim), F32)

    def run():
        r = resid.copy()
        orc.lib().or_hadamard_mlp(C.byref(w), orc.p(pre), orc.p(pa), orc.p(pb), dim, rows, cols, orc.p(r))
        return r
    scalar, tier = both(orc, run)
    magnitude = max(1.0, float(np.max(np.abs(scalar))))
    assert np.max(np.abs(scalar.astype(np.float64) - tier)) <= 1e-5 * magnitude
    assert not np.array_equal(scalar.view(np.uint32), tier.view(np.uint32))  # the tiers do differ


@pytest.fixture(scope="module")
def small(orc):
    return OracleModel(orc, needle3_archive(SMALL, 3))


def toks(seed, n):
    return np.random.default_rng(seed).integers(0, SMALL["vocab"], n).astype(np.int32)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, F32).view(np.uint32), np.asarray(b, F32).view(np.uint32))


def test_tier_engine_batched_single_chunk_sequential(tiers, small):
    """The tier-1 engine keeps batched == single and chunk == sequential
    (BatchedDecodeTests.cs:61-132, ChunkParityTests.cs:22-39), and its logits
    differ from tier 0's only by the tiers' rounding (same argmax here)."""
    orc = tiers
    orc.lib().or_n3_set_tier(1)
    a = OracleEngine(orc, small, slots=2, capacity=96, max_chunks=8)
    b = OracleEngine(orc, small, slots=2, capacity=96, max_chunks=8)
    p0, p1 = toks(1, 7), toks(2, 9)
    both_rows = a.step(np.r_[p0, p1], [0] * 7 + [1] * 9, [6, 15])
    seq = np.concatenate([b.step(p0[i:i + 1], [0], [0]) for i in range(7)])
    s1 = b.step(p1, [1] * 9, [8])
    assert bits_equal(both_rows, np.r_[seq[-1:], s1])
    a.close()
    b.close()
    orc.lib().or_n3_set_tier(0)
    c = OracleEngine(orc, small, slots=1, capacity=96, max_chunks=8)
    scalar = c.step(p0, [0] * 7, [6])
    c.close()
    assert not bits_equal(scalar, seq[-1:])
    assert cosine(scalar[0], seq[-1]) >= 0.999
