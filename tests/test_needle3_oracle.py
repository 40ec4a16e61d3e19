"""Pins of the oracle's Needle 3 layer program (oracle/needle3_model.c).

Each row operation is checked two ways:
  * against a float64 statement of what it computes (a mistake of order,
    sign, index or a dropped term moves the result far beyond the float32
    rounding these bounds allow), and
  * where the reference's own tests fix a composition bit for bit
    (tests/Needle.Tests/KernelTests.cs:560-704, FusedKernelTests), against
    that composition.
The Kronecker-Hadamard MLP is pinned against a float64 restatement of
KernelTests.cs:360-405 (HadamardMlpTests.Reference) at the reference's shapes
and tolerance 2e-4 * (1 + |expected|), with planted mistakes that must fail.
The engram row hashing is pinned by a formulation over the whole token
sequence (the engine carries only the slot's last two tokens between steps).
Whole-engine invariants of the oracle (batched == single, chunk ==
sequential, rewind == fresh) close the file.
"""
import ctypes as C
import math

import numpy as np
import pytest
from scipy.linalg import hadamard

from needle_cs_amd.archive import SMALL, needle3_archive
from oracle.needle3 import OracleEngine, OracleModel

F32 = np.float32


def arr(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def fill(rng, n, magnitude):
    """FusedKernelTests.Fill: (u - 0.5) * magnitude."""
    return arr((rng.random(n) - 0.5) * magnitude)


def fake_a8(orc, x):
    y = arr(x).copy()
    orc.lib().or_fake_a8(orc.p(y), len(y))
    return y


def bits_equal(a, b):
    return np.array_equal(arr(a).view(np.uint32), arr(b).view(np.uint32))


def sig64(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64)))


# ------------------------------------------------ the reference's fusions --

@pytest.mark.parametrize("n", [768, 3072])
def test_rms_fake_a8_is_rms_unit_then_fake_a8(orc, n):
    x = fill(np.random.default_rng(13), n, 4.0)
    want = np.zeros(n, F32)
    orc.lib().or_rms_unit(orc.p(x), n, orc.p(want))
    want = fake_a8(orc, want)
    got = np.zeros(n, F32)
    orc.lib().or_rms_fake_a8(orc.p(x), n, orc.p(got))
    assert bits_equal(got, want)


@pytest.mark.parametrize("n", [768, 3072])
def test_centered_rms_fake_a8_is_norm_then_fake_a8(orc, n):
    rng = np.random.default_rng(17)
    x, s = fill(rng, n, 4.0), fill(rng, n, 0.5)
    want = np.zeros(n, F32)
    orc.lib().or_zero_centered_rms(orc.p(x), orc.p(s), n, orc.p(want))
    want = fake_a8(orc, want)
    got = np.zeros(n, F32)
    orc.lib().or_centered_rms_fake_a8(orc.p(x), orc.p(s), n, orc.p(got))
    assert bits_equal(got, want)


def test_gate_fake_a8_is_sigmoid_product_then_fake_a8(orc):
    n = 768
    rng = np.random.default_rng(19)
    x, g = fill(rng, n, 4.0), fill(rng, n, 4.0)
    want = fake_a8(orc, arr([x[i] * orc.lib().or_sigmoid(float(g[i])) for i in range(n)]))
    got = x.copy()
    orc.lib().or_gate_fake_a8(orc.p(got), orc.p(g), n)
    assert bits_equal(got, want)


def test_post_norm_add_is_norm_then_add_scaled(orc):
    n = 768
    rng = np.random.default_rng(29)
    residual, x, s = fill(rng, n, 2.0), fill(rng, n, 4.0), fill(rng, n, 0.5)
    norm = np.zeros(n, F32)
    orc.lib().or_zero_centered_rms(orc.p(x), orc.p(s), n, orc.p(norm))
    want = residual + F32(0.8) * norm  # Ops.AddScaled, elementwise in float32
    got = residual.copy()
    orc.lib().or_post_norm_add(orc.p(got), orc.p(x), orc.p(s), 0.8, n)
    assert bits_equal(got, want)


# --------------------------------------------------------- float64 pins --

@pytest.mark.parametrize("mode", ["rms", "centered", "gate"])
def test_fake_int8_rows_snap_to_the_grid_of_the_float64_result(orc, mode):
    """Every output is k * scale with integer k in [-128, 127], within half a
    step of the float64 value (KernelTests.FakeA8SnapsToTheInt8Grid)."""
    n = 1024
    rng = np.random.default_rng({"rms": 1, "centered": 2, "gate": 3}[mode])
    x, s = fill(rng, n, 6.0), fill(rng, n, 0.6)
    x64 = x.astype(np.float64)
    got = np.zeros(n, F32)
    if mode == "rms":
        orc.lib().or_rms_fake_a8(orc.p(x), n, orc.p(got))
        exact = x64 / math.sqrt(np.mean(x64 * x64) + 1e-6)
    elif mode == "centered":
        orc.lib().or_centered_rms_fake_a8(orc.p(x), orc.p(s), n, orc.p(got))
        exact = (1 + s.astype(np.float64)) * x64 / math.sqrt(np.mean(x64 * x64) + 1e-6)
    else:
        got, gate = x.copy(), arr(s * 8)
        orc.lib().or_gate_fake_a8(orc.p(got), orc.p(gate), n)
        exact = x64 * sig64(gate)
    scale = np.abs(exact).max() / 127
    k = got.astype(np.float64) / scale
    assert np.abs(k - np.round(k)).max() < 1e-3 and np.abs(k).max() <= 128
    assert np.abs(got - exact).max() <= 0.5 * scale * (1 + 1e-4)


def test_sigmoid_and_attention_gate_match_float64(orc):
    xs = np.linspace(-20, 20, 801)
    for x in xs:
        assert abs(orc.lib().or_sigmoid(float(x)) - sig64(F32(x))) <= 4e-7 * sig64(F32(x)) + 1e-30
        assert abs(orc.lib().or_n3_attn_gate(float(x)) - sig64(F32(x))) <= 2e-7 * sig64(F32(x)) + 1e-30


def test_post_norm_add_matches_float64(orc):
    n = 640
    rng = np.random.default_rng(5)
    residual, x, s = fill(rng, n, 2.0), fill(rng, n, 4.0), fill(rng, n, 0.5)
    got = residual.copy()
    orc.lib().or_post_norm_add(orc.p(got), orc.p(x), orc.p(s), 0.37, n)
    x64 = x.astype(np.float64)
    want = residual + 0.37 * (1 + s.astype(np.float64)) * x64 / math.sqrt(np.mean(x64 * x64) + 1e-6)
    assert np.abs(got - want).max() < 1e-5


def test_mix4_and_combine_diff4x4_match_float64(orc):
    dim = 384
    rng = np.random.default_rng(23)
    s, x, u = fill(rng, 4 * dim, 2.0), fill(rng, dim, 2.0), fill(rng, dim, 2.0)
    mix, post = fill(rng, 16, 2.0), fill(rng, 4, 2.0)
    got = np.zeros(4 * dim, F32)
    orc.lib().or_combine_diff4x4(orc.p(s), dim, orc.p(mix), orc.p(x), orc.p(u), orc.p(post), orc.p(got))
    S = s.astype(np.float64).reshape(4, dim)
    want = post.astype(np.float64)[:, None] * (x - u.astype(np.float64))[None, :] + mix.astype(np.float64).reshape(4, 4) @ S
    assert np.abs(got.reshape(4, dim) - want).max() < 1e-5
    m4 = np.zeros(dim, F32)
    orc.lib().or_mix4(orc.p(s), dim, 0.1, -0.7, 1.3, 0.25, orc.p(m4))
    assert np.abs(m4 - np.array([0.1, -0.7, 1.3, 0.25], dtype=np.float32).astype(np.float64) @ S).max() < 1e-5


def sinkhorn64(logits):
    r = np.exp(logits - logits.max(axis=1, keepdims=True))
    for _ in range(20):
        r /= r.sum(axis=1, keepdims=True)
        r /= r.sum(axis=0, keepdims=True)
    return r


@pytest.mark.parametrize("seed", range(6))
def test_sinkhorn4x4_matches_float64_and_is_doubly_stochastic(orc, seed):
    """Sinkhorn4x4 (Ops.cs:453): rows then columns normalised 20 times."""
    lg = arr((np.random.default_rng(31 + seed).random(16) - 0.5) * 6)
    got = np.zeros(16, F32)
    orc.lib().or_sinkhorn4x4(orc.p(lg), orc.p(got))
    want = sinkhorn64(lg.astype(np.float64).reshape(4, 4))
    assert np.abs(got.reshape(4, 4) - want).max() < 2e-6
    assert np.abs(got.reshape(4, 4).sum(axis=0) - 1).max() < 1e-6
    assert np.abs(got.reshape(4, 4).sum(axis=1) - 1).max() < 1e-2


def test_gather_row_is_the_dequantized_rotated_row(orc):
    """Quant.GatherRow: codebook level x fp16 norm per element, then the
    orthonormal Walsh-Hadamard transform (Sylvester order) of every 128-group."""
    rows, cols = 6, 384
    rng = np.random.default_rng(9)
    levels = arr(np.sort(rng.uniform(-1, 1, 16)))
    book = orc.Codebook()
    orc.lib().or_codebook_fill(C.byref(book), orc.p(levels), 16)
    idx = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    norms = np.array([np.float16(v).view(np.uint16) for v in rng.uniform(0.01, 0.2, rows * cols // 128)],
                     dtype=np.uint16)
    cq = orc.Cq(idx.ctypes.data, norms.ctypes.data, C.pointer(book), rows, cols, 4)
    H = hadamard(128) / math.sqrt(128)
    for r in range(rows):
        got = np.zeros(cols, F32)
        orc.lib().or_gather_row(C.byref(cq), r, orc.p(got))
        codes = np.empty(cols, dtype=np.int64)
        b = idx[r * cols // 2:(r + 1) * cols // 2]
        codes[0::2], codes[1::2] = b & 15, b >> 4
        dense = levels[codes].astype(np.float64)
        for g in range(cols // 128):
            dense[g * 128:(g + 1) * 128] *= float(np.uint16(norms[r * cols // 128 + g]).view(np.float16))
            want = H @ dense[g * 128:(g + 1) * 128]
            assert np.abs(got[g * 128:(g + 1) * 128] - want).max() < 2e-6 * (1 + np.abs(want).max())


def test_rope_tables_match_float64(orc):
    theta, qk, cap = 100000.0, 48, 300
    half = qk // 2
    cos_t, sin_t = np.zeros(cap * half, F32), np.zeros(cap * half, F32)
    orc.lib().or_n3_rope_tables(theta, qk, cap, orc.p(cos_t), orc.p(sin_t))
    freq = 1.0 / theta ** (2.0 * np.arange(half) / qk)
    angle = np.arange(cap)[:, None] * freq[None, :]
    # float32 angles carry the relative rounding of p * freq
    tol = 2e-6 + 2 * np.abs(angle) * 2.0 ** -23
    assert (np.abs(cos_t.reshape(cap, half) - np.cos(angle)) <= tol).all()
    assert (np.abs(sin_t.reshape(cap, half) - np.sin(angle)) <= tol).all()


# ------------------------------------------------------- Hadamard MLP --

def mlp_case(dim, rows, cols, seed):
    """HadamardMlpTests.Batch's draws (KernelTests.cs:335-360) with numpy."""
    rng = np.random.default_rng(seed)
    width = rows * cols

    def u(n, spread, offset=0.0):
        return arr(offset + spread * (rng.random(n) * 2 - 1))

    w = dict(d1=u(dim, 0.5, 1), d2=u(width, 0.5, 1), b2=u(width, 0.2), d3=u(width, 0.5, 1), d4=u(dim, 0.5, 1),
             w1a=u(rows * rows, 0.3), w1b=u(cols * cols, 0.3), w2a=u(rows * rows, 0.3), w2b=u(cols * cols, 0.3),
             w3a=u(rows * rows, 0.3), w3b=u(cols * cols, 0.3), cond_v=u(dim * 8, 0.1), cond_u=u(8 * width, 0.3))
    pre = u(dim, 0.3)
    pa = rng.permutation(width).astype(np.int32)
    pb = rng.permutation(width).astype(np.int32)
    return w, pre, pa, pb


def mlp64(w, pre, pa, pb, dim, rows, cols, residual, mistake=None):
    """KernelTests.cs:360-405 (Reference) in float64, Scale 1."""
    W = {k: v.astype(np.float64) for k, v in w.items()}
    width = rows * cols
    r = residual.astype(np.float64)
    inverse = 1 / math.sqrt(np.mean(r * r) + 1e-6)
    norm = (1 + pre.astype(np.float64)) * r * inverse
    logits = norm @ W["cond_v"].reshape(dim, 8)
    weights = np.exp(logits - logits.max())
    weights /= weights.sum()

    def product(z, left, right):
        L, R = left.reshape(rows, rows), right.reshape(cols, cols)
        return (L.T @ z.reshape(rows, cols) @ R).reshape(-1)

    first = np.zeros(width)
    first[:dim] = norm * W["d1"]
    p1 = product(first, W["w1a"], W["w1b"])
    cond = 1 + weights @ W["cond_u"].reshape(8, width)
    perm_a, perm_b = (pb, pa) if mistake == "swap_perms" else (pa, pb)
    v = W["d2"] * cond * p1[perm_a] + W["b2"]
    second = v / (1 + np.exp(-v)) if mistake != "no_activation" else v
    p2 = product(second, W["w2a"], W["w2b"])
    third = p2[perm_b] * W["d3"]
    p3 = product(third, W["w3a"], W["w3b"]) if mistake != "transpose_left" else \
        (W["w3a"].reshape(rows, rows) @ third.reshape(rows, cols) @ W["w3b"].reshape(cols, cols)).reshape(-1)
    return r + p3[:dim] * W["d4"]


def run_mlp(orc, w, pre, pa, pb, dim, rows, cols, residual):
    mlp = orc.N3.Mlp()
    for k, v in w.items():
        setattr(mlp, k, v.ctypes.data)
    out = arr(residual).copy()
    orc.lib().or_hadamard_mlp(C.byref(mlp), orc.p(pre), pa.ctypes.data, pb.ctypes.data, dim, rows, cols, orc.p(out))
    return out


@pytest.mark.parametrize("dim,rows,cols", [(768, 32, 32), (96, 8, 16), (48, 8, 8), (32, 8, 8), (256, 16, 32)])
def test_hadamard_mlp_matches_the_float64_reference(orc, dim, rows, cols):
    w, pre, pa, pb = mlp_case(dim, rows, cols, 11)
    for t in range(3):
        residual = arr(np.random.default_rng(5 + t).random(dim) * 2 - 1)
        got = run_mlp(orc, w, pre, pa, pb, dim, rows, cols, residual)
        want = mlp64(w, pre, pa, pb, dim, rows, cols, residual)
        assert np.isfinite(got).all()
        assert (np.abs(got - want) <= 2e-4 * (1 + np.abs(want))).all()


@pytest.mark.parametrize("mistake", ["swap_perms", "no_activation", "transpose_left"])
def test_hadamard_mlp_float64_bound_rejects_planted_mistakes(orc, mistake):
    dim, rows, cols = 96, 8, 16
    w, pre, pa, pb = mlp_case(dim, rows, cols, 11)
    residual = arr(np.random.default_rng(5).random(dim) * 2 - 1)
    got = run_mlp(orc, w, pre, pa, pb, dim, rows, cols, residual)
    wrong = mlp64(w, pre, pa, pb, dim, rows, cols, residual, mistake)
    assert not (np.abs(got - wrong) <= 2e-4 * (1 + np.abs(wrong))).all()


# ------------------------------------------------------- engram rows --

def hash_row(table, order, gram, slots):
    """The engram hash of one n-gram (most recent token first)."""
    acc = (0x9E3779B9 * (table + 1)) & 0xFFFFFFFF
    for tok in gram:
        acc = ((acc ^ (tok & 0xFFFFFFFF)) * 0x01000193) & 0xFFFFFFFF
    acc ^= acc >> 15
    return table * slots + acc % slots


def test_engram_rows_follow_the_whole_sequence_across_steps(orc):
    """Rows computed step by step (the slot carries its length and last two
    tokens) equal the hash of each position's n-gram over the full sequence;
    -1 before an order's first full n-gram."""
    g = orc.N3.Dims()
    g.engram_tables, g.engram_slots, g.order_count = 4, 97, 2
    g.orders[0], g.orders[1] = 2, 3
    heads = 2
    rng = np.random.default_rng(7)
    seq = {0: rng.integers(0, 5000, 40), 1: rng.integers(0, 5000, 40)}
    lengths = np.zeros(2, dtype=np.int32)
    prev = np.zeros(4, dtype=np.int32)
    fed = {0: 0, 1: 0}
    for size0, size1 in [(5, 1), (1, 7), (3, 3), (1, 1), (9, 2), (1, 1), (4, 6)]:
        toks = np.r_[seq[0][fed[0]:fed[0] + size0], seq[1][fed[1]:fed[1] + size1]].astype(np.int32)
        slots = np.array([0] * size0 + [1] * size1, dtype=np.int32)
        out = np.zeros(len(toks) * 4, dtype=np.int32)
        orc.lib().or_n3_engram_rows(C.byref(g), orc.p(toks), orc.p(slots), len(toks), orc.p(lengths), orc.p(prev),
                                    orc.p(out))
        out = out.reshape(-1, 4)
        row = 0
        for slot, size in ((0, size0), (1, size1)):
            for i in range(size):
                pos = fed[slot] + i
                for o, order in enumerate((2, 3)):
                    for h in range(heads):
                        table = o * heads + h
                        want = -1 if pos < order - 1 else hash_row(
                            table, order, [int(seq[slot][pos - j]) for j in range(order)], 97)
                        assert out[row, table] == want, (slot, pos, table)
                row += 1
            # the engine's carry (ForwardBatch, Engine.cs:2326-2340)
            run = seq[slot][fed[slot]:fed[slot] + size]
            prev[2 * slot], prev[2 * slot + 1] = (run[-2], run[-1]) if size > 1 else (prev[2 * slot + 1], run[-1])
            lengths[slot] += size
            fed[slot] += size


# ---------------------------------------------- engine invariants (CPU) --

@pytest.fixture(scope="module")
def small(orc):
    return OracleModel(orc, needle3_archive(SMALL, 3))


def toks(seed, n):
    return np.random.default_rng(seed).integers(0, SMALL["vocab"], n).astype(np.int32)


def engine(orc, om, slots=3):
    return OracleEngine(orc, om, slots=slots, capacity=96, max_chunks=8)


def test_oracle_engine_batched_equals_single(orc, small):
    a, b = engine(orc, small), engine(orc, small)
    p0, p1 = toks(1, 7), toks(2, 9)
    both = a.step(np.r_[p0, p1], [0] * 7 + [1] * 9, [6, 15])
    s0 = b.step(p0, [0] * 7, [6])
    s1 = b.step(p1, [1] * 9, [8])
    assert bits_equal(both, np.r_[s0, s1])
    for i in range(10):  # past the window of 6
        t = toks(10 + i, 2)
        both = a.step(t, [0, 1], [0, 1])
        assert bits_equal(both, np.r_[b.step(t[:1], [0], [0]), b.step(t[1:], [1], [0])])
    a.close()
    b.close()


def test_oracle_engine_chunk_equals_sequential_and_rewind_equals_fresh(orc, small):
    a, b, c = engine(orc, small), engine(orc, small), engine(orc, small)
    p = toks(5, 12)
    chunk = a.step(p, [0] * 12, list(range(12)))
    seq = np.concatenate([b.step(p[i:i + 1], [0], [0]) for i in range(12)])
    assert bits_equal(chunk, seq)
    a.mark(0)
    more = toks(6, 4)
    first = a.step(more, [0] * 4, [0, 1, 2, 3])
    a.step(toks(7, 3), [0] * 3, [2])
    a.rewind(0)
    assert a.length(0) == 12
    assert bits_equal(a.step(more, [0] * 4, [0, 1, 2, 3]), first)
    c.step(np.r_[p, more[:2]], [1] * 14, [13])
    assert bits_equal(c.step(more[2:], [1] * 2, [0, 1]), first[2:])
    for e in (a, b, c):
        e.close()


def test_oracle_engine_context_changes_logits(orc, small):
    """The layers matter: the same token after different histories (also
    beyond the sliding window, through the global layer and the engram)
    gives different logits."""
    a = engine(orc, small)
    base = toks(8, 10)
    other = base.copy()
    other[0] = (other[0] + 1) % SMALL["vocab"]  # 9 positions back: outside the window of 6
    la = a.step(base, [0] * 10, [9])
    lb = a.step(other, [1] * 10, [9])
    assert not bits_equal(la, lb)
    a.close()
