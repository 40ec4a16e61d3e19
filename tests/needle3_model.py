"""Random-init Needle 3 archives for the engine tests.

write_archive() lays out a .cact archive of a chosen geometry in the order
Model.Open reads it (src/Needle/Model.cs:307-371): the 4-bit embedding, per
layer LayerWeights (Model.cs:133-151: NormIn, Q, K, V, QTaps, KTaps, VTaps,
QNorm, KNorm, Gate, Out, PostNorm, AttnGate, PreHada, then MlpWeights,
src/Needle/Audio.cs:11-26), HyperConnections (Model.cs:160-173, the two
permutations stored as float records), the engram sites (Model.cs:181-187),
FinalNorm and the tokenizer blob; header words as Geometry reads them
(Model.cs:75-104).  Values are seeded random draws scaled to keep every
activation finite and in range (the reference ships no generator for
Needle 3 weights).

oracle_model() parses such an archive the way Model.Open does and fills the
oracle's or_n3_model with views of it (codebook records as Cq views, dense
records decoded to float with HalfToSingle, AttnGate as the host libm
sigmoid of its record).
"""
from __future__ import annotations

import ctypes as C
import math
import struct

import numpy as np

import cact

SMALL = dict(vocab=512, dim=256, heads=4, kv_heads=2, qk=48, vd=64, layers=3, max_seq=256, hada_n=512, window=6,
             global_layers=(1,), engram_slots=64, engram_sub=128, engram_tables=2, engram_dilation=2, orders=(2, 3),
             sites=(1,), rope_theta=100000.0)


def hada_split(n: int) -> tuple[int, int]:
    """Geometry.HadaRows / HadaCols (Model.cs:106-107)."""
    rows = 1 << ((n - 1).bit_length() // 2)
    return rows, n // rows


def header_words(g: dict) -> dict:
    mask = sum(1 << l for l in g["global_layers"])
    w = {3: 0, 5: g["vocab"], 7: g["dim"], 8: g["heads"], 9: g["kv_heads"], 10: g["layers"], 11: g["qk"],
         12: g["vd"], 13: g["max_seq"], 14: g["hada_n"], 15: 4, 16: g["window"], 17: mask & 0xFFFFFFFF,
         18: mask >> 32, 19: 3, 20: g["engram_slots"], 21: g["engram_sub"], 22: g["engram_tables"], 23: 4,
         24: g["engram_dilation"], 25: 0, 26: len(g["orders"]), 31: len(g["sites"])}
    for i, o in enumerate(g["orders"]):
        w[27 + i] = o
    for i, s in enumerate(g["sites"]):
        w[32 + i] = s
    return w


def write_archive(g: dict, seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    d, H, KV, qk, vd, L = g["dim"], g["heads"], g["kv_heads"], g["qk"], g["vd"], g["layers"]
    qw, kw, vw, ow = H * qk, KV * qk, KV * vd, H * vd
    rows, cols = hada_split(g["hada_n"])
    width = rows * cols
    codebook = np.concatenate([np.array([-1.5, -0.5, 0.5, 1.5]), rng.uniform(-1, 1, 8),
                               np.sort(rng.uniform(-1, 1, 16))]).astype(np.float32)
    tensors = []

    def cq(n, k, bits, lo=0.002, hi=0.02):
        idx = rng.integers(0, 256, n * k * bits // 8, dtype=np.uint8)
        norms = np.array([np.float16(v).view(np.uint16) for v in rng.uniform(lo, hi, n * (k // 128))],
                         dtype=np.uint16)
        tensors.append((cact.CQ, (n, k), cact.cq_payload(idx, norms), bits))

    def dense(shape, values, half=False):
        a = np.asarray(values, dtype=np.float16 if half else np.float32).reshape(-1)
        tensors.append((cact.FP16 if half else cact.FP32, shape, a.tobytes(), 0))

    cq(g["vocab"], d, 4, 0.02, 0.2)
    for _ in range(L):
        dense((d,), rng.uniform(-0.2, 0.2, d), half=True)                      # NormIn
        cq(qw, d, 2)
        cq(kw, d, 2)
        cq(vw, d, 2)
        for w_ in (qw, kw, vw):                                                 # QTaps, KTaps, VTaps
            dense((3, w_), np.concatenate([rng.uniform(0.6, 1.0, w_), rng.uniform(-0.3, 0.3, 2 * w_)]))
        dense((qk,), rng.uniform(-0.2, 0.2, qk))                                # QNorm
        dense((qk,), rng.uniform(-0.2, 0.2, qk), half=True)                     # KNorm
        cq(ow, d, 2)                                                            # Gate
        cq(d, ow, 2)                                                            # Out
        dense((d,), rng.uniform(-0.2, 0.2, d))                                  # PostNorm
        dense((1,), rng.uniform(-1, 1, 1))                                      # AttnGate (logit)
        dense((d,), rng.uniform(-0.2, 0.2, d))                                  # PreHada
        dense((d,), rng.uniform(0.5, 1.5, d))                                   # D1
        dense((width,), rng.uniform(0.5, 1.5, width))                           # D2
        dense((width,), rng.uniform(-0.1, 0.1, width))                          # B2
        dense((width,), rng.uniform(0.5, 1.5, width))                           # D3
        dense((d,), rng.uniform(0.05, 0.2, d))                                  # D4
        for n in (rows, cols, rows, cols, rows, cols):                          # W1A, W1B, W2A, W2B, W3A, W3B
            dense((n, n), rng.standard_normal(n * n) / math.sqrt(n))
        dense((d, 8), rng.standard_normal(d * 8) * 0.05)                        # CondV
        dense((8, width), rng.uniform(-0.2, 0.2, 8 * width))                    # CondU
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # APre
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # APost
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # ARes
    dense((L * 4,), rng.uniform(-1, 1, L * 4))                                  # BPre
    dense((L * 4,), rng.uniform(-1, 1, L * 4))                                  # BPost
    dense((L * 16,), rng.uniform(-1, 1, L * 16))                                # BRes
    cq(L * 4, 4 * d, 4)                                                         # PhiPre
    cq(L * 4, 4 * d, 4)                                                         # PhiPost
    cq(L * 16, 4 * d, 4)                                                        # PhiRes
    dense((width,), rng.permutation(width).astype(np.float32))                  # PermA
    dense((width,), rng.permutation(width).astype(np.float32))                  # PermB
    for _ in g["sites"]:
        cq(g["engram_tables"] * g["engram_slots"], g["engram_sub"], 2, 0.05, 0.3)  # Tables
        cq(d, d, 2)                                                             # Key
        cq(d, d, 2)                                                             # Value
        dense((4, d), rng.uniform(-0.5, 0.5, 4 * d))                            # Taps
    dense((d,), rng.uniform(-0.2, 0.2, d))                                      # FinalNorm
    tensors.append((cact.RAW, (16,), bytes(range(16)), 0))                      # tokenizer blob
    return cact.write(tensors, codebook, header_words(g), rope_theta=g["rope_theta"])


def parse(archive: bytes):
    """(header words, theta, codebook floats, records) of an archive."""
    words = struct.unpack_from("<48I", archive, 0)
    theta = struct.unpack_from("<f", archive, 192)[0]
    base = struct.calcsize(cact.HEADER)
    book = np.frombuffer(archive, dtype=np.float32, count=words[2], offset=base)
    table = base + 4 * words[2]
    size = struct.calcsize(cact.RECORD)
    recs = [struct.unpack_from(cact.RECORD, archive, table + i * size) for i in range(words[1])]
    return words, theta, book, recs


class OracleModel:
    """The oracle's or_n3_model over an archive (keeps every array alive)."""

    def __init__(self, orc, archive: bytes):
        self.orc = orc
        self.buf = np.frombuffer(archive, dtype=np.uint8).copy()
        words, theta, book, recs = parse(archive)
        self.keep = [self.buf]
        lib = orc.lib()
        self.book2, self.book4 = orc.Codebook(), orc.Codebook()
        b = np.ascontiguousarray(book, dtype=np.float32)
        self.keep.append(b)
        lib.or_codebook_fill(C.byref(self.book2), orc.p(b), 4)
        lib.or_codebook_fill(C.byref(self.book4), orc.p(b[12:].copy()), 16)
        self.recs = recs
        self.next = 0
        base_ptr = self.buf.ctypes.data
        N = orc.N3
        g = N.Dims()
        w = words
        g.vocab, g.dim, g.heads, g.kv_heads, g.layers = w[5], w[7], w[8], w[9], w[10]
        g.qk, g.vd, g.hada_n = w[11], w[12], w[14]
        g.hada_rows, g.hada_cols = hada_split(w[14])
        g.window, g.engram_slots, g.engram_sub, g.engram_tables = w[16], w[20], w[21], w[22]
        g.engram_dilation, g.order_count = w[24], w[26]
        for i in range(4):
            g.orders[i] = w[27 + i]
        g.site_count = w[31]
        for i in range(16):
            g.sites[i] = w[32 + i]
        g.global_mask = w[17] | (w[18] << 32)
        g.rope_theta = theta
        self.dims = g

        def quant():
            dt, nd, _, s0, s1, _, _, off, nbytes, group, bits = recs[self.next]
            self.next += 1
            assert dt == 3 and bits in (2, 4)
            idx = base_ptr + off
            norms = idx + s0 * s1 * bits // 8
            return orc.Cq(idx, norms, C.pointer(self.book2 if bits == 2 else self.book4), s0, s1, bits)

        def dense():
            dt, nd, _, s0, s1, s2, s3, off, nbytes, group, bits = recs[self.next]
            self.next += 1
            if dt == 1:
                h = np.frombuffer(archive, dtype=np.uint16, count=nbytes // 2, offset=off)
                a = orc.half_to_single_array(h)
            else:
                assert dt == 2
                a = np.frombuffer(archive, dtype=np.float32, count=nbytes // 4, offset=off).copy()
            a = np.ascontiguousarray(a, dtype=np.float32)
            self.keep.append(a)
            return a

        def ptr(a):
            return a.ctypes.data

        m = N.Model()
        m.g = g
        m.embedding = quant()
        layers = (N.Layer * g.layers)()
        for l in range(g.layers):
            ly = layers[l]
            ly.norm_in = ptr(dense())
            ly.q, ly.k, ly.v = quant(), quant(), quant()
            ly.q_taps, ly.k_taps, ly.v_taps = ptr(dense()), ptr(dense()), ptr(dense())
            ly.q_norm, ly.k_norm = ptr(dense()), ptr(dense())
            ly.gate, ly.out = quant(), quant()
            ly.post_norm = ptr(dense())
            ly.attn_gate = lib.or_n3_attn_gate(float(dense()[0]))
            ly.pre_hada = ptr(dense())
            mlp = ly.mlp
            for name in ("d1", "d2", "b2", "d3", "d4", "w1a", "w1b", "w2a", "w2b", "w3a", "w3b", "cond_v", "cond_u"):
                setattr(mlp, name, ptr(dense()))
        self.layers = layers
        m.layer = C.cast(layers, C.POINTER(N.Layer))
        for name in ("a_pre", "a_post", "a_res", "b_pre", "b_post", "b_res"):
            setattr(m, name, ptr(dense()))
        m.phi_pre, m.phi_post, m.phi_res = quant(), quant(), quant()
        self.perm_a = dense().astype(np.int32)
        self.perm_b = dense().astype(np.int32)
        self.keep += [self.perm_a, self.perm_b]
        m.perm_a, m.perm_b = ptr(self.perm_a), ptr(self.perm_b)
        sites = (N.Site * max(1, g.site_count))()
        for s in range(g.site_count):
            sites[s].tables, sites[s].key, sites[s].value = quant(), quant(), quant()
            sites[s].taps = ptr(dense())
        self.sites = sites
        m.site = C.cast(sites, C.POINTER(N.Site))
        m.final_norm = ptr(dense())
        assert recs[self.next][0] == 4 and self.next == len(recs) - 1
        self.model = m


class OracleEngine:
    def __init__(self, orc, om: OracleModel, slots: int, capacity: int, max_chunks: int = 64):
        self.orc, self.om = orc, om
        self.e = orc.N3.Engine()
        self.e.m = C.pointer(om.model)
        self.e.slots, self.e.capacity, self.e.max_chunks = slots, capacity, max_chunks
        assert orc.lib().or_n3_init(C.byref(self.e)) == 0
        self.vocab = om.dims.vocab

    def step(self, tokens, row_slots, head_rows):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        s = np.ascontiguousarray(row_slots, dtype=np.int32)
        h = np.ascontiguousarray(head_rows, dtype=np.int32).reshape(-1)
        lg = np.zeros((len(h), self.vocab), dtype=np.float32)
        self.orc.lib().or_n3_forward(C.byref(self.e), self.orc.p(t), self.orc.p(s), len(t),
                                     self.orc.p(h) if len(h) else None, len(h), self.orc.p(lg) if len(h) else None)
        return lg

    def reset(self, slot):
        self.orc.lib().or_n3_reset(C.byref(self.e), slot)

    def mark(self, slot):
        self.orc.lib().or_n3_mark(C.byref(self.e), slot)

    def rewind(self, slot):
        self.orc.lib().or_n3_rewind(C.byref(self.e), slot)

    def length(self, slot):
        return self.e.length[slot]

    def close(self):
        if self.e.keys:
            self.orc.lib().or_n3_free(C.byref(self.e))
