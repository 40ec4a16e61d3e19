"""The oracle's view of a Needle 3 archive (needle_cs_amd/archive.py writes them).

TEST INFRASTRUCTURE ONLY: imported by tests/ and by bench.py's CPU baseline
leg, never by the product.

OracleModel parses an archive the way Model.Open does (src/Needle/Model.cs:
307-371) and fills the oracle's or_n3_model with views of it (codebook records
as Cq views, dense records decoded to float with HalfToSingle, AttnGate as the
host libm sigmoid of its record); OracleEngine steps it with or_n3_forward
(EngineCore.ForwardBatch, src/Needle/Engine.cs:2303-2350).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from needle_cs_amd.archive import hada_split, parse


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

    def step(self, tokens, row_slots, head_rows, trace=False):
        """Logits [heads][vocab] of the head rows; with trace=True also the
        stream [layers + 1][rows][4][dim] after the embedding and each layer."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        s = np.ascontiguousarray(row_slots, dtype=np.int32)
        h = np.ascontiguousarray(head_rows, dtype=np.int32).reshape(-1)
        lg = np.zeros((len(h), self.vocab), dtype=np.float32)
        g = self.om.dims
        states = np.zeros((g.layers + 1, len(t), 4, g.dim), dtype=np.float32) if trace else None
        self.e.trace = states.ctypes.data if trace else None
        self.orc.lib().or_n3_forward(C.byref(self.e), self.orc.p(t), self.orc.p(s), len(t),
                                     self.orc.p(h) if len(h) else None, len(h), self.orc.p(lg) if len(h) else None)
        self.e.trace = None
        return (lg, states) if trace else lg

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
