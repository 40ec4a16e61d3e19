"""Synthetic int8 decoder: model generation and the GPU engine binding.

The benchmark's decode-loop model (12 layers, d_model 1024, 16 heads x 64,
SwiGLU 4096, vocab 32000, RMSNorm, rotary positions; every linear int8 with
fp16 group-32 scales U(0.002, 0.02); embeddings N(0,1); norm gains 1) is
generated from one seed with the conformance XorShift64 stream
(tests/Needle.Tests/Conformance/Conformance.cs:10-38), in this order: the
embedding, then per layer Wqkv, Wo, Wgu (gate rows then up rows), Wd (each
int8 weights then fp16 scales), then the LM head.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import check, lib, synth_half_uniform, synth_int8, synth_normal, synth_uniform

CONFIG4 = dict(layers=12, d=1024, heads=16, kv_heads=16, head_dim=64, ffn=4096, vocab=32000, theta=10000.0,
               eps=1e-5)


def synthetic_model(dims: dict, seed: int) -> dict:
    st = C.c_uint64(seed)
    d, H, KV, hd, F, V = dims["d"], dims["heads"], dims["kv_heads"], dims["head_dim"], dims["ffn"], dims["vocab"]
    model = {"dims": dict(dims)}
    model["embedding"] = synth_normal(st, V * d).reshape(V, d)

    def linear(rows, cols):
        w = synth_int8(st, rows * cols).reshape(rows, cols)
        s = synth_half_uniform(st, rows * cols // 32, 0.002, 0.02).reshape(rows, cols // 32)
        return w, s

    layers = []
    for _ in range(dims["layers"]):
        lw = {}
        lw["wqkv"], lw["sqkv"] = linear((H + 2 * KV) * hd, d)
        lw["wo"], lw["so"] = linear(d, H * hd)
        lw["wgu"], lw["sgu"] = linear(2 * F, d)
        lw["wd"], lw["sd"] = linear(d, F)
        lw["attn_norm"] = np.ones(d, dtype=np.float32)
        lw["ffn_norm"] = np.ones(d, dtype=np.float32)
        layers.append(lw)
    model["layers"] = layers
    model["final_norm"] = np.ones(d, dtype=np.float32)
    model["wlm"], model["slm"] = linear(V, d)
    return model


def random_prompt(seed: int, length: int, vocab: int) -> np.ndarray:
    """Prompt ids U[4, vocab) from the conformance stream (ids 0-3 are the
    special ids TopKLogSoftmax masks)."""
    st = C.c_uint64(seed)
    v = synth_uniform(st, length, 0.0, 1.0).astype(np.float64)
    return (4 + np.minimum((v * (vocab - 4)).astype(np.int64), vocab - 5)).astype(np.int32)


class DecoderDims(C.Structure):
    _fields_ = [("layers", C.c_int32), ("d", C.c_int32), ("heads", C.c_int32), ("kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("ffn", C.c_int32), ("vocab", C.c_int32), ("capacity", C.c_int32),
                ("slots", C.c_int32), ("max_rows", C.c_int32), ("max_chunks", C.c_int32), ("theta", C.c_double),
                ("eps", C.c_float)]


class DecodeStats(C.Structure):
    _fields_ = [("prefill_seconds", C.c_double), ("decode_seconds", C.c_double), ("fed_rows", C.c_int64),
                ("steps", C.c_int32)]


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class GpuDecoder:
    """libneedle_hip's decoder engine holding a synthetic model in HBM."""

    def __init__(self, model: dict, slots: int, capacity: int, max_rows: int, max_chunks: int = 64):
        dm = model["dims"]
        self.dims = DecoderDims(dm["layers"], dm["d"], dm["heads"], dm["kv_heads"], dm["head_dim"], dm["ffn"],
                                dm["vocab"], capacity, slots, max_rows, max_chunks, dm["theta"], dm["eps"])
        h = C.c_void_p()
        check(lib().nhip_decoder_create(C.byref(self.dims), C.byref(h)))
        self.h = h.value
        self.set_model(model)
        self.vocab = dm["vocab"]

    def set_model(self, model: dict) -> None:
        """Uploads (or replaces) every layer's weights and the head."""
        for l, lw in enumerate(model["layers"]):
            check(lib().nhip_decoder_set_layer(self.h, l, *[_p(lw[n]) for n in ("wqkv", "sqkv", "wo", "so", "wgu",
                                                                                "sgu", "wd", "sd", "attn_norm",
                                                                                "ffn_norm")]))
        check(lib().nhip_decoder_set_head(self.h, _p(model["embedding"]), _p(model["final_norm"]), _p(model["wlm"]),
                                          _p(model["slm"])))

    def forward(self, tokens, slots, positions, k=0, logits=True):
        rows = len(tokens)
        t, s, ps = (np.ascontiguousarray(a, dtype=np.int32) for a in (tokens, slots, positions))
        lg = np.zeros((rows, self.vocab), dtype=np.float32) if logits else None
        idx = np.zeros((rows, max(k, 1)), dtype=np.int32)
        lp = np.zeros((rows, max(k, 1)), dtype=np.float32)
        check(lib().nhip_decoder_forward(self.h, _p(t), _p(s), _p(ps), rows, _p(lg) if logits else None, k, _p(idx),
                                         _p(lp)))
        return lg, idx[:, :k], lp[:, :k]

    def forward_masked(self, tokens, slots, positions, masks):
        """One forward with the sparse, masked head: masks [rows][words]
        uint32 id bitsets; returns the chosen ids (-1: none) and their
        logits."""
        rows = len(tokens)
        t, s, ps = (np.ascontiguousarray(a, dtype=np.int32) for a in (tokens, slots, positions))
        m = np.ascontiguousarray(masks, dtype=np.uint32).reshape(rows, -1)
        best = np.zeros(rows, dtype=np.int32)
        val = np.zeros(rows, dtype=np.float32)
        check(lib().nhip_decoder_forward_masked(self.h, _p(t), _p(s), _p(ps), rows, _p(m), m.shape[1], _p(best),
                                                _p(val)))
        return best, val

    def copy_slot(self, dst, src, length):
        check(lib().nhip_decoder_copy_slot(self.h, dst, src, length))

    def step(self, tokens, row_slots, head_rows, k=0, logits=True, argmax=False):
        """BatchedEngine.ForwardBatch: positions from the slots' lengths;
        returns the head rows' logits [heads][vocab] (or None), top-k ids and
        log-probabilities [heads][k], and Ops.ArgMax ids [heads] (or None)."""
        rows, heads = len(tokens), len(head_rows)
        t, s = (np.ascontiguousarray(a, dtype=np.int32) for a in (tokens, row_slots))
        hr = np.ascontiguousarray(head_rows, dtype=np.int32).reshape(-1)
        lg = np.zeros((heads, self.vocab), dtype=np.float32) if logits else None
        idx = np.zeros((max(heads, 1), max(k, 1)), dtype=np.int32)
        lp = np.zeros((max(heads, 1), max(k, 1)), dtype=np.float32)
        am = np.zeros(max(heads, 1), dtype=np.int32)
        check(lib().nhip_decoder_step(self.h, _p(t), _p(s), rows, _p(hr) if heads else None, heads,
                                      _p(lg) if logits and heads else None, k, _p(idx), _p(lp),
                                      _p(am) if argmax else None))
        return lg, idx[:heads, :k], lp[:heads, :k], (am[:heads] if argmax else None)

    def slot_reset(self, slot):
        check(lib().nhip_decoder_slot_reset(self.h, slot))

    def slot_mark(self, slot):
        check(lib().nhip_decoder_slot_mark(self.h, slot))

    def slot_rewind(self, slot):
        check(lib().nhip_decoder_slot_rewind(self.h, slot))

    def slot_length(self, slot) -> int:
        n = C.c_int32()
        check(lib().nhip_decoder_slot_length(self.h, slot, C.byref(n)))
        return n.value

    def greedy(self, prompt, max_new, stop=-1):
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_new, 1), dtype=np.int32)
        n = C.c_int32()
        stats = DecodeStats()
        check(lib().nhip_decoder_greedy(self.h, _p(pr), len(pr), max_new, stop, _p(out), C.byref(n),
                                        C.byref(stats)))
        return out[:n.value].copy(), stats

    def beam_search(self, prompt, width, max_new, eos):
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max_new + 1, dtype=np.int32)
        n = C.c_int32()
        score = C.c_float()
        stats = DecodeStats()
        check(lib().nhip_decoder_beam_search(self.h, _p(pr), len(pr), width, max_new, eos, _p(out), C.byref(n),
                                             C.byref(score), C.byref(stats)))
        return out[:n.value].copy(), score.value, stats

    def close(self):
        if self.h:
            lib().nhip_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
