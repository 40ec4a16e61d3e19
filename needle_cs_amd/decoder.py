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

from . import synth_half_uniform, synth_int8, synth_normal, synth_uniform

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
