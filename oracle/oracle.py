"""ctypes binding of the oracle (libneedle_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (needle_cs_amd/).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libneedle_oracle.so")


class Codebook(C.Structure):
    _fields_ = [("levels", C.c_float * 16), ("bytes", C.c_uint8 * 32), ("byte_scale", C.c_float)]


class Cq(C.Structure):
    _fields_ = [("indices", C.c_void_p), ("norms", C.c_void_p), ("book", C.POINTER(Codebook)),
                ("rows", C.c_int), ("cols", C.c_int), ("bits", C.c_int)]


class Activations(C.Structure):
    _fields_ = [("values", C.c_void_p), ("scales", C.c_void_p), ("offsets", C.c_void_p),
                ("cols", C.c_int), ("groups", C.c_int), ("stride", C.c_int)]


class AttnTile(C.Structure):
    _fields_ = [("queries", C.c_void_p), ("query_scales", C.c_void_p), ("heads", C.c_int),
                ("keys", C.c_void_p), ("key_scales", C.c_void_p), ("values", C.c_void_p),
                ("value_scales", C.c_void_p), ("key_stride", C.c_int), ("value_stride", C.c_int),
                ("scale_stride", C.c_int), ("first", C.c_int), ("count", C.c_int),
                ("scores", C.c_void_p), ("output", C.c_void_p), ("probabilities", C.c_void_p),
                ("probability_stride", C.c_int), ("peaks", C.c_void_p), ("sums", C.c_void_p)]


class DecoderDims(C.Structure):
    _fields_ = [("layers", C.c_int), ("d", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("capacity", C.c_int),
                ("slots", C.c_int), ("max_chunks", C.c_int), ("theta", C.c_double), ("eps", C.c_float)]


class LayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wqkv", "sqkv", "wo", "so", "wgu", "sgu", "wd", "sd", "attn_norm",
                                          "ffn_norm")]


class Decoder(C.Structure):
    _fields_ = [("dims", DecoderDims), ("layers", C.POINTER(LayerWeights)), ("embedding", C.c_void_p),
                ("final_norm", C.c_void_p), ("wlm", C.c_void_p), ("slm", C.c_void_p), ("threads", C.c_int),
                ("simd", C.c_int),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("keys", C.c_void_p), ("values", C.c_void_p),
                ("key_scales", C.c_void_p), ("value_scales", C.c_void_p)]


class _N3:
    """ctypes mirrors of needle_oracle.h's Needle 3 structs."""

    class Dims(C.Structure):
        _fields_ = [(n, C.c_int) for n in ("vocab", "dim", "heads", "kv_heads", "layers", "qk", "vd", "hada_n",
                                            "hada_rows", "hada_cols", "window", "engram_slots", "engram_sub",
                                            "engram_tables", "engram_dilation", "order_count")] + \
                   [("orders", C.c_int * 4), ("site_count", C.c_int), ("sites", C.c_int * 16),
                    ("global_mask", C.c_uint64), ("rope_theta", C.c_float)]

    class Mlp(C.Structure):
        _fields_ = [(n, C.c_void_p) for n in ("d1", "d2", "b2", "d3", "d4", "w1a", "w1b", "w2a", "w2b", "w3a", "w3b",
                                               "cond_v", "cond_u")]

    class Layer(C.Structure):
        pass

    class Site(C.Structure):
        pass

    class Model(C.Structure):
        pass

    class Engine(C.Structure):
        pass


_N3.Layer._fields_ = [("norm_in", C.c_void_p), ("q", Cq), ("k", Cq), ("v", Cq), ("q_taps", C.c_void_p),
                      ("k_taps", C.c_void_p), ("v_taps", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p),
                      ("gate", Cq), ("out", Cq), ("post_norm", C.c_void_p), ("attn_gate", C.c_float),
                      ("pre_hada", C.c_void_p), ("mlp", _N3.Mlp)]
_N3.Site._fields_ = [("tables", Cq), ("key", Cq), ("value", Cq), ("taps", C.c_void_p)]
_N3.Model._fields_ = [("g", _N3.Dims), ("embedding", Cq), ("layer", C.POINTER(_N3.Layer))] + \
                     [(n, C.c_void_p) for n in ("a_pre", "a_post", "a_res", "b_pre", "b_post", "b_res")] + \
                     [("phi_pre", Cq), ("phi_post", Cq), ("phi_res", Cq), ("perm_a", C.c_void_p),
                      ("perm_b", C.c_void_p), ("site", C.POINTER(_N3.Site)), ("final_norm", C.c_void_p)]
_N3.Engine._fields_ = [("m", C.POINTER(_N3.Model)), ("slots", C.c_int), ("capacity", C.c_int),
                       ("max_chunks", C.c_int)] + \
                      [(n, C.c_void_p) for n in ("rope_cos", "rope_sin", "keys", "values", "key_scales",
                                                  "value_scales", "qkv_hist", "engram_hist", "snap_qkv",
                                                  "snap_engram")] + \
                      [("length", C.POINTER(C.c_int)), ("marked", C.POINTER(C.c_int)), ("prev", C.POINTER(C.c_int)),
                       ("snap_prev", C.POINTER(C.c_int)), ("trace", C.c_void_p)]
N3 = _N3

_u64p, _vp, _i, _f, _sz = C.POINTER(C.c_uint64), C.c_void_p, C.c_int, C.c_float, C.c_size_t
_PROTOS = {
    "or_xs_seed": (C.c_uint64, [C.c_uint64]),
    "or_xs_next": (C.c_uint64, [_u64p]),
    "or_xs_next_int": (_i, [_u64p, _i, _i]),
    "or_xs_next_float": (_f, [_u64p, _f]),
    "or_fill_uniform": (None, [_vp, _i, _u64p, _f]),
    "or_fill_edges": (None, [_vp, _i, _u64p, _f]),
    "or_fill_sbyte": (None, [_vp, _i, _u64p, _i]),
    "or_fill_bytes": (None, [_vp, _i, _u64p, _i]),
    "or_half_bits": (C.c_uint16, [_f]),
    "or_synth_u53": (C.c_double, [_u64p]),
    "or_synth_normal": (None, [_vp, _sz, _u64p]),
    "or_synth_uniform": (None, [_vp, _sz, _u64p, _f, _f]),
    "or_synth_int8": (None, [_vp, _sz, _u64p]),
    "or_synth_half_uniform": (None, [_vp, _sz, _u64p, _f, _f]),
    "or_single_to_half_rne": (C.c_uint16, [_f]),
    "or_half_to_single": (_f, [C.c_uint16]),
    "or_half_to_single_upstream": (_f, [C.c_uint16]),
    "or_codebook_fill": (None, [C.POINTER(Codebook), _vp, _i]),
    "or_hadamard": (None, [_vp, _vp]),
    "or_abs_max": (_f, [_vp, _i]),
    "or_round_trip": (None, [_vp, _i, _f, _f]),
    "or_quantize_int8": (_f, [_vp, _i, _vp]),
    "or_planes": (None, [_vp, _i, _vp, C.POINTER(_i)]),
    "or_prepare": (None, [_vp, _i, _i, _i, C.POINTER(Activations)]),
    "or_decode_row": (None, [C.POINTER(Cq), _i, _vp]),
    "or_matmul_rows": (None, [C.POINTER(Cq), C.POINTER(Activations), _i, _vp, _i, _i, _i]),
    "or_group_dots_cq": (None, [C.POINTER(Cq), C.POINTER(Activations), _i, _i, _i, _vp]),
    "or_matmul_rows_i8": (None, [_vp, _vp, _i, _i, _i, _vp, _vp, _i, _vp, _i, _i, _i]),
    "or_group_dots_i8": (None, [_vp, _i, _i, _i, _vp, _i, _i, _i, _vp]),
    "or_quantize_rows": (None, [_vp, _i, _i, _vp, _vp]),
    "or_exp_poly": (_f, [_f]),
    "or_softmax": (None, [_vp, _i, _i]),
    "or_attention_head": (None, [_vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i, _i]),
    "or_attention_tile_run": (None, [C.POINTER(AttnTile), _i]),
    "or_attention_partial": (None, [_vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp,
                                    C.POINTER(_f), C.POINTER(_f)]),
    "or_merge_partials": (None, [_vp, _i, _i, _vp, _i]),
    "or_merge_partials_double": (None, [_vp, _i, _i, _vp]),
    "or_attention_span": (None, [_i, _i, _i, C.POINTER(_i), C.POINTER(_i)]),
    "or_attention_plan": (_i, [_i, _i, C.POINTER(_i)]),
    "or_merge_head": (None, [_vp, _i, _vp, _vp, _i, _i, _vp, _i]),
    "or_attention_decode": (None, [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp]),
    "or_log_poly": (_f, [_f]),
    "or_add_rmsnorm_quant": (_f, [_vp, _vp, _vp, _i, _f, _vp, _vp]),
    "or_rope_table": (None, [_i, _i, C.c_double, _vp, _vp]),
    "or_rope_head": (None, [_vp, _vp, _vp]),
    "or_swiglu_quant": (_f, [_vp, _vp, _i, _vp, _vp]),
    "or_topk_lse": (None, [_vp, _i, _i, _i, _vp, _vp]),
    "or_decoder_init": (_i, [C.POINTER(Decoder)]),
    "or_decoder_free": (None, [C.POINTER(Decoder)]),
    "or_decoder_forward": (None, [C.POINTER(Decoder), _vp, _vp, _vp, _i, _vp, _i, _vp, _vp]),
    "or_decoder_copy_slot": (None, [C.POINTER(Decoder), _i, _i, _i]),
    "or_beam_search": (_i, [C.POINTER(Decoder), _vp, _i, _i, _i, _i, _vp, C.POINTER(_f), C.POINTER(C.c_long), _vp]),
    "or_argmax": (_i, [_vp, _i]),
    "or_topk_select": (None, [_vp, _i, _i, _i, _vp, _vp]),
    "or_greedy": (_i, [C.POINTER(Decoder), _vp, _i, _i, _i, _vp, _vp]),
    "or_zero_centered_rms": (None, [_vp, _vp, _i, _vp]),
    "or_rope_rotate": (None, [_vp, _i, _vp, _vp]),
    "or_needle3_attention_inputs": (None, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                           _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "or_argmax_masked": (_i, [_vp, _vp, _i, _i]),
    "or_topk_log_softmax": (None, [_vp, _i, _i, _vp, _vp, _vp, _i]),
    "or_baseline_start": (_i, [_i]),
    "or_baseline_stop": (None, []),
    "or_baseline_matmul_i8": (None, [_vp, _vp, _i, _i, _i, _vp, _vp, _i, _vp, _i, _i, _i]),
    "or_simd_tier": (_i, []),
    "or_sigmoid": (_f, [_f]),
    "or_n3_attn_gate": (_f, [_f]),
    "or_rms_fake_a8": (None, [_vp, _i, _vp]),
    "or_centered_rms_fake_a8": (None, [_vp, _vp, _i, _vp]),
    "or_gate_fake_a8": (None, [_vp, _vp, _i]),
    "or_fake_a8": (_f, [_vp, _i]),
    "or_post_norm_add": (None, [_vp, _vp, _vp, _f, _i]),
    "or_mix4": (None, [_vp, _i, _f, _f, _f, _f, _vp]),
    "or_combine_diff4x4": (None, [_vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "or_sinkhorn4x4": (None, [_vp, _vp]),
    "or_rms_unit": (None, [_vp, _i, _vp]),
    "or_dot": (_f, [_vp, _vp, _i]),
    "or_gather_row": (None, [C.POINTER(Cq), _i, _vp]),
    "or_hadamard_mlp": (None, [C.POINTER(_N3.Mlp), _vp, _vp, _vp, _i, _i, _i, _vp]),
    "or_n3_engram_rows": (None, [C.POINTER(_N3.Dims), _vp, _vp, _i, _vp, _vp, _vp]),
    "or_n3_rope_tables": (None, [_f, _i, _i, _vp, _vp]),
    "or_n3_init": (_i, [C.POINTER(_N3.Engine)]),
    "or_n3_free": (None, [C.POINTER(_N3.Engine)]),
    "or_n3_reset": (None, [C.POINTER(_N3.Engine), _i]),
    "or_n3_mark": (None, [C.POINTER(_N3.Engine), _i]),
    "or_n3_rewind": (None, [C.POINTER(_N3.Engine), _i]),
    "or_n3_forward": (None, [C.POINTER(_N3.Engine), _vp, _vp, _i, _vp, _i, _vp]),
    "or_n3_set_plant": (None, [_i]),
    "or_n3_set_threads": (None, [_i]),
    "or_n3_set_tier": (None, [_i]),
    "or_n3_tier": (_i, []),
    "or_v256_sum": (C.c_float, [_vp, _vp, _i]),
    "or_tier_sum_of_squares": (C.c_float, [_vp, _i]),
    "or_simd_matmul_i8": (None, [_i, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _i, _i, _i]),
    "or_baseline_simd_matmul_i8": (None, [_i, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _i, _i, _i]),
}

_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _build  # noqa: F401  (package-relative when imported as oracle.oracle)
            _build.build()
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def state(seed: int) -> C.c_uint64:
    return C.c_uint64(lib().or_xs_seed(seed))


# ------------------------------------------------------------- helpers --

def codebook(levels: np.ndarray, count: int) -> Codebook:
    book = Codebook()
    lv = np.zeros(16, dtype=np.float32)
    lv[:count] = levels[:count]
    lib().or_codebook_fill(C.byref(book), p(lv), count)
    return book


def activations(tokens: int, cols: int):
    """Host buffers laid out as Quant.cs:33-41 (Activations(ref Arena, ...))."""
    groups = cols // 128
    stride = (groups + 7) & ~7
    values = np.zeros(tokens * cols, dtype=np.int8)
    scales = np.zeros(tokens * stride, dtype=np.float32)
    offsets = np.zeros(tokens * stride, dtype=np.float32)
    act = Activations(p(values), p(scales), p(offsets), cols, groups, stride)
    return act, values, scales, offsets


def prepare(x: np.ndarray, tokens: int, cols: int, bits: int):
    act, values, scales, offsets = activations(tokens, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().or_prepare(p(x), tokens, cols, bits, C.byref(act))
    return act, values, scales, offsets


def matmul_rows(cq: Cq, act: Activations, tokens: int, y: np.ndarray, ldy: int, r0: int, r1: int) -> None:
    lib().or_matmul_rows(C.byref(cq), C.byref(act), tokens, p(y), ldy, r0, r1)


def matmul_rows_i8(w, scales, q, qscale, tokens, y, ldy, r0, r1, group=32):
    rows, cols = w.shape
    lib().or_matmul_rows_i8(p(w), p(scales), rows, cols, group, p(q), p(qscale), tokens, p(y), ldy, r0, r1)


def group_dots_i8(w, q, tokens, r0, r1, group=32):
    rows, cols = w.shape
    out = np.zeros((tokens, r1 - r0, cols // group), dtype=np.int32)
    lib().or_group_dots_i8(p(w), rows, cols, group, p(q), tokens, r0, r1, p(out))
    return out


def group_dots_cq(cq: Cq, act: Activations, tokens: int, r0: int, r1: int):
    out = np.zeros((tokens, r1 - r0, cq.cols // 128), dtype=np.int32)
    lib().or_group_dots_cq(C.byref(cq), C.byref(act), tokens, r0, r1, p(out))
    return out


def quantize_rows(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    tokens, cols = x.shape
    q = np.zeros((tokens, cols), dtype=np.int8)
    s = np.zeros(tokens, dtype=np.float32)
    lib().or_quantize_rows(p(x), tokens, cols, p(q), p(s))
    return q, s


def synth_normal(st: C.c_uint64, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().or_synth_normal(p(out), n, C.byref(st))
    return out


def synth_int8(st: C.c_uint64, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int8)
    lib().or_synth_int8(p(out), n, C.byref(st))
    return out


def synth_half_uniform(st: C.c_uint64, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().or_synth_half_uniform(p(out), n, C.byref(st), lo, hi)
    return out


def half_to_single_array(h: np.ndarray) -> np.ndarray:
    f = lib().or_half_to_single
    return np.array([f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def attention_plan(count: int, max_chunks: int):
    length = C.c_int(0)
    chunks = lib().or_attention_plan(count, max_chunks, C.byref(length))
    return chunks, length.value


def attention_decode(q, q_scales, heads, kv_heads, qk, keys, key_scales, values, value_scales, capacity,
                     row_slot, row_first, row_count, max_chunks):
    rows = len(row_count)
    out = np.zeros((rows, heads, 64), dtype=np.float32)
    arrs = [np.ascontiguousarray(a) for a in (q, q_scales, keys, key_scales, values, value_scales)]
    ints = [np.ascontiguousarray(a, dtype=np.int32) for a in (row_slot, row_first, row_count)]
    lib().or_attention_decode(p(arrs[0]), p(arrs[1]), rows, heads, kv_heads, qk, p(arrs[2]), p(arrs[3]),
                              p(arrs[4]), p(arrs[5]), capacity, p(ints[0]), p(ints[1]), p(ints[2]), max_chunks,
                              p(out))
    return out


def kv_cache(st, slots: int, capacity: int, kv_heads: int, qk: int):
    """Pooled int8 KV cache filled from N(0,1) values quantized per (position,
    kv head) with QuantizeInt8, as Engine.cs:1376-1384 writes it."""
    kf = np.zeros(slots * capacity * kv_heads * qk, dtype=np.float32)
    vf = np.zeros(slots * capacity * kv_heads * 64, dtype=np.float32)
    lib().or_synth_normal(p(kf), kf.size, C.byref(st))
    lib().or_synth_normal(p(vf), vf.size, C.byref(st))
    kq, ks = quantize_rows(kf.reshape(-1, qk))
    vq, vs = quantize_rows(vf.reshape(-1, 64))
    return (kq.reshape(slots, capacity, kv_heads * qk), ks.reshape(slots, capacity, kv_heads),
            vq.reshape(slots, capacity, kv_heads * 64), vs.reshape(slots, capacity, kv_heads))


class CpuDecoder:
    """The oracle's decoder over a synthetic model's numpy arrays (see
    needle_cs_amd.decoder.synthetic_model for the layout)."""

    def __init__(self, model: dict, slots: int, capacity: int, max_chunks: int = 64, threads: int = 1, simd: int = 0):
        dm = model["dims"]
        self._keep = model
        self.layers = (LayerWeights * dm["layers"])()
        for l, lw in enumerate(model["layers"]):
            for name in ("wqkv", "sqkv", "wo", "so", "wgu", "sgu", "wd", "sd", "attn_norm", "ffn_norm"):
                setattr(self.layers[l], name, p(lw[name]))
        self.dec = Decoder()
        self.dec.dims = DecoderDims(dm["layers"], dm["d"], dm["heads"], dm["kv_heads"], dm["head_dim"], dm["ffn"],
                                    dm["vocab"], capacity, slots, max_chunks, dm["theta"], dm["eps"])
        self.dec.layers = C.cast(self.layers, C.POINTER(LayerWeights))
        self.dec.embedding = p(model["embedding"])
        self.dec.final_norm = p(model["final_norm"])
        self.dec.wlm = p(model["wlm"])
        self.dec.slm = p(model["slm"])
        self.dec.threads = threads
        self.dec.simd = simd
        assert lib().or_decoder_init(C.byref(self.dec)) == 0
        self.vocab = dm["vocab"]

    def forward(self, tokens, slots, positions, k=0, logits=True):
        rows = len(tokens)
        t, s, ps = (np.ascontiguousarray(a, dtype=np.int32) for a in (tokens, slots, positions))
        lg = np.zeros((rows, self.vocab), dtype=np.float32) if logits else None
        idx = np.zeros((rows, max(k, 1)), dtype=np.int32)
        lp = np.zeros((rows, max(k, 1)), dtype=np.float32)
        lib().or_decoder_forward(C.byref(self.dec), p(t), p(s), p(ps), rows, p(lg) if logits else None, k, p(idx),
                                 p(lp))
        return lg, idx[:, :k], lp[:, :k]

    def copy_slot(self, dst, src, length):
        lib().or_decoder_copy_slot(C.byref(self.dec), dst, src, length)

    def beam_search(self, prompt, width, max_new, eos):
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max_new + 1, dtype=np.int32)
        score = C.c_float()
        fed = C.c_long()
        self.seconds = np.zeros(2, dtype=np.float64)
        n = lib().or_beam_search(C.byref(self.dec), p(pr), len(pr), width, max_new, eos, p(out), C.byref(score),
                                 C.byref(fed), p(self.seconds))
        return out[:n].copy(), score.value, fed.value

    def greedy(self, prompt, max_new, stop=-1):
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_new, 1), dtype=np.int32)
        self.seconds = np.zeros(2, dtype=np.float64)
        n = lib().or_greedy(C.byref(self.dec), p(pr), len(pr), max_new, stop, p(out), p(self.seconds))
        return out[:n].copy()

    def close(self):
        if self.dec.keys:
            lib().or_decoder_free(C.byref(self.dec))
