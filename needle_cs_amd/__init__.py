"""needle_cs_amd -- MI355X (gfx950) quantized decode hot path of needle-cs.

The product is the C-ABI library ``libneedle_hip.so`` built from ``csrc/``
(declared in ``include/needle_hip.h``).  This module is a thin ctypes binding
of that ABI for Python callers (tests, benchmarks): it loads the in-tree
library and raises if it is missing -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libneedle_hip.so")

__all__ = [
    "LIB_PATH", "NeedleHipError", "lib", "check", "Codebook", "Cq", "Activations", "AttnTile", "RecordInfo",
    "DeviceBuffer", "Weights", "Stream", "Event", "Graph", "synth_normal", "synth_uniform", "synth_int8",
    "synth_half_uniform", "available",
]


class NeedleHipError(RuntimeError):
    pass


# ------------------------------------------------------ reference structs --

class Codebook(C.Structure):
    """src/Needle/Model.cs:36-42."""
    _fields_ = [("levels", C.c_float * 16), ("bytes", C.c_uint8 * 32), ("byte_scale", C.c_float)]


class Cq(C.Structure):
    """src/Needle/Model.cs:8-34."""
    _fields_ = [("indices", C.c_void_p), ("norms", C.c_void_p), ("book", C.POINTER(Codebook)),
                ("rows", C.c_int32), ("cols", C.c_int32), ("bits", C.c_int32)]


class Activations(C.Structure):
    """src/Needle/Quant.cs:11-28."""
    _fields_ = [("values", C.c_void_p), ("scales", C.c_void_p), ("offsets", C.c_void_p),
                ("cols", C.c_int32), ("groups", C.c_int32), ("stride", C.c_int32)]


class AttnTile(C.Structure):
    """src/Needle/Blocks.cs:11-27."""
    _fields_ = [("queries", C.c_void_p), ("query_scales", C.c_void_p), ("heads", C.c_int32),
                ("keys", C.c_void_p), ("key_scales", C.c_void_p), ("values", C.c_void_p),
                ("value_scales", C.c_void_p), ("key_stride", C.c_int32), ("value_stride", C.c_int32),
                ("scale_stride", C.c_int32), ("first", C.c_int32), ("count", C.c_int32),
                ("scores", C.c_void_p), ("output", C.c_void_p), ("probabilities", C.c_void_p),
                ("probability_stride", C.c_int32), ("peaks", C.c_void_p), ("sums", C.c_void_p)]


class RecordInfo(C.Structure):
    """nhip_record_info: one .cact record (src/Needle/Model.cs:190-197)."""
    _fields_ = [("dtype", C.c_int32), ("ndim", C.c_int32), ("shape", C.c_uint32 * 4), ("offset", C.c_uint64),
                ("bytes", C.c_uint64), ("group", C.c_uint32), ("bits", C.c_uint32)]


_i32, _u64p, _vp, _sz = C.c_int32, C.POINTER(C.c_uint64), C.c_void_p, C.c_size_t
_PROTOS = {
    "nhip_last_error": (C.c_char_p, []),
    "nhip_describe": (C.c_char_p, []),
    "nhip_matmul_rows": (None, [C.POINTER(Cq), C.POINTER(Activations), _i32, _vp, _i32, _i32, _i32]),
    "nhip_prepare": (None, [_vp, _i32, _i32, _i32, C.POINTER(Activations)]),
    "nhip_attention_tile": (None, [C.POINTER(AttnTile)]),
    "nhip_merge_partials": (None, [_vp, _i32, _i32, _vp]),
    "nhip_quantize_int8": (C.c_float, [_vp, _i32, _vp]),
    "nhip_fill_kernel_table": (_i32, [C.POINTER(_vp), _i32]),
    "nhip_init": (_i32, [_i32]),
    "nhip_device_count": (_i32, [C.POINTER(_i32)]),
    "nhip_malloc": (_i32, [C.POINTER(_vp), _sz]),
    "nhip_free": (_i32, [_vp]),
    "nhip_memcpy_htod": (_i32, [_vp, _vp, _sz]),
    "nhip_memcpy_dtoh": (_i32, [_vp, _vp, _sz]),
    "nhip_memcpy_dtod": (_i32, [_vp, _vp, _sz, _vp]),
    "nhip_copy_dev": (_i32, [_vp, _vp, _sz, _vp]),
    "nhip_decoder_create": (_i32, [_vp, _vp]),
    "nhip_decoder_set_layer": (_i32, [_vp, _i32] + [_vp] * 10),
    "nhip_decoder_set_head": (_i32, [_vp, _vp, _vp, _vp, _vp]),
    "nhip_decoder_forward": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp]),
    "nhip_decoder_forward_masked": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp]),
    "nhip_argmax_masked_dev": (_i32, [_vp, _i32, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "nhip_read_stream_dev": (_i32, [_vp, C.c_size_t, _vp, _vp]),
    "nhip_topk_lse_workspace": (C.c_size_t, [_i32, _i32]),
    "nhip_topk_lse_dev": (_i32, [_vp, _i32, _i32, _i32, _vp, C.c_size_t, _vp, _vp, _vp]),
    "nhip_needle3_attention_inputs_dev": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32] + [_vp] * 10 +
                                          [_i32, _i32] + [_vp] * 7),
    "nhip_decoder_copy_slot": (_i32, [_vp, _i32, _i32, _i32]),
    "nhip_argmax_dev": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "nhip_decoder_step": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "nhip_decoder_slot_reset": (_i32, [_vp, _i32]),
    "nhip_decoder_slot_mark": (_i32, [_vp, _i32]),
    "nhip_decoder_slot_rewind": (_i32, [_vp, _i32]),
    "nhip_decoder_slot_length": (_i32, [_vp, _i32, _vp]),
    "nhip_decoder_greedy": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "nhip_decoder_beam_search": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "nhip_decoder_destroy": (_i32, [_vp]),
    "nhip_open": (_i32, [_vp, _sz, C.POINTER(_vp)]),
    "nhip_model_info": (_i32, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_float), C.POINTER(_i32)]),
    "nhip_model_record": (_i32, [_vp, _i32, C.POINTER(RecordInfo)]),
    "nhip_model_weights": (_vp, [_vp, _i32]),
    "nhip_model_dense": (_vp, [_vp, _i32]),
    "nhip_model_close": (_i32, [_vp]),
    "nhip_model_raw": (_vp, [_vp, _i32]),
    "nhip_model_codebooks": (_i32, [_vp, C.POINTER(Codebook), C.POINTER(Codebook)]),
    "nhip_ctx_create": (_i32, [_vp, _i32, _i32, _i32, _i32, C.POINTER(_vp)]),
    "nhip_ctx_destroy": (_i32, [_vp]),
    "nhip_ctx_info": (_i32, [_vp, _vp, _vp, _vp, _vp]),
    "nhip_step": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "nhip_slot_feed": (_i32, [_vp, _i32, _vp, _i32, _vp]),
    "nhip_slot_reset": (_i32, [_vp, _i32]),
    "nhip_slot_mark": (_i32, [_vp, _i32]),
    "nhip_slot_rewind": (_i32, [_vp, _i32]),
    "nhip_slot_length": (_i32, [_vp, _i32, _vp]),
    "nhip_slot_copy": (_i32, [_vp, _i32, _i32]),
    "nhip_matmul_i8_fused_dev": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp]),
    "nhip_attention_decode_workspace": (_sz, [_i32, _i32, _i32]),
    "nhip_attention_decode_workspace_init": (_i32, [_vp, _sz, _vp]),
    "nhip_attention_decode_dev": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp,
                                         _vp, _i32, _vp, _sz, _vp, _vp]),
    "nhip_table_release": (_i32, [_vp, _sz, _vp]),
    "nhip_table_cached": (_i32, [_vp, _vp]),
    "nhip_matmul_batch_dev": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "nhip_attention_decode_noalloc_dev": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32,
                                                 _vp, _vp, _vp, _i32, _vp, _vp]),
    "nhip_memset": (_i32, [_vp, _i32, _sz]),
    "nhip_stream_create": (_i32, [C.POINTER(_vp)]),
    "nhip_stream_destroy": (_i32, [_vp]),
    "nhip_stream_sync": (_i32, [_vp]),
    "nhip_device_sync": (_i32, []),
    "nhip_event_create": (_i32, [C.POINTER(_vp)]),
    "nhip_event_destroy": (_i32, [_vp]),
    "nhip_event_record": (_i32, [_vp, _vp]),
    "nhip_event_elapsed_ms": (_i32, [_vp, _vp, C.POINTER(C.c_float)]),
    "nhip_graph_begin": (_i32, [_vp]),
    "nhip_graph_end": (_i32, [_vp, C.POINTER(_vp)]),
    "nhip_graph_launch": (_i32, [_vp, _vp]),
    "nhip_graph_destroy": (_i32, [_vp]),
    "nhip_weights_i8_create": (_i32, [_vp, _vp, _i32, _i32, C.POINTER(_vp)]),
    "nhip_weights_i8_create_dev": (_i32, [_vp, _vp, _i32, _i32, C.POINTER(_vp)]),
    "nhip_weights_cq_create": (_i32, [C.POINTER(Cq), C.POINTER(_vp)]),
    "nhip_weights_destroy": (_i32, [_vp]),
    "nhip_weights_info": (_i32, [_vp, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_sz)]),
    "nhip_quantize_rows_dev": (_i32, [_vp, _i32, _i32, _vp, _vp, _vp]),
    "nhip_prepare_dev": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _i32, _vp]),
    "nhip_matmul_i8_dev": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp]),
    "nhip_matmul_cq_dev": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp]),
    "nhip_group_dots_i8_dev": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "nhip_group_dots_cq_dev": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "nhip_synth_normal": (None, [_u64p, _vp, _sz]),
    "nhip_synth_uniform": (None, [_u64p, _vp, _sz, C.c_float, C.c_float]),
    "nhip_synth_int8": (None, [_u64p, _vp, _sz]),
    "nhip_synth_half_uniform": (None, [_u64p, _vp, _sz, C.c_float, C.c_float]),
}

_LIB = None


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> C.CDLL:
    """The loaded libneedle_hip.so with every prototype set; raises if the
    library has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise NeedleHipError(f"{LIB_PATH} is not built; run needle_cs_amd/build.py (or __graft_entry__.build())")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def last_error() -> str:
    return (lib().nhip_last_error() or b"").decode()


def check(rc: int) -> None:
    if rc != 0:
        raise NeedleHipError(f"needle_hip error {rc}: {last_error()}")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ------------------------------------------------------------- plumbing --

class DeviceBuffer:
    """A device allocation owned by Python (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().nhip_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().nhip_memcpy_htod(self.ptr + offset, _ptr(a), a.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        check(lib().nhip_memcpy_dtoh(_ptr(out), self.ptr + offset, out.nbytes))
        return out

    def zero(self) -> None:
        check(lib().nhip_memset(self.ptr, 0, self.nbytes))

    def close(self) -> None:
        if getattr(self, "ptr", 0):
            lib().nhip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = C.c_void_p()
        check(lib().nhip_stream_create(C.byref(p)))
        self.ptr = p.value

    def sync(self) -> None:
        check(lib().nhip_stream_sync(self.ptr))

    def close(self) -> None:
        if self.ptr:
            lib().nhip_stream_destroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(lib().nhip_event_create(C.byref(p)))
        self.ptr = p.value

    def record(self, stream: "Stream | None" = None) -> None:
        check(lib().nhip_event_record(self.ptr, stream.ptr if stream else None))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        check(lib().nhip_event_elapsed_ms(self.ptr, later.ptr, C.byref(ms)))
        return ms.value


class Graph:
    """Calls issued on `stream` inside ``with Graph.capture(stream) as g:``
    are recorded, not run; ``g.launch()`` replays them."""

    def __init__(self, stream: "Stream | None" = None):
        self.stream = stream
        self.ptr = None

    @classmethod
    def capture(cls, stream: "Stream | None" = None) -> "Graph":
        return cls(stream)

    def __enter__(self) -> "Graph":
        check(lib().nhip_graph_begin(self.stream.ptr if self.stream else None))
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        p = C.c_void_p()
        rc = lib().nhip_graph_end(self.stream.ptr if self.stream else None, C.byref(p))
        if exc_type is None:
            check(rc)
            self.ptr = p.value

    def launch(self) -> None:
        check(lib().nhip_graph_launch(self.ptr, self.stream.ptr if self.stream else None))

    def close(self) -> None:
        if self.ptr:
            lib().nhip_graph_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Weights:
    """An HBM-resident weight matrix (literal int8/g32 or .cact codebook)."""

    def __init__(self, handle: int):
        self.handle = handle
        rows, cols, bits, nbytes = C.c_int32(), C.c_int32(), C.c_int32(), C.c_size_t()
        check(lib().nhip_weights_info(handle, C.byref(rows), C.byref(cols), C.byref(bits), C.byref(nbytes)))
        self.rows, self.cols, self.bits, self.device_bytes = rows.value, cols.value, bits.value, nbytes.value

    @classmethod
    def int8(cls, w: np.ndarray, scales: np.ndarray) -> "Weights":
        w = np.ascontiguousarray(w, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        rows, cols = w.shape
        assert scales.shape == (rows, cols // 32)
        h = C.c_void_p()
        check(lib().nhip_weights_i8_create(_ptr(w), _ptr(scales), rows, cols, C.byref(h)))
        return cls(h.value)

    @classmethod
    def int8_dev(cls, d_w: DeviceBuffer, d_scales: DeviceBuffer, rows: int, cols: int) -> "Weights":
        h = C.c_void_p()
        check(lib().nhip_weights_i8_create_dev(d_w.ptr, d_scales.ptr, rows, cols, C.byref(h)))
        return cls(h.value)

    @classmethod
    def codebook(cls, indices: np.ndarray, norms: np.ndarray, book: Codebook, rows: int, cols: int,
                 bits: int) -> "Weights":
        indices = np.ascontiguousarray(indices, dtype=np.uint8)
        norms = np.ascontiguousarray(norms, dtype=np.uint16)
        cq = Cq(_ptr(indices), _ptr(norms), C.pointer(book), rows, cols, bits)
        h = C.c_void_p()
        check(lib().nhip_weights_cq_create(C.byref(cq), C.byref(h)))
        return cls(h.value)

    def close(self) -> None:
        if self.handle:
            lib().nhip_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------------- synthetic workloads --

def _state(seed_or_state) -> C.c_uint64:
    return seed_or_state if isinstance(seed_or_state, C.c_uint64) else C.c_uint64(seed_or_state or 0x9E3779B97F4A7C15)


def synth_normal(state: C.c_uint64, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().nhip_synth_normal(C.byref(state), _ptr(out), n)
    return out


def synth_uniform(state: C.c_uint64, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().nhip_synth_uniform(C.byref(state), _ptr(out), n, lo, hi)
    return out


def synth_int8(state: C.c_uint64, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int8)
    lib().nhip_synth_int8(C.byref(state), _ptr(out), n)
    return out


def synth_half_uniform(state: C.c_uint64, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().nhip_synth_half_uniform(C.byref(state), _ptr(out), n, lo, hi)
    return out
