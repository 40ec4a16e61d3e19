"""BatchedEngine over an opened .cact archive (src/Needle/BatchEngine.cs:5-50).

``Model`` is Model.FromMemory (src/Needle/Model.cs:400-411): the archive is
parsed and every tensor uploaded to HBM once (``nhip_open``).  ``BatchedEngine``
holds one ``nhip_ctx``: up to 16 slots of independent sequences stepped
together by ``forward_batch`` (EngineCore.ForwardBatch,
src/Needle/Engine.cs:2303-2350) or fed one slot at a time by ``feed_slot``
(Engine.cs:2285-2301), with the reference's slot operations.  Everything runs
in libneedle_hip.so on the GPU; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import Codebook, check, lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Model:
    """An archive opened on the GPU (Model.FromMemory)."""

    def __init__(self, archive: bytes):
        buf = (C.c_uint8 * len(archive)).from_buffer_copy(archive)
        h = C.c_void_p()
        check(lib().nhip_open(C.cast(buf, C.c_void_p), len(archive), C.byref(h)))
        self.h = h.value

    def header(self) -> tuple[list[int], float]:
        words = (C.c_uint32 * 48)()
        theta = C.c_float()
        check(lib().nhip_model_info(self.h, words, C.byref(theta), None))
        return list(words), theta.value

    def codebooks(self) -> tuple[Codebook, Codebook]:
        b2, b4 = Codebook(), Codebook()
        check(lib().nhip_model_codebooks(self.h, C.byref(b2), C.byref(b4)))
        return b2, b4

    def close(self) -> None:
        if self.h:
            check(lib().nhip_model_close(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class BatchedEngine:
    """BatchedEngine(model, contextLength, chunkSize, slots) on the GPU."""

    def __init__(self, model: Model, context_length: int = 1024, chunk_size: int = 64, slots: int = 8,
                 max_chunks: int = 0):
        self.model = model
        h = C.c_void_p()
        check(lib().nhip_ctx_create(model.h, context_length, slots, chunk_size, max_chunks, C.byref(h)))
        self.h = h.value
        vocab, n, cap, chunk = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().nhip_ctx_info(self.h, C.byref(vocab), C.byref(n), C.byref(cap), C.byref(chunk)))
        self.vocab_size, self.slots, self.capacity, self.chunk = vocab.value, n.value, cap.value, chunk.value

    def slot_length(self, slot: int) -> int:
        n = C.c_int32()
        check(lib().nhip_slot_length(self.h, slot, C.byref(n)))
        return n.value

    def reset_slot(self, slot: int) -> None:
        check(lib().nhip_slot_reset(self.h, slot))

    def mark_slot(self, slot: int) -> None:
        check(lib().nhip_slot_mark(self.h, slot))

    def rewind_slot(self, slot: int) -> None:
        check(lib().nhip_slot_rewind(self.h, slot))

    def copy_slot(self, dst: int, src: int) -> None:
        check(lib().nhip_slot_copy(self.h, dst, src))

    def feed_slot(self, slot: int, tokens, compute_logits: bool = True):
        """FeedSlot: the last token's logits [vocab] (or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        lg = np.zeros(self.vocab_size, dtype=np.float32) if compute_logits else None
        check(lib().nhip_slot_feed(self.h, slot, _p(t) if len(t) else None, len(t),
                                   _p(lg) if compute_logits else None))
        return lg

    def forward_batch(self, tokens, row_slots, head_rows, k: int = 0, logits: bool = True, argmax: bool = False):
        """ForwardBatch: the head rows' logits [heads][vocab] (or None), top-k
        ids and log-probabilities [heads][k], Ops.ArgMax ids [heads] (or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        s = np.ascontiguousarray(row_slots, dtype=np.int32).reshape(-1)
        if len(s) != len(t):
            raise ValueError(f"{len(t)} tokens but {len(s)} row slots")
        hr_in = np.asarray(head_rows).reshape(-1)
        if hr_in.size and not np.issubdtype(hr_in.dtype, np.integer):
            raise ValueError("head_rows must be integers")
        hr = np.ascontiguousarray(hr_in, dtype=np.int32)
        heads = len(hr)
        lg = np.zeros((heads, self.vocab_size), dtype=np.float32) if logits else None
        idx = np.zeros((max(heads, 1), max(k, 1)), dtype=np.int32)
        lp = np.zeros((max(heads, 1), max(k, 1)), dtype=np.float32)
        am = np.zeros(max(heads, 1), dtype=np.int32)
        check(lib().nhip_step(self.h, _p(t), _p(s), len(t), _p(hr) if heads else None, heads,
                              _p(lg) if logits and heads else None, k, _p(idx), _p(lp), _p(am) if argmax else None))
        return lg, idx[:heads, :k], lp[:heads, :k], (am[:heads] if argmax else None)

    def close(self) -> None:
        if self.h:
            check(lib().nhip_ctx_destroy(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
