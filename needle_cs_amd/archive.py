"""Synthetic .cact archives in the reference's layout.

write() lays out an archive as Model.Open reads it (src/Needle/Model.cs:190-197
Record, ModelInfo.cs:7-8 magic and the 196-byte header; the same struct
formats as tools/golden.py:16-17): a header of 48 uint32 words + the RoPE
theta float, the codebook floats, the table of packed 44-byte records, then
each record's data.

needle3_archive() writes a random-init Needle 3 model of a chosen geometry
in the order Model.Open reads it (Model.cs:307-371): the 4-bit embedding, per
layer LayerWeights (Model.cs:133-151: NormIn, Q, K, V, QTaps, KTaps, VTaps,
QNorm, KNorm, Gate, Out, PostNorm, AttnGate, PreHada, then MlpWeights,
src/Needle/Audio.cs:11-26), HyperConnections (Model.cs:160-173, the two
permutations stored as float records), the engram sites (Model.cs:181-187),
FinalNorm and the tokenizer blob; header words as Geometry reads them
(Model.cs:75-104).  Values are seeded random draws scaled to keep every
activation finite and in range: the reference ships no Needle 3 weights
offline, so these archives drive the engine's parity tests and benchmarks.

Record shapes follow the real archive where the reference's numpy forward
reads them (tools/golden.py): D1 and D4 span the MLP width (it multiplies
them with the zero-padded width, golden.py:186-195; the engine reads their
first `dim` entries, Blocks.cs:1135 and :1216), BPre / BPost are [layers][4]
and BRes [layers][4][4] (golden.py:258-263).  The engram value weights and
the MLP's output scale D4 are drawn large enough that the engram and the MLP
move each layer's output by well over the engine's int8 activation noise, so
a misplaced engram site or MLP shows against that forward.
"""
from __future__ import annotations

import math
import struct

import numpy as np

MAGIC = 0x05E12A84
HEADER = "<48If"
RECORD = "<BBHIIIIQQII"
FP16, FP32, CQ, RAW = 1, 2, 3, 4


def write(tensors, codebook, header_words=None, rope_theta=10000.0, pad=0):
    """tensors: list of (dtype, shape, payload bytes, bits); returns the
    archive bytes.  `pad` extra bytes between blobs (alignment tests)."""
    words = [0] * 48
    for k, v in (header_words or {}).items():
        words[k] = v
    words[0] = MAGIC
    words[1] = len(tensors)
    words[2] = len(codebook)
    head = struct.pack(HEADER, *words, rope_theta)
    cb = np.asarray(codebook, dtype=np.float32).tobytes()
    table_size = struct.calcsize(RECORD) * len(tensors)
    offset = len(head) + len(cb) + table_size
    records, blobs = [], []
    for dtype, shape, payload, bits in tensors:
        offset += pad
        shp = list(shape) + [0] * (4 - len(shape))
        group = 128 if dtype == CQ else 0
        records.append(struct.pack(RECORD, dtype, len(shape), 0, *shp, offset, len(payload), group, bits))
        blobs.append(b"\0" * pad + payload)
        offset += len(payload)
    return head + cb + b"".join(records) + b"".join(blobs)


def cq_payload(indices: np.ndarray, norms: np.ndarray) -> bytes:
    """A codebook-quantized record's data: index bytes, then fp16 norms."""
    return np.ascontiguousarray(indices, dtype=np.uint8).tobytes() + np.ascontiguousarray(norms, np.uint16).tobytes()


def record_offsets(archive: bytes):
    n = struct.unpack_from("<I", archive, 4)[0]
    cb = struct.unpack_from("<I", archive, 8)[0]
    base = struct.calcsize(HEADER) + cb * 4
    size = struct.calcsize(RECORD)
    return [struct.unpack_from(RECORD, archive, base + i * size)[7] for i in range(n)]


# ------------------------------------------------------------ Needle 3 --

# Needle 3's geometry as FormatTests.RealModelReportsItsFormatAndGeometry pins
# it (tests/Needle.Tests/FormatTests.cs:106-121): vocab 8192, hidden 768, 20
# layers, 12 query / 2 KV heads, qk 48, v 64, 8192 positions, window 1024, 5
# engram sites, RoPE theta 1e5.  The MLP size 1024 (32 x 32 Kronecker
# factors) is HadamardMlpTests' Needle 3 shape (KernelTests.cs:440);
# 3 engram heads per order and the dilation 3 are tools/golden.py:146-172's.
# Not pinned by any file here, so chosen: the global layers (every fourth),
# the engram sites, the orders (2, 3) and 16384 slots per table.
NEEDLE3 = dict(vocab=8192, dim=768, heads=12, kv_heads=2, qk=48, vd=64, layers=20, max_seq=8192, hada_n=1024,
               window=1024, global_layers=(3, 7, 11, 15, 19), engram_slots=16384, engram_sub=128, engram_tables=6,
               engram_dilation=3, orders=(2, 3), sites=(1, 5, 9, 13, 17), rope_theta=100000.0)

# A small model of the same layer program for fast parity tests: one global
# layer between windowed ones (window 6), one engram site.
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


def needle3_archive(g: dict, seed: int) -> bytes:
    """A random-init Needle 3 archive of geometry g (NEEDLE3, SMALL, ...)."""
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
        norms = rng.uniform(lo, hi, n * (k // 128)).astype(np.float16).view(np.uint16)
        tensors.append((CQ, (n, k), cq_payload(idx, norms), bits))

    def dense(shape, values, half=False):
        a = np.asarray(values, dtype=np.float16 if half else np.float32).reshape(-1)
        tensors.append((FP16 if half else FP32, shape, a.tobytes(), 0))

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
        dense((width,), np.r_[rng.uniform(0.5, 1.5, d), np.ones(width - d)])    # D1
        dense((width,), rng.uniform(0.5, 1.5, width))                           # D2
        dense((width,), rng.uniform(-0.1, 0.1, width))                          # B2
        dense((width,), rng.uniform(0.5, 1.5, width))                           # D3
        dense((width,), np.r_[rng.uniform(0.2, 0.8, d), np.ones(width - d)])    # D4
        for n in (rows, cols, rows, cols, rows, cols):                          # W1A, W1B, W2A, W2B, W3A, W3B
            dense((n, n), rng.standard_normal(n * n) / math.sqrt(n))
        dense((d, 8), rng.standard_normal(d * 8) * 0.05)                        # CondV
        dense((8, width), rng.uniform(-0.2, 0.2, 8 * width))                    # CondU
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # APre
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # APost
    dense((L,), rng.uniform(0.5, 1.5, L))                                       # ARes
    dense((L, 4), rng.uniform(-1, 1, L * 4))                                    # BPre
    dense((L, 4), rng.uniform(-1, 1, L * 4))                                    # BPost
    dense((L, 4, 4), rng.uniform(-1, 1, L * 16))                                # BRes
    cq(L * 4, 4 * d, 4)                                                         # PhiPre
    cq(L * 4, 4 * d, 4)                                                         # PhiPost
    cq(L * 16, 4 * d, 4)                                                        # PhiRes
    dense((width,), rng.permutation(width).astype(np.float32))                  # PermA
    dense((width,), rng.permutation(width).astype(np.float32))                  # PermB
    for _ in g["sites"]:
        cq(g["engram_tables"] * g["engram_slots"], g["engram_sub"], 2, 0.05, 0.3)  # Tables
        cq(d, d, 2)                                                             # Key
        cq(d, d, 2, 0.02, 0.2)                                                  # Value
        dense((4, d), rng.uniform(-0.5, 0.5, 4 * d))                            # Taps
    dense((d,), rng.uniform(-0.2, 0.2, d))                                      # FinalNorm
    tensors.append((RAW, (16,), bytes(range(16)), 0))                           # tokenizer blob
    return write(tensors, codebook, header_words(g), rope_theta=g["rope_theta"])


def parse(archive: bytes):
    """(header words, theta, codebook floats, records) of an archive."""
    words = struct.unpack_from("<48I", archive, 0)
    theta = struct.unpack_from("<f", archive, 192)[0]
    base = struct.calcsize(HEADER)
    book = np.frombuffer(archive, dtype=np.float32, count=words[2], offset=base)
    table = base + 4 * words[2]
    size = struct.calcsize(RECORD)
    recs = [struct.unpack_from(RECORD, archive, table + i * size) for i in range(words[1])]
    return words, theta, book, recs
