"""Synthetic .cact archives for the reader's tests, in the reference's
layout (src/Needle/Model.cs:190-197 Record, ModelInfo.cs:7-8 magic and the
196-byte header; the same struct formats as tools/golden.py:16-17): a
header of 48 uint32 words + the RoPE theta float, the codebook floats, the
table of packed 44-byte records, then each record's data."""
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
