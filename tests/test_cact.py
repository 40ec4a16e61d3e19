"""The .cact reader (nhip_open, Model.Open's parse and upload): malformed
archives are rejected before any device work (src/Needle/Model.cs:372-389's
checks); a synthetic archive's codebook-quantized records become device
weights whose matmuls are bit-exact with the oracle over the archive's own
bytes, its dense records fp32 device arrays (fp16 by HalfToSingle)."""
import ctypes as C
import struct

import numpy as np
import pytest

import cact

NHIP_ERR_FORMAT = -4


def codebook_floats(seed=3):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(28) * 0.5).astype(np.float32)


def open_archive(N, data: bytes):
    buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
    h = C.c_void_p()
    rc = N.lib().nhip_open(C.cast(buf, C.c_void_p), len(data), C.byref(h))
    return rc, h, buf


def small_archive():
    cq = cact.cq_payload(np.zeros(16 * 128 // 2, np.uint8), np.zeros(16, np.uint16))
    return cact.write([(cact.CQ, (16, 128), cq, 4), (cact.FP32, (3,), np.ones(3, np.float32).tobytes(), 0)],
                      codebook_floats())


REC = struct.calcsize(cact.RECORD)  # 44: the reference's packed Record
TABLE = 196 + 28 * 4                 # the record table after the header and codebook


@pytest.mark.parametrize("case", ["short", "magic", "table", "record_end", "bits", "group", "dense_end",
                                  "codebook", "dtype", "wrap"])
def test_malformed_archives_are_rejected_before_device_work(case):
    import needle_cs_amd as N
    data = bytearray(small_archive())
    if case == "short":
        data = data[:100]
    elif case == "magic":
        data[0] ^= 1
    elif case == "table":
        struct.pack_into("<I", data, 4, 1000)  # 1000 records cannot fit
    elif case == "record_end":
        struct.pack_into("<Q", data, TABLE + 28, len(data))  # bytes past the end
    elif case == "bits":
        struct.pack_into("<I", data, TABLE + 40, 3)
    elif case == "group":
        struct.pack_into("<I", data, TABLE + 36, 64)
    elif case == "dense_end":
        struct.pack_into("<I", data, TABLE + REC + 4, 1 << 20)  # shape0 far past the data
    elif case == "codebook":
        data = bytearray(cact.write([(cact.FP32, (1,), b"\0" * 4, 0)], codebook_floats()[:20]))
    elif case == "dtype":
        data[TABLE + REC] = 9
    elif case == "wrap":
        # 2^32-ish shapes whose 64-bit element product wraps to a small number
        struct.pack_into("<BBHIIII", data, TABLE + REC, cact.FP32, 3, 0, 1 << 31, 1 << 31, 1 << 2, 0)
    rc, h, _ = open_archive(N, bytes(data))
    assert rc == NHIP_ERR_FORMAT, (case, rc, N.lib().nhip_last_error())
    assert not h.value
    expected = {"short": b"shorter", "magic": b"magic", "table": b"tables", "record_end": b"ends at",
                "bits": b"bits", "group": b"group of 128", "dense_end": b"elements end", "codebook": b"codebook",
                "dtype": b"dtype", "wrap": b"elements end"}[case]
    assert expected in N.lib().nhip_last_error(), (case, N.lib().nhip_last_error())


@pytest.mark.gpu
def test_open_uploads_records(hip, orc):
    rng = np.random.default_rng(11)
    cbf = codebook_floats()
    r4, c4, r2, c2 = 64, 256, 37, 384
    idx4 = rng.integers(0, 256, r4 * c4 // 2, dtype=np.uint8)
    nrm4 = np.array([orc.lib().or_single_to_half_rne(float(v)) for v in rng.uniform(0.2, 2.0, r4 * c4 // 128)],
                    dtype=np.uint16)
    idx2 = rng.integers(0, 256, r2 * c2 // 4, dtype=np.uint8)
    nrm2 = np.array([orc.lib().or_single_to_half_rne(float(v)) for v in rng.uniform(0.2, 2.0, r2 * c2 // 128)],
                    dtype=np.uint16)
    halves = rng.standard_normal(100).astype(np.float16)
    dense32 = rng.standard_normal(15).astype(np.float32)
    blob = b"tokenizer bytes"
    tensors = [(cact.CQ, (r4, c4), cact.cq_payload(idx4, nrm4), 4),
               (cact.FP16, (100,), halves.tobytes(), 0),
               (cact.CQ, (r2, c2), cact.cq_payload(idx2, nrm2), 2),
               (cact.FP32, (3, 5), dense32.tobytes(), 0),
               (cact.RAW, (len(blob),), blob, 0)]
    words = {5: 8192, 7: 768, 8: 12, 9: 2, 10: 4}
    data = cact.write(tensors, cbf, header_words=words, rope_theta=5e5, pad=3)  # unaligned blobs
    rc, h, buf = open_archive(hip, data)
    assert rc == 0, hip.lib().nhip_last_error()
    N = hip
    head = (C.c_uint32 * 48)()
    theta, count = C.c_float(), C.c_int32()
    N.check(N.lib().nhip_model_info(h, head, C.byref(theta), C.byref(count)))
    assert count.value == 5 and theta.value == np.float32(5e5)
    assert head[0] == cact.MAGIC and all(head[k] == v for k, v in words.items())
    offsets = cact.record_offsets(data)
    for i, (dtype, shape, payload, bits) in enumerate(tensors):
        info = N.RecordInfo()
        N.check(N.lib().nhip_model_record(h, i, C.byref(info)))
        assert info.dtype == dtype and info.ndim == len(shape) and tuple(info.shape[:len(shape)]) == shape
        assert info.offset == offsets[i] and info.bytes == len(payload)
        assert bool(N.lib().nhip_model_weights(h, i)) == (dtype == cact.CQ)
        assert bool(N.lib().nhip_model_dense(h, i)) == (dtype in (cact.FP16, cact.FP32))
    assert data[offsets[4]:offsets[4] + len(blob)] == blob

    def download(ptr, n):
        out = np.zeros(n, np.float32)
        N.check(N.lib().nhip_memcpy_dtoh(out.ctypes.data, ptr, n * 4))
        return out
    assert np.array_equal(download(N.lib().nhip_model_dense(h, 1), 100), halves.astype(np.float32))
    assert np.array_equal(download(N.lib().nhip_model_dense(h, 3), 15), dense32)

    # matmuls over the uploaded records == the oracle over the archive's bytes
    # with the reference's codebooks (2-bit: levels 0..3, 4-bit: 12..27)
    arch = np.frombuffer(data, np.uint8)
    for i, bits, rows, cols, nrm in [(0, 4, r4, c4, nrm4), (2, 2, r2, c2, nrm2)]:
        book = orc.codebook(cbf[12:28] if bits == 4 else cbf[0:4], 16 if bits == 4 else 4)
        indices = np.ascontiguousarray(arch[offsets[i]:offsets[i] + rows * cols * bits // 8])
        cq = orc.Cq(orc.p(indices), orc.p(nrm), C.pointer(book), rows, cols, bits)
        tokens = 3
        x = rng.standard_normal(tokens * cols).astype(np.float32)
        act, values, sc, off = orc.prepare(x, tokens, cols, bits)
        want = np.zeros(tokens * rows, np.float32)
        orc.matmul_rows(cq, act, tokens, want, rows, 0, rows)
        dv, ds, do = (N.DeviceBuffer.from_array(a) for a in (values, sc, off))
        dy = N.DeviceBuffer(tokens * rows * 4)
        N.check(N.lib().nhip_matmul_cq_dev(N.lib().nhip_model_weights(h, i), dv.ptr, ds.ptr, do.ptr, act.stride,
                                           tokens, dy.ptr, rows, 0, rows, None))
        assert np.array_equal(dy.download(np.float32).view(np.uint32), want.view(np.uint32)), bits
    N.check(N.lib().nhip_model_close(h))
