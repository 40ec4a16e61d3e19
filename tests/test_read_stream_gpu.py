"""The bandwidth-calibration read (nhip_read_stream_dev) reads every byte:
each 32 KB workgroup's sink word is the XOR of the words it covers (the
tail chunk partial), checked against numpy."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 32768, 3 * 32768 + 4080, 17930240])
def test_read_stream_folds_every_word(hip, nbytes):
    rng = np.random.default_rng(nbytes)
    data = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = hip.DeviceBuffer.from_array(data)
    chunks = -(-nbytes // 32768)
    sink = hip.DeviceBuffer(chunks * 4)
    hip.check(hip.lib().nhip_read_stream_dev(src.ptr, nbytes, sink.ptr, None))
    got = sink.download(np.uint32)
    pad = np.zeros(chunks * 8192, dtype=np.uint32)
    pad[: data.size] = data
    want = np.bitwise_xor.reduce(pad.reshape(chunks, 8192), axis=1)
    assert np.array_equal(got, want)


def test_read_stream_rejects_unaligned_sizes(hip):
    buf = hip.DeviceBuffer(1024)
    assert hip.lib().nhip_read_stream_dev(buf.ptr, 1000, buf.ptr, None) != 0
