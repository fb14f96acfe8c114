"""GPU tests of the streaming-ceiling kernels (sgl_rocm_kv_stream): the copy
moves the bytes exactly, the write writes its documented pattern, the read
leaves its destination alone, and lengths are checked on the host."""
import numpy as np
import pytest

import sgl_rocm_kv as kv
from sgl_rocm_kv import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k():
    if hip.device_count() == 0:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    ctx = kv.RocmKvPairCopyKernels(0)
    yield ctx
    ctx.close()


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 3 * (1 << 20) + 16 * 7])
def test_copy_write_read(k, nbytes):
    rng = np.random.default_rng(nbytes)
    src_h = rng.integers(0, 256, nbytes + 64, dtype=np.uint8)
    src, dst = hip.DeviceBuffer.from_array(src_h), hip.DeviceBuffer(nbytes + 64)
    dst.fill(0xAB)
    sb, db = kv.device_buffer(src.ptr, src.nbytes), kv.device_buffer(dst.ptr, dst.nbytes)
    k.stream_ceiling(kv.STREAM_COPY, sb, db, nbytes)
    hip.synchronize()
    got = dst.download()
    np.testing.assert_array_equal(got[:nbytes], src_h[:nbytes])
    assert (got[nbytes:] == 0xAB).all()

    k.stream_ceiling(kv.STREAM_WRITE, None, db, nbytes)
    hip.synchronize()
    words = dst.download()[:nbytes].view(np.uint32).reshape(-1, 4)
    np.testing.assert_array_equal(words[:, 0], np.arange(len(words), dtype=np.uint32))
    assert (words[:, 1:] == np.array([1, 2, 3], np.uint32)).all()

    dst.fill(0xCD)
    k.stream_ceiling(kv.STREAM_READ, sb, db, nbytes)
    hip.synchronize()
    assert (dst.download() == 0xCD).all()


def test_host_checks(k):
    a = hip.DeviceBuffer(64)
    ab = kv.device_buffer(a.ptr, a.nbytes)
    with pytest.raises(kv.KvError) as ei:
        k.stream_ceiling(kv.STREAM_COPY, ab, ab, 40)
    assert ei.value.name == "bytes"
    with pytest.raises(kv.KvError) as ei:
        k.stream_ceiling(kv.STREAM_COPY, ab, ab, 128)
    assert ei.value.name == "src"
    with pytest.raises(kv.KvError) as ei:
        k.stream_ceiling(3, ab, ab, 16)
    assert ei.value.name == "kind"
