"""p0_upload_file (the pack reader's I/O, engine/core/store.js:221-244) through the C ABI: a byte range of a file lands
in device memory exactly, across the 16 MB chunks of the two pinned staging buffers, at any byte offsets."""
import numpy as np
import pytest

from p0pc0rn_amd import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,offset,dst_off", [(40 * (1 << 20) + 12345, 4096 + 7, 256 + 3), (100, 0, 0),
                                                   (16 << 20, 1, 0)])
def test_upload_file_range_exact(dev, tmp_path, nbytes, offset, dst_off):
    data = np.random.default_rng(nbytes).integers(0, 256, offset + nbytes + 999, dtype=np.uint8)
    p = tmp_path / "shard.bin"
    data.tofile(str(p))
    buf = capi.Buffer(dst_off + nbytes + 64).fill_u32(0xDEADBEEF)
    capi.upload_file(str(p), offset, nbytes, buf, dst_off)
    got = buf.read(np.uint8)
    assert np.array_equal(got[dst_off:dst_off + nbytes], data[offset:offset + nbytes])
    assert np.all(got[:dst_off] == np.frombuffer(np.uint32(0xDEADBEEF).tobytes() * (dst_off // 4 + 1), np.uint8)[:dst_off])
    buf.free()


def test_upload_file_errors(dev, tmp_path):
    buf = capi.Buffer(64)
    with pytest.raises(capi.P0Error, match="No such file"):
        capi.upload_file(str(tmp_path / "missing.bin"), 0, 16, buf)
    (tmp_path / "short.bin").write_bytes(b"\1" * 10)
    with pytest.raises(capi.P0Error, match="end of file"):
        capi.upload_file(str(tmp_path / "short.bin"), 0, 16, buf)
    buf.free()
