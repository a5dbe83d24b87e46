"""The packed expert file (reference serve/pack_store.py:1-90, read by nvtier.py:96-112, 460-486): records of the
blob rounded up to 4 KiB, read back bit for bit through ExpertFile with and without direct I/O, into destinations
with and without room for the whole record (only the blob may land in a blob-sized destination)."""
import ctypes
import mmap
import os

import numpy as np
import pytest

from exl3xpu import nvtier


def _aligned(n):
    m = mmap.mmap(-1, n)                       # page-aligned anonymous memory
    return m, ctypes.addressof(ctypes.c_char.from_buffer(m))


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    H, I, K, L, E = 128, 128, 3, 2, 5
    src = nvtier.SyntheticExpertSource(H, I, K, seed=41, n_distinct=7)
    path = str(tmp_path_factory.mktemp("xf") / "experts.bin")
    meta = nvtier.write_expert_file(path, src, L, E, H, I, K)
    return src, path, meta, L * E


def test_record_layout(packed):
    src, path, meta, n = packed
    assert meta["rec"] % 4096 == 0 and meta["rec"] >= meta["blob"] == src.blob
    assert os.path.getsize(path) == n * meta["rec"]
    raw = np.fromfile(path, dtype=np.uint8).reshape(n, meta["rec"])
    for r in range(n):
        assert np.array_equal(raw[r, :src.blob], src.blob_of(r))
        assert not raw[r, src.blob:].any()     # zero padding up to the 4 KiB boundary


@pytest.mark.parametrize("direct", [None, False])
def test_read_back_full_room(packed, direct):
    src, path, meta, n = packed
    f = nvtier.ExpertFile(path, direct=direct)
    try:
        m, addr = _aligned(meta["rec"])
        for r in (0, 3, n - 1):
            f.read(r, addr, meta["rec"])
            got = np.frombuffer(m, dtype=np.uint8, count=src.blob)
            assert np.array_equal(got, src.blob_of(r))
        assert f.reads == 3
    finally:
        f.close()


@pytest.mark.parametrize("direct", [None, False])
def test_read_into_blob_sized_room(packed, direct):
    """A destination with room for the blob only (a store whose stride is not 4 KiB-rounded): nothing past the blob
    is written, whatever the I/O mode."""
    src, path, meta, n = packed
    f = nvtier.ExpertFile(path, direct=direct)
    try:
        m, addr = _aligned(2 * meta["rec"])
        guard = np.frombuffer(m, dtype=np.uint8)
        guard[:] = 0xA5
        f.read(4, addr, src.blob)
        assert np.array_equal(guard[:src.blob], src.blob_of(4))
        assert (guard[src.blob:] == 0xA5).all()
        f.read(2, addr)                        # room defaults to the blob
        assert np.array_equal(guard[:src.blob], src.blob_of(2))
        assert (guard[src.blob:] == 0xA5).all()
    finally:
        f.close()


def test_short_read_raises(packed):
    src, path, meta, n = packed
    f = nvtier.ExpertFile(path, direct=False)
    try:
        m, addr = _aligned(meta["rec"])
        with pytest.raises(OSError):
            f.read(n, addr, meta["rec"])       # one record past the end
    finally:
        f.close()


def test_meta_rejects_unaligned_records(packed, tmp_path):
    src, path, meta, n = packed
    bad = dict(meta, rec=meta["blob"] + 1)
    with pytest.raises(ValueError):
        nvtier.ExpertFile(path, meta=bad)
