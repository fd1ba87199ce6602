"""The weight upload path (iris_hip_memcpy_h2d): copies of 8 MiB and more go
through pinned staging buffers with the host copy overlapped with the DMA.
Bitwise round trips for ragged sizes and unaligned sources, source reuse right
after the call, and the rate from a memory-mapped file (the loaders' case:
safetensors files are mapped, iris_safetensors.c)."""
import os
import time

import numpy as np
import pytest

import iris_testlib as tl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return tl.hip()


def roundtrip(lib, src):
    d = tl.Dev(src.nbytes)
    assert lib.iris_hip_memcpy_h2d(d.ptr, src.ctypes.data, src.nbytes) == 0, lib.iris_hip_last_error()
    assert lib.iris_hip_sync() == 0
    return d


@pytest.mark.parametrize("nbytes,offset", [(100 * 2**20 + 12345, 3), (8 * 2**20, 0), (8 * 2**20 - 1, 1),
                                           (64 * 2**20 + 1, 7)])
def test_bitwise(lib, nbytes, offset):
    raw = np.random.default_rng(nbytes).integers(0, 256, nbytes + offset, dtype=np.uint8)
    src = raw[offset:]
    d = roundtrip(lib, src)
    assert np.array_equal(d.get(np.uint8, (nbytes,)), src)


def test_source_reusable_after_return(lib):
    """The call returns once the source is copied out: overwriting it right
    away does not change what lands on the device."""
    n = 48 * 2**20
    buf = np.full(n, 7, np.uint8)
    d1, d2 = tl.Dev(n), tl.Dev(n)
    assert lib.iris_hip_memcpy_h2d(d1.ptr, buf.ctypes.data, n) == 0
    buf[:] = 9
    assert lib.iris_hip_memcpy_h2d(d2.ptr, buf.ctypes.data, n) == 0
    assert lib.iris_hip_sync() == 0
    assert (d1.get(np.uint8, (n,)) == 7).all() and (d2.get(np.uint8, (n,)) == 9).all()


def test_mmap_file_rate(lib, tmp_path):
    """1 GiB from a memory-mapped file (in the page cache, as after the first
    load of a model): correct, and the rate is printed."""
    n = 2**30
    path = str(tmp_path / "blob.bin")
    pattern = np.arange(2**20, dtype=np.uint32)
    with open(path, "wb") as f:
        for i in range(n // pattern.nbytes):
            f.write((pattern + np.uint32(i)).tobytes())
    m = np.memmap(path, np.uint8, "r")
    d = tl.Dev(n)
    m.sum(dtype=np.uint64)   # page cache warm
    t0 = time.perf_counter()
    assert lib.iris_hip_memcpy_h2d(d.ptr, m.ctypes.data, n) == 0
    assert lib.iris_hip_sync() == 0
    dt = time.perf_counter() - t0
    # the same bytes as 4 MiB copies, which take the plain pageable hipMemcpyAsync path
    piece = 4 * 2**20
    t0 = time.perf_counter()
    for off in range(0, n, piece):
        assert lib.iris_hip_memcpy_h2d(d.ptr + off, m.ctypes.data + off, piece) == 0
    assert lib.iris_hip_sync() == 0
    dt_plain = time.perf_counter() - t0
    print(f"upload 1 GiB from a mapped file: staged {dt * 1e3:.1f} ms = {n / dt / 1e9:.1f} GB/s, "
          f"pageable 4 MiB copies {dt_plain * 1e3:.1f} ms = {n / dt_plain / 1e9:.1f} GB/s")
    got = d.get(np.uint8, (n,))
    assert np.array_equal(got, np.asarray(m))
    del m
    os.remove(path)
