"""Cold-tier format pins (CPU): FNV-1a 64 against its published vectors and
the compiled reference checksum() (storage/file_store.cpp:12-16); the oracle
image byte-identical to a file written by the compiled reference
SegmentedKVStore (storage/segmented_store.cpp:18-38, 77-82); the product
library's host writer byte-identical to the oracle image; the geometry the
reference refuses (segmented_store.cpp:31) refused here too."""
import ctypes

import numpy as np
import pytest

from hs_data import rng

VECTORS = {b"": 0xCBF29CE484222325, b"a": 0xAF63DC4C8601EC8C, b"foobar": 0x85944171F73967E8}


def test_fnv1a_published_vectors(port):
    for data, want in VECTORS.items():
        assert port.fnv1a64(np.frombuffer(data, dtype=np.uint8)) == want


def test_fnv1a_against_reference(port, ref):
    if ref is None:
        pytest.skip("compiled reference not built")
    g = rng(3)
    for n in (1, 7, 4096, 10000):
        data = g.integers(0, 256, size=n, dtype=np.uint8)
        assert port.fnv1a64(data) == ref.checksum(data)


@pytest.mark.parametrize("layers,positions,layer,count", [(3, 70, 1, 5), (1, 1, 0, 1),
                                                           (4, 130, 3, 130)])
def test_oracle_image_equals_reference_file(port, ref, tmp_path, layers, positions, layer, count):
    if ref is None:
        pytest.skip("compiled reference not built")
    g = rng(layers * 1000 + count)
    rows = g.integers(0, 256, size=(count, 4096), dtype=np.uint8)
    want = ref.segmented_file(tmp_path / "kv", 991, layers, positions, layer, rows)
    got = port.kv_store_image(991, layers, positions, layer, rows)
    assert got.size == want.size and np.array_equal(got, want)


def product_image(hs, request, layers, positions, layer, rows, first=0):
    L = hs.lib()
    extent = L.hs_kv_store_bytes(layers, positions)
    image = np.zeros(extent, dtype=np.uint8)
    p = image.ctypes.data_as(ctypes.c_void_p)
    assert L.hs_kv_store_init(p, request, layers, positions) == 0
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    assert L.hs_kv_store_append(p, layer, first, rows.ctypes.data_as(ctypes.c_void_p),
                                rows.shape[0]) == 0
    return image


def test_product_writer_equals_oracle(port):
    import hillserve_amd as hs
    g = rng(9)
    rows = g.integers(0, 256, size=(9, 4096), dtype=np.uint8)
    got = product_image(hs, 1234, 2, 40, 1, rows, first=17)
    want = port.kv_store_image(1234, 2, 40, 1, rows, first=17)
    assert np.array_equal(got, want)


def test_refused_geometry():
    import hillserve_amd as hs
    L = hs.lib()
    assert L.hs_kv_store_bytes(0, 10) == 0 and L.hs_kv_store_bytes(129, 10) == 0
    assert L.hs_kv_store_bytes(1, 0) == 0 and L.hs_kv_store_bytes(1, 66049) == 0
    assert L.hs_kv_store_bytes(32, 66048) > 0
    image = np.zeros(L.hs_kv_store_bytes(1, 8), dtype=np.uint8)
    p = image.ctypes.data_as(ctypes.c_void_p)
    assert L.hs_kv_store_init(p, 1, 1, 8) == 0
    row = np.zeros(4096 * 2, dtype=np.uint8).ctypes.data_as(ctypes.c_void_p)
    assert L.hs_kv_store_append(p, 0, 7, row, 2) == hs.HS_ERR_ARGUMENT  # past capacity
    assert L.hs_kv_store_append(p, 1, 0, row, 1) == hs.HS_ERR_ARGUMENT  # no such layer
