"""GPU cold fetch (hs_kv_cold_fetch) from a SegmentedKVStore image in pinned
host memory: the rows come back byte for byte, and every identity or digest
failure the reference's reader refuses (storage/segmented_store.cpp:92-94)
is reported in the status."""
import ctypes

import numpy as np
import pytest
import torch

from hs_data import rng

pytestmark = pytest.mark.gpu


def pinned_image(hs, request, layers, positions, layer, rows):
    L = hs.lib()
    extent = L.hs_kv_store_bytes(layers, positions)
    image = torch.empty(extent, dtype=torch.uint8, pin_memory=True)
    p = ctypes.c_void_p(image.data_ptr())
    assert L.hs_kv_store_init(p, request, layers, positions) == 0
    r = np.ascontiguousarray(rows, dtype=np.uint8)
    assert L.hs_kv_store_append(p, layer, 0, r.ctypes.data_as(ctypes.c_void_p), r.shape[0]) == 0
    return image


def cold_fetch(hs, image, layer, positions):
    L = hs.lib()
    pos = torch.tensor(positions, dtype=torch.int32, device="cuda")
    out = torch.empty((len(positions), 4096), dtype=torch.uint8, device="cuda")
    status = hs.ops.new_status("cuda")
    ws = hs.ops.workspace(L.hs_kv_cold_fetch_workspace_bytes(len(positions)), "cuda")
    hs.check(L.hs_kv_cold_fetch(ctypes.c_void_p(image.data_ptr()), layer,
                                ctypes.c_void_p(pos.data_ptr()), len(positions),
                                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(status.data_ptr()),
                                ctypes.c_void_p(ws.data_ptr()),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return out.cpu().numpy(), hs.ops.read_status(status)


def test_rows_round_trip(hs):
    g = rng(1)
    rows = g.integers(0, 256, size=(300, 4096), dtype=np.uint8)
    image = pinned_image(hs, 77, 3, 512, 2, rows)
    positions = [int(x) for x in g.integers(0, 300, size=1000)]
    out, st = cold_fetch(hs, image, 2, positions)
    assert st["code"] == 0 and st["k"] == 0
    assert np.array_equal(out, rows[positions])


def test_corruption_detected(hs):
    g = rng(2)
    rows = g.integers(0, 256, size=(64, 4096), dtype=np.uint8)
    image = pinned_image(hs, 5, 2, 64, 1, rows)
    raw = image.numpy()
    rec = lambda p: 4096 + (1 * 64 + p) * 4128
    raw[rec(3) + 32 + 1000] ^= 0x40          # payload byte: digest mismatch
    raw[rec(9) + 16] ^= 1                     # request field
    raw[rec(12) + 24] ^= 1                    # layer field
    out, st = cold_fetch(hs, image, 1, list(range(64)))
    assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 3
    # a record never appended (version 0) and a position past the capacity
    blank = pinned_image(hs, 5, 2, 64, 1, rows[:10])
    _, st = cold_fetch(hs, blank, 1, [0, 1, 20])
    assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 1
    _, st = cold_fetch(hs, blank, 1, [0, 64])
    assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 1


def test_bad_header_refused(hs):
    rows = np.zeros((1, 4096), dtype=np.uint8)
    image = pinned_image(hs, 5, 1, 4, 0, rows)
    image.numpy()[0] ^= 1  # magic
    with pytest.raises(hs.HsError):
        cold_fetch(hs, image, 0, [0])
