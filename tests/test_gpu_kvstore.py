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


def cold_fetch(hs, image, layer, positions, split=False):
    """Fetched records as [count][4096] bytes; with split, fetched into a K
    array and a V array of 2048 B rows and joined again here."""
    pos = torch.tensor(positions, dtype=torch.int32, device="cuda")
    if split:
        k_out = torch.empty((len(positions), 2048), dtype=torch.uint8, device="cuda")
        v_out = torch.empty((len(positions), 2048), dtype=torch.uint8, device="cuda")
        status = hs.ops.kv_cold_fetch(image, layer, pos, k_out, v_out=v_out, row_bytes=2048)
        out = torch.cat([k_out, v_out], dim=1)
    else:
        out = torch.empty((len(positions), 4096), dtype=torch.uint8, device="cuda")
        status = hs.ops.kv_cold_fetch(image, layer, pos, out)
    return out.cpu().numpy(), hs.ops.read_status(status)


@pytest.mark.parametrize("split", [False, True])
def test_rows_round_trip(hs, split):
    g = rng(1)
    rows = g.integers(0, 256, size=(300, 4096), dtype=np.uint8)
    image = pinned_image(hs, 77, 3, 512, 2, rows)
    positions = [int(x) for x in g.integers(0, 300, size=1000)]
    out, st = cold_fetch(hs, image, 2, positions, split=split)
    assert st["code"] == 0 and st["k"] == 0
    assert np.array_equal(out, rows[positions])


def test_corruption_detected(hs):
    g = rng(2)
    rows = g.integers(0, 256, size=(64, 4096), dtype=np.uint8)
    image = pinned_image(hs, 5, 2, 64, 1, rows)
    raw = image.numpy()
    rec = lambda p: 4096 + (1 * 64 + p) * 4128
    raw[rec(3) + 32 + 1000] ^= 0x40          # K half payload byte: digest mismatch
    raw[rec(5) + 32 + 3000] ^= 0x01          # V half payload byte
    raw[rec(9) + 16] ^= 1                     # request field
    raw[rec(12) + 24] ^= 1                    # layer field
    for split in (False, True):  # the digest covers the K and the V half
        out, st = cold_fetch(hs, image, 1, list(range(64)), split=split)
        assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 4
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


def test_cold_plan_and_padded_fetch(hs):
    # selection bitmaps of 4 heads over n tokens, half the 64-token blocks hot
    g = rng(4)
    n, heads = 4000, 4
    words = (n + 31) // 32
    member = g.integers(0, 2**32, size=(heads, words), dtype=np.uint64).astype(np.uint32)
    member &= g.integers(0, 2**32, size=(heads, words), dtype=np.uint64).astype(np.uint32)
    member[:, -1] &= (1 << (n - 32 * (words - 1))) - 1
    hot_blocks = g.permutation((n + 63) // 64)[: (n + 63) // 128]
    slot = np.full(n, -1, dtype=np.int32)
    next_slot = 0
    for b in sorted(hot_blocks):
        for t in range(b * 64, min(n, b * 64 + 64)):
            slot[t] = next_slot
            next_slot += 1
    cold_tokens = int((slot < 0).sum())
    staging_base = next_slot
    L = hs.lib()
    md = torch.from_numpy(member.view(np.int32)).cuda()
    sd = torch.from_numpy(slot).cuda()
    pos = torch.empty(cold_tokens, dtype=torch.int32, device="cuda")
    rows = torch.empty(n, dtype=torch.int32, device="cuda")
    count = torch.empty(1, dtype=torch.int32, device="cuda")
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    hs.check(L.hs_gqa_cold_plan(vp(md), heads, n, vp(sd), staging_base, cold_tokens, vp(pos),
                                vp(rows), vp(count), st))
    any_sel = np.zeros(n, dtype=bool)
    for h in range(heads):
        bits = np.unpackbits(member[h].view(np.uint8), bitorder="little")[:n].astype(bool)
        any_sel |= bits
    want = np.nonzero(any_sel & (slot < 0))[0]
    got_pos = pos.cpu().numpy().view(np.uint32)
    assert int(count.item()) == want.size
    assert np.array_equal(got_pos[: want.size], want)
    assert np.all(got_pos[want.size:] == 0xFFFFFFFF)
    want_rows = np.where(slot >= 0, slot, -1)
    want_rows[want] = staging_base + np.arange(want.size)
    assert np.array_equal(rows.cpu().numpy(), want_rows)
    # the padded list fetches exactly the listed cold records
    data = g.integers(0, 256, size=(n, 4096), dtype=np.uint8)
    image = pinned_image(hs, 9, 1, n, 0, data)
    out = torch.zeros((cold_tokens, 4096), dtype=torch.uint8, device="cuda")
    status = hs.ops.new_status("cuda")
    hs.ops.kv_cold_fetch(image, 0, pos, out, status=status)
    assert hs.ops.read_status(status)["code"] == 0
    o = out.cpu().numpy()
    assert np.array_equal(o[: want.size], data[want])
    assert not o[want.size:].any()  # padding rows untouched
