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


def runs_fetch(hs, image, layer, positions, split=False):
    """The same read through hs_kv_cold_fetch_runs (the copy engines move the
    runs of consecutive positions into a raw staging buffer)."""
    pos = torch.tensor(positions, dtype=torch.int32, device="cuda")
    raw = torch.empty((len(positions), 4128), dtype=torch.uint8, device="cuda")
    runs = hs.ops.cold_runs(positions)
    if split:
        k_out = torch.empty((len(positions), 2048), dtype=torch.uint8, device="cuda")
        v_out = torch.empty((len(positions), 2048), dtype=torch.uint8, device="cuda")
        status = hs.ops.kv_cold_fetch_runs(image, layer, runs, raw, pos, k_out, v_out=v_out,
                                           row_bytes=2048)
        out = torch.cat([k_out, v_out], dim=1)
    else:
        out = torch.empty((len(positions), 4096), dtype=torch.uint8, device="cuda")
        status = hs.ops.kv_cold_fetch_runs(image, layer, runs, raw, pos, out)
    return out.cpu().numpy(), hs.ops.read_status(status), runs[2]


@pytest.mark.parametrize("split", [False, True])
def test_runs_fetch_equals_kernel_fetch(hs, split):
    """Ascending positions in runs of random lengths (64-token blocks and
    single rows): the staged rows equal the kernel read's byte for byte."""
    g = rng(3)
    n = 4096
    rows = g.integers(0, 256, size=(n, 4096), dtype=np.uint8)
    image = pinned_image(hs, 91, 2, n, 1, rows)
    blocks = np.sort(g.permutation(n // 64)[: n // 128])
    positions = sorted({int(b) * 64 + t for b in blocks for t in range(64)} |
                       {int(x) for x in g.integers(0, n, size=200)})
    want, st_k = cold_fetch(hs, image, 1, positions, split=split)
    got, st_r, runs = runs_fetch(hs, image, 1, positions, split=split)
    assert runs > 1
    assert st_k["code"] == 0 and st_r["code"] == 0 and st_r["k"] == 0
    assert np.array_equal(got, want)
    assert np.array_equal(got, rows[positions])


def test_runs_fetch_corruption_and_rejections(hs):
    g = rng(4)
    rows = g.integers(0, 256, size=(128, 4096), dtype=np.uint8)
    image = pinned_image(hs, 6, 1, 128, 0, rows)
    raw = image.numpy()
    rec = lambda p: 4096 + p * 4128
    raw[rec(70) + 32 + 17] ^= 0x80           # payload: digest mismatch
    raw[rec(90) + 8] ^= 1                     # position field
    positions = list(range(64, 128))
    _, st, _ = runs_fetch(hs, image, 0, positions)
    assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 2
    # an expected position that differs from the staged record's is an identity failure
    L = hs.lib()
    pos = torch.tensor(positions[:8], dtype=torch.int32, device="cuda")
    wrong = torch.tensor([64, 65, 66, 67, 68, 69, 71, 71], dtype=torch.int32, device="cuda")
    out = torch.empty((8, 4096), dtype=torch.uint8, device="cuda")
    stage = torch.empty((8, 4128), dtype=torch.uint8, device="cuda")
    st = hs.ops.kv_cold_fetch_runs(image, 0, hs.ops.cold_runs(range(64, 72)), stage, wrong, out)
    assert hs.ops.read_status(st) == {"code": hs.HS_ERR_CORRUPT, "k": 1, "boundary_tied_heads": 0,
                                      "head0_max_key": 0}
    # runs that do not hold exactly `count` records, or leave the layer
    ws = hs.ops.workspace(L.hs_kv_cold_fetch_workspace_bytes(8))
    status = hs.ops.new_status()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    for firsts, counts in (([64], [7]), ([64], [9]), ([124], [8]), ([200], [8])):
        f = (ctypes.c_uint32 * 1)(*firsts)
        c = (ctypes.c_uint32 * 1)(*counts)
        rc = L.hs_kv_cold_fetch_runs(vp(image), 0, ctypes.cast(f, ctypes.c_void_p),
                                     ctypes.cast(c, ctypes.c_void_p), 1, vp(stage), vp(pos), 8,
                                     vp(out), ctypes.c_void_p(out.data_ptr() + 2048), 4096,
                                     vp(status), vp(ws), None)
        assert rc == hs.HS_ERR_ARGUMENT, (firsts, counts)
