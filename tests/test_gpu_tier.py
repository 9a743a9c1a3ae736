"""The hot/cold chain of configs[4] end to end on the GPU (the hot / cold
split of FullGqaRuntimePolicy::fetch, policy/full_gqa_runtime.cpp:586-690,
and the record checks of SegmentedKVStore::fetch,
storage/segmented_store.cpp:85-95).

Per sequence: half of the 64-token blocks sit in an HBM hot pool (seeded
block permutation), every row is in a pinned SegmentedKVStore image.  The
chain is batched score -> batched id-order selection -> cold plan -> device
cold fetch into staging rows after the hot rows -> sparse attention through
the hot/staging row map.  The output must equal, bit for bit, the same
attention over an all-hot pool (the row map only moves where a row is read
from), the selected ids must equal the oracle's, and the output must be
within 2e-3 of the FP64 oracle attention over the oracle's selection."""
import ctypes

import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, pool_rows, rng, rope_keys, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3
ALPHA, RATIO = 5.0, 0.2


def _sequence(g, n, seed):
    k = rope_keys(n, seed)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    rows = pool_rows(k, v)  # [n][2048] u16: 4096 B records, K then V
    blocks = (n + 63) // 64
    hot_blocks = np.sort(g.permutation(blocks)[: blocks // 2])
    slot = np.full(n, -1, dtype=np.int32)
    hot = []
    for b in hot_blocks:
        for t in range(b * 64, min(n, b * 64 + 64)):
            slot[t] = len(hot)
            hot.append(t)
    return k, rows, slot, np.asarray(hot, dtype=np.int64)


def _image(hs, rows, request):
    L = hs.lib()
    n = rows.shape[0]
    image = torch.empty(L.hs_kv_store_bytes(1, n), dtype=torch.uint8, pin_memory=True)
    p = ctypes.c_void_p(image.data_ptr())
    assert L.hs_kv_store_init(p, request, 1, n) == 0
    r = np.ascontiguousarray(rows).view(np.uint8)
    assert L.hs_kv_store_append(p, 0, 0, r.ctypes.data_as(ctypes.c_void_p), n) == 0
    return image


@pytest.mark.parametrize("n", [4096, 6080])
def test_hot_cold_chain(hs, port, n):
    g = rng(4400 + n)
    seqs = []
    for s in range(2):
        k, rows, slot, hot = _sequence(g, n, 70 + 10 * s + n)
        q16 = f16_bits(g.standard_normal((32, 128)))
        q32 = g.standard_normal((32, 128)).astype(np.float32)
        seqs.append(dict(k=k, rows=rows, slot=slot, hot=hot, q16=q16, q32=q32))
    # batched score over every token's HBM-resident K, batched id-order select
    jobs = []
    for s, d in enumerate(seqs):
        jobs.append(dict(q16=to_dev(d["q16"].reshape(-1)), keys=to_dev(d["k"].reshape(-1)),
                         tokens=n, head0_partial=torch.empty((n + 63) // 64, dtype=torch.int32,
                                                             device="cuda")))
    scores = hs.ops.score_batched(jobs)
    words = (n + 31) // 32
    members = [torch.empty((32, words), dtype=torch.int32, device="cuda") for _ in seqs]
    sel = hs.ops.select_batched(
        [dict(scores=scores[s], n=n, head0_partial=jobs[s]["head0_partial"], member=members[s])
         for s in range(len(seqs))], 32, ALPHA, RATIO, scale_raw=True, id_order=True,
        require_k=True)
    L = hs.lib()
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for s, d in enumerate(seqs):
        ids, counts, member, status = sel[s]
        stt = hs.ops.read_status(status)
        assert stt["code"] == 0
        kk = stt["k"]
        # the oracle's selection over the same raw scores
        raw = port.score(d["q16"], d["rows"].reshape(-1), n, 2048)
        assert np.array_equal(from_dev(scores[s]), raw)
        rc, ok, pids, _, _ = port.select(port.scale(raw), 32, n, n, ALPHA, RATIO)
        assert rc == 0 and ok == kk
        assert np.array_equal(from_dev(ids)[:, :kk], np.sort(pids, axis=1))
        # hot pool + staging rows; cold plan; cold fetch from the pinned image
        hot_rows = d["hot"].size
        cold_tokens = n - hot_rows
        pool = torch.zeros((hot_rows + cold_tokens, 2048), dtype=torch.float16, device="cuda")
        pool[:hot_rows] = to_dev(d["rows"][d["hot"]])
        image = _image(hs, d["rows"], 900 + s)
        slot_d = to_dev(d["slot"])
        pos = torch.empty(cold_tokens, dtype=torch.int32, device="cuda")
        rowmap = torch.empty(n, dtype=torch.int32, device="cuda")
        count = torch.empty(1, dtype=torch.int32, device="cuda")
        hs.check(L.hs_gqa_cold_plan(vp(member), 32, n, vp(slot_d), hot_rows, cold_tokens,
                                    vp(pos), vp(rowmap), vp(count), st))
        staging = pool[hot_rows:]
        cstatus = hs.ops.kv_cold_fetch(image, 0, pos, staging)
        q32 = torch.from_numpy(d["q32"]).cuda()
        out = hs.ops.sparse_attention(q32, pool.reshape(-1), n, member, rows=rowmap)
        assert hs.ops.read_status(cstatus)["code"] == 0
        # every selected cold token was fetched, and only those
        any_sel = np.zeros(n, dtype=bool)
        for h in range(32):
            any_sel[np.sort(pids[h])] = True
        want = np.nonzero(any_sel & (d["slot"] < 0))[0]
        assert int(count.item()) == want.size
        assert np.array_equal(from_dev(pos)[: want.size], want)
        # the same attention over an all-hot pool (rows in id order, no map)
        full = to_dev(d["rows"].reshape(-1))
        ref_dev = hs.ops.sparse_attention(q32, full, n, member)
        got = out.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref_dev.cpu().numpy().view(np.uint32)), \
            "hot + fetched-cold attention differs from the all-hot attention"
        ref = port.attention(d["q32"], d["rows"].view(np.uint8).reshape(-1), list(pids))
        err = np.max(np.linalg.norm(got.astype(np.float64) - ref, axis=1)
                     / np.linalg.norm(ref, axis=1))
        assert err <= TOL, err


@pytest.mark.parametrize("n", [4096])
def test_hot_cold_chain_copy_engines(hs, port, n):
    """configs[4]'s copy-engine variant: every cold row of the layer staged by
    hs_kv_cold_fetch_runs (runs of consecutive cold positions, one
    hipMemcpyAsync each), a static row map (hot token -> its slot, cold token
    -> staging row of its rank among the cold positions), attention through
    it.  Output bit for bit the all-hot attention."""
    g = rng(5400 + n)
    k, rows, slot, hot = _sequence(g, n, 333)
    q16 = f16_bits(g.standard_normal((32, 128)))
    q32 = g.standard_normal((32, 128)).astype(np.float32)
    part = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    raw = hs.ops.score(to_dev(q16.reshape(-1)), to_dev(k.reshape(-1)), n, head0_partial=part)
    member = torch.empty((32, (n + 31) // 32), dtype=torch.int32, device="cuda")
    _, _, _, status = hs.ops.select(raw, 32, n, n, ALPHA, RATIO, scale_raw=True, id_order=True,
                                    require_k=True, head0_partial=part, member=member)
    assert hs.ops.read_status(status)["code"] == 0
    cold = np.nonzero(slot < 0)[0]
    hot_rows = n - cold.size
    pool = torch.zeros((n, 2048), dtype=torch.float16, device="cuda")
    pool[:hot_rows] = to_dev(rows[hot])
    rowmap = slot.astype(np.int32).copy()
    rowmap[cold] = hot_rows + np.arange(cold.size, dtype=np.int32)
    image = _image(hs, rows, 77)
    runs = hs.ops.cold_runs(cold)
    assert runs[2] > 1
    stage = torch.empty((cold.size, 4128), dtype=torch.uint8, device="cuda")
    cstatus = hs.ops.kv_cold_fetch_runs(image, 0, runs, stage, to_dev(cold.astype(np.int32)),
                                        pool[hot_rows:])
    q = torch.from_numpy(q32).cuda()
    out = hs.ops.sparse_attention(q, pool.reshape(-1), n, member, rows=to_dev(rowmap))
    assert hs.ops.read_status(cstatus)["code"] == 0
    ref_dev = hs.ops.sparse_attention(q, to_dev(rows.reshape(-1)), n, member)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref_dev.cpu().numpy().view(np.uint32))


def test_corrupt_cold_record_surfaces(hs):
    """A damaged cold record in the chain is reported by the fetch status
    (the reference's fetch throws), not consumed silently."""
    g = rng(4471)
    n = 4096
    k, rows, slot, hot = _sequence(g, n, 4471)
    image = _image(hs, rows, 31)
    cold = np.nonzero(slot < 0)[0]
    raw = image.numpy()
    victim = int(cold[17])
    raw[4096 + victim * 4128 + 32 + 777] ^= 0x10  # a payload byte of a cold row
    pos = torch.from_numpy(cold.astype(np.int32)).cuda()
    staging = torch.zeros((cold.size, 4096), dtype=torch.uint8, device="cuda")
    status = hs.ops.kv_cold_fetch(image, 0, pos, staging)
    st = hs.ops.read_status(status)
    assert st["code"] == hs.HS_ERR_CORRUPT and st["k"] == 1


@pytest.mark.parametrize("current_cold", [False, True])
def test_cover_prefetch_then_misses(hs, port, current_cold):
    """The payload prefetch of the reference's executor on the device
    (prefetch_payload, policy/full_gqa_runtime.cpp:299-344, consumed at
    runtime/gqa_executor.cpp:202-221): before the current token exists, the
    history cover's cold rows are fetched on a side stream; after the final
    selection (which completes the current token), only the selected cold
    rows outside the cover are fetched, on the main stream.  Attention then
    reads hot rows, cover rows and miss rows through one row map.

    The current token's K row copies the history's best head-0 key, so it is
    selected; when its row is cold it is the one miss (the cover holds
    history only), else there is none.  Checks: the final ids equal the
    oracle's one-shot selection over all n columns; the cover fetched exactly
    its cold union; the misses are exactly the selected cold rows outside it;
    the attention equals the all-hot attention bit for bit and is within
    2e-3 of the FP64 oracle."""
    n = 4096
    g = rng(8100 + current_cold)
    k, rows, slot, hot = _sequence(g, n, 8200 + current_cold)
    q16 = f16_bits(g.standard_normal((32, 128)))
    hist_raw = port.score(q16, rows[: n - 1].reshape(-1), n - 1, 2048)
    best = int(np.argmax(hist_raw[0].view(np.float16).astype(np.float32)))
    k = k.copy()
    k[n - 1] = k[best]
    rows = pool_rows(k, rows.reshape(n, 2, 8, 128)[:, 1].reshape(n, 8, 128))
    if current_cold != (slot[n - 1] < 0):  # place the current token's row as asked
        b = (n - 1) // 64
        if current_cold:
            slot[b * 64:] = -1
        else:
            slot[b * 64:] = np.arange(hot.size, hot.size + n - b * 64, dtype=np.int32)
        hot = np.nonzero(slot >= 0)[0]
        order = np.argsort(slot[hot])
        hot = hot[order]
    hot_rows, cold_tokens = hot.size, n - hot.size
    q32 = g.standard_normal((32, 128)).astype(np.float32)
    image = _image(hs, rows, 71)
    pool = torch.zeros((hot_rows + 2 * cold_tokens, 2048), dtype=torch.float16, device="cuda")
    pool[:hot_rows] = to_dev(rows[hot])
    keys = to_dev(k.reshape(-1))
    slot_d = to_dev(slot)
    side = torch.cuda.Stream()
    main = torch.cuda.current_stream()
    # one layer early: the history (n - 1 columns), its cover, the cover's cold plan and fetch
    scores = torch.empty((32, n), dtype=torch.float16, device="cuda")
    part = torch.empty((n - 1 + 63) // 64, dtype=torch.int32, device="cuda")
    hs.ops.score(to_dev(q16.reshape(-1)), keys, n - 1, out=scores, score_stride=n,
                 head0_partial=part)
    words_h = (n - 1 + 31) // 32
    cover_member = torch.zeros((32, words_h), dtype=torch.int32, device="cuda")
    _, _, _, cst = hs.ops.select(scores, 32, n, n - 1, ALPHA, RATIO, scale_raw=True, cover=True,
                                 head0_partial=part, member=cover_member)
    cover_rows = torch.empty(n, dtype=torch.int32, device="cuda")
    cover_pos, _, cover_count = hs.ops.cold_plan(cover_member, 32, n - 1, slot_d, hot_rows,
                                                 cold_tokens, rows=cover_rows)
    cover_rows[n - 1:] = slot_d[n - 1:]  # the current token's own slot (hot or -1)
    fetched = torch.cuda.Event()
    fetched_from = main.record_event()
    with torch.cuda.stream(side):
        side.wait_event(fetched_from)
        cover_status = hs.ops.kv_cold_fetch(image, 0, cover_pos,
                                            pool[hot_rows: hot_rows + cold_tokens], stream=side)
        fetched.record(side)
    # the final selection: the current token completed, every column
    words = (n + 31) // 32
    member = torch.zeros((32, words), dtype=torch.int32, device="cuda")
    sel = hs.ops.select_batched(
        [dict(scores=scores, n=n, head0_partial=part, member=member,
              current_q=to_dev(q16.reshape(-1)), current_key=keys[(n - 1) * 1024:])],
        32, ALPHA, RATIO, scale_raw=True, id_order=True, require_k=True)
    ids, _, _, status = sel[0]
    miss_pos, final_rows, miss_count = hs.ops.cold_plan(member, 32, n, cover_rows,
                                                        hot_rows + cold_tokens, cold_tokens)
    miss_status = hs.ops.kv_cold_fetch(image, 0, miss_pos, pool[hot_rows + cold_tokens:])
    main.wait_event(fetched)
    q = torch.from_numpy(q32).cuda()
    out = hs.ops.sparse_attention(q, pool.reshape(-1), n, member, rows=final_rows)
    torch.cuda.synchronize()
    st = hs.ops.read_status(status)
    assert hs.ops.read_status(cst)["code"] == 0 and st["code"] == 0
    assert hs.ops.read_status(cover_status)["code"] == 0
    assert hs.ops.read_status(miss_status)["code"] == 0
    # final selection = the oracle's one-shot selection over all n columns
    raw = port.score(q16, rows.reshape(-1), n, 2048)
    assert np.array_equal(from_dev(scores), raw)
    rc, kk, pids, _, _ = port.select(port.scale(raw), 32, n, n, ALPHA, RATIO)
    assert rc == 0 and st["k"] == kk
    assert np.array_equal(from_dev(ids)[:, :kk], np.sort(pids, axis=1))
    # the cover fetched its cold union; the misses are the selected cold rows outside it
    cbits = from_dev(cover_member).view(np.uint32)
    cover_union = np.nonzero(np.unpackbits(np.bitwise_or.reduce(cbits, axis=0).view(np.uint8),
                                           bitorder="little")[: n - 1])[0]
    cover_cold = cover_union[slot[cover_union] < 0]
    assert int(cover_count.item()) == cover_cold.size
    assert np.array_equal(from_dev(cover_pos)[: cover_cold.size], cover_cold)
    selected = np.unique(np.concatenate([np.asarray(p) for p in pids]))
    misses = np.setdiff1d(selected[slot[selected] < 0], cover_cold)
    assert int(miss_count.item()) == misses.size
    assert np.array_equal(from_dev(miss_pos)[: misses.size], misses)
    assert misses.size == (1 if current_cold else 0) and (not current_cold or misses[0] == n - 1)
    # attention through hot + cover + miss rows = the all-hot attention, bit for bit
    ref_dev = hs.ops.sparse_attention(q, to_dev(rows.reshape(-1)), n, member)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref_dev.cpu().numpy().view(np.uint32))
    ref = port.attention(q32, rows.view(np.uint8).reshape(-1), list(pids))
    err = np.max(np.linalg.norm(got.astype(np.float64) - ref, axis=1) / np.linalg.norm(ref, axis=1))
    assert err <= TOL, err
