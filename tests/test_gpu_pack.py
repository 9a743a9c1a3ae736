"""GPU parity of kernel #3 (union, pack, row-map gather): byte-exact."""
import numpy as np
import pytest
import torch

from hs_data import from_dev, rng, to_dev
from test_oracle_pack import kat_payload, random_trial

pytestmark = pytest.mark.gpu


def dev_ids(selected):
    stride = max(1, max(len(r) for r in selected))
    ids = np.zeros((32, stride), dtype=np.uint32)
    lens = np.zeros(32, dtype=np.uint32)
    for h, r in enumerate(selected):
        ids[h, : len(r)] = r
        lens[h] = len(r)
    return to_dev(ids), to_dev(lens), stride


def gpu_pack(hs, selected, queries, physical, payload, count, extra_rows=0, split=False):
    ids, lens, stride = dev_ids(selected)
    row_of_id = np.full(max(int(np.max(physical)) + 1, 1) + extra_rows, -1, dtype=np.int32)
    row_of_id[np.asarray(physical, dtype=np.int64)] = np.arange(len(physical), dtype=np.int32)
    pos = torch.tensor(np.asarray(queries, dtype=np.uint64).view(np.int64), device="cuda")
    records = np.ascontiguousarray(payload, dtype=np.uint8).reshape(-1, 4096)
    if split:  # the hot pool as a K array and a V array of 2048 B rows
        kp = torch.from_numpy(np.ascontiguousarray(records[:, :2048])).cuda()
        vp = torch.from_numpy(np.ascontiguousarray(records[:, 2048:])).cuda()
        k, v, mask, status = hs.ops.pack(kp, ids, lens, stride, pos, count,
                                         row_of_id=to_dev(row_of_id), v_pool=vp, row_bytes=2048)
    else:
        pool = torch.from_numpy(records).cuda()
        k, v, mask, status = hs.ops.pack(pool, ids, lens, stride, pos, count,
                                         row_of_id=to_dev(row_of_id))
    st = hs.ops.read_status(status)
    return st, from_dev(k), from_dev(v), mask.cpu().numpy()


def test_pack_known_values(hs, port):
    ids = [[8, 12] for _ in range(32)]
    ids[4] = [12, 8]
    st, k, v, mask = gpu_pack(hs, ids, [10, 12], [8, 12], kat_payload(), 32)
    rc, pk, pv, pmask = port.pack(ids, [10, 12], [8, 12], kat_payload(), 32)
    assert st["code"] == 0 and rc == 0
    assert np.array_equal(k, pk) and np.array_equal(v, pv)
    assert np.array_equal(mask.view(np.uint32), pmask.view(np.uint32))
    bad = [list(r) for r in ids]
    bad[0] = [13]
    assert gpu_pack(hs, bad, [12], [8, 12], kat_payload(), 32)[0]["code"] == hs.HS_ERR_MISSING


@pytest.mark.parametrize("trial", range(0, 48, 3))
def test_pack_random(hs, port, trial):
    g = rng(781 + trial)
    n, slots, rows, payload, selected, queries = random_trial(g, trial)
    # every other trial reads a hot pool of separate K and V arrays
    st, k, v, mask = gpu_pack(hs, selected, queries, rows, payload, slots, split=trial % 2 == 1)
    rc, pk, pv, pmask = port.pack(selected, queries, rows, payload, slots)
    assert st["code"] == 0 and rc == 0
    assert np.array_equal(k, pk) and np.array_equal(v, pv)
    assert np.array_equal(mask.view(np.uint32), pmask.view(np.uint32))


def test_pack_many_queries_and_slack_slots(hs, port):
    g = rng(55)
    n = 500
    rows = g.permutation(n).astype(np.uint32)
    payload = g.integers(0, 256, size=n * 4096, dtype=np.uint8)
    selected = [np.sort(g.choice(n, size=int(g.integers(1, 200)), replace=False)) for _ in range(32)]
    queries = sorted(g.choice(n, size=70, replace=False).tolist())
    queries[-1] = n - 1
    st, k, v, mask = gpu_pack(hs, selected, queries, rows, payload, 224)
    rc, pk, pv, pmask = port.pack(selected, queries, rows, payload, 224)
    assert st["code"] == 0 and rc == 0
    assert np.array_equal(k, pk) and np.array_equal(v, pv)
    assert np.array_equal(mask.view(np.uint32), pmask.view(np.uint32))


@pytest.mark.parametrize("trial", range(0, 48, 7))
def test_union_random(hs, port, trial):
    g = rng(900 + trial)
    n, slots, rows, payload, selected, queries = random_trial(g, trial)
    ids, lens, stride = dev_ids(selected)
    out, out_n, status = hs.ops.physical_union(ids, lens, stride, n)
    st = hs.ops.read_status(status)
    m = int(out_n.item())
    assert st["code"] == 0
    assert np.array_equal(from_dev(out)[:m], port.physical_union(selected, n)[1])
    dup = [list(r) for r in selected]
    dup[31].append(dup[31][0])
    ids, lens, stride = dev_ids(dup)
    _, _, status = hs.ops.physical_union(ids, lens, stride, n)
    assert hs.ops.read_status(status)["code"] == hs.HS_ERR_DUPLICATE


def test_gather_rows(hs, port):
    g = rng(4242)
    n, slots, rows, payload, selected, queries = random_trial(g, 7)
    pre_rows = [int(x) for x in rows[: n // 2]]
    miss_rows = [int(x) for x in rows[n // 2:]]
    where = {int(id_): i for i, id_ in enumerate(rows)}
    pre = np.concatenate([payload[where[i] * 4096:(where[i] + 1) * 4096] for i in pre_rows])
    mis = np.concatenate([payload[where[i] * 4096:(where[i] + 1) * 4096] for i in miss_rows])
    row_map = np.full(32 * slots, -1, dtype=np.int32)
    for h in range(32):
        for s, id_ in enumerate(selected[h]):
            id_ = int(id_)
            row_map[h * slots + s] = (pre_rows.index(id_) if id_ in set(pre_rows)
                                      else -2 - miss_rows.index(id_))
    k, v, status = hs.ops.gather_rows(torch.from_numpy(pre).cuda(), torch.from_numpy(mis).cuda(),
                                      to_dev(row_map), slots)
    pk, pv = port.gather_rows(pre.view(np.uint16), mis.view(np.uint16), row_map, slots)
    assert hs.ops.read_status(status)["code"] == 0
    assert np.array_equal(from_dev(k), pk) and np.array_equal(from_dev(v), pv)
    row_map[5] = len(pre_rows)  # beyond the prefetched payload
    _, _, status = hs.ops.gather_rows(torch.from_numpy(pre).cuda(), torch.from_numpy(mis).cuda(),
                                      to_dev(row_map), slots)
    assert hs.ops.read_status(status)["code"] == hs.HS_ERR_MISSING


@pytest.mark.parametrize("queries", [1, 64])
def test_pack_and_gather_at_layer_size(hs, port, queries):
    """configs[2] size: N = 32768 hot rows, k = 6553 ids per head (the cap at
    ratio 0.2), sparse_slots = 6560, with 1 and 64 query positions.  K, V and
    the F32 mask equal the oracle byte for byte; the row-map gather over the
    same selection (half the rows prefetched, half misses) too."""
    n, k, slots = 32768, 6553, 6560
    g = rng(6553 + queries)
    payload = g.integers(0, 256, size=n * 4096, dtype=np.uint8)
    selected = [np.sort(g.choice(n, size=k, replace=False)) for _ in range(32)]
    qpos = sorted(g.choice(n, size=queries, replace=False).tolist())
    qpos[-1] = n - 1
    rows = np.arange(n, dtype=np.uint32)
    st, kd, vd, mask = gpu_pack(hs, selected, qpos, rows, payload, slots, split=queries == 64)
    rc, pk, pv, pmask = port.pack(selected, qpos, rows, payload, slots)
    assert st["code"] == 0 and rc == 0
    assert np.array_equal(kd, pk) and np.array_equal(vd, pv)
    assert np.array_equal(mask.view(np.uint32), pmask.view(np.uint32))
    del kd, vd, mask, pk, pv, pmask
    # gather: even ids prefetched (row id / 2), odd ids misses (row id // 2)
    rec = payload.reshape(n, 4096)
    pre, mis = np.ascontiguousarray(rec[0::2]), np.ascontiguousarray(rec[1::2])
    row_map = np.full((32, slots), -1, dtype=np.int32)
    for h in range(32):
        s = selected[h].astype(np.int64)
        row_map[h, : len(s)] = np.where(s % 2 == 0, s // 2, -2 - s // 2)
    kd, vd, status = hs.ops.gather_rows(torch.from_numpy(pre.reshape(-1)).cuda(),
                                        torch.from_numpy(mis.reshape(-1)).cuda(),
                                        to_dev(row_map.reshape(-1)), slots)
    gk, gv = port.gather_rows(pre.view(np.uint16), mis.view(np.uint16), row_map.reshape(-1), slots)
    assert hs.ops.read_status(status)["code"] == 0
    assert np.array_equal(from_dev(kd), gk) and np.array_equal(from_dev(vd), gv)


def test_status_needs_no_clearing(hs, port):
    """Pack and gather stamp their status themselves: a status holding a stale
    error (or another call's stamp) reads HS_OK after a clean call, an error
    after a failing one, and HS_OK again after the next clean call."""
    ids = [[8, 12] for _ in range(32)]
    bad = [list(r) for r in ids]
    bad[0] = [13]
    stale = np.array([hs.HS_ERR_MISSING, np.int32(-2147483643), 5, 6], dtype=np.int32)
    status = torch.from_numpy(stale.copy()).cuda()

    def run(sel):
        dids, lens, stride = dev_ids(sel)
        row_of_id = np.full(13, -1, dtype=np.int32)
        row_of_id[[8, 12]] = [0, 1]
        pos = torch.tensor([12], dtype=torch.int64, device="cuda")
        pool = torch.from_numpy(kat_payload().reshape(-1, 4096)).cuda()
        hs.ops.pack(pool, dids, lens, stride, pos, 32, row_of_id=to_dev(row_of_id), status=status)
        return hs.ops.read_status(status)["code"]

    assert run(ids) == 0
    assert run(bad) == hs.HS_ERR_MISSING
    assert run(ids) == 0
    status.copy_(torch.from_numpy(stale))
    pre = torch.from_numpy(kat_payload()).cuda()
    row_map = np.full(32 * 32, -1, dtype=np.int32)
    row_map[::32] = 0
    _, _, st = hs.ops.gather_rows(pre, None, to_dev(row_map), 32, status=status)
    assert hs.ops.read_status(st)["code"] == 0
    row_map[5] = 3  # beyond the two prefetched rows
    _, _, st = hs.ops.gather_rows(pre, None, to_dev(row_map), 32, status=status)
    assert hs.ops.read_status(st)["code"] == hs.HS_ERR_MISSING
