"""Pins of union / pack / row-map gather restatements (oracle, CPU).

Known values are those of tests/gqa_pack_tests.cpp:6-16; random trials are
checked against the compiled reference pack_gqa_workspace and
gqa_physical_union (tests/gqa_pack_tests.cpp:17-41 style).
"""
import numpy as np
import pytest

from hs_data import rng


def kat_payload():
    raw = np.zeros(4096, dtype=np.uint16)
    for t in range(2):
        for h in range(8):
            for d in range(128):
                raw[t * 2048 + h * 128 + d] = 1000 * t + 100 * h + d
                raw[t * 2048 + 1024 + h * 128 + d] = 5000 + 1000 * t + 100 * h + d
    return raw.view(np.uint8)


def test_pack_known_values(port):
    ids = [[8, 12] for _ in range(32)]
    ids[4] = [12, 8]
    rc, k, v, mask = port.pack(ids, [10, 12], [8, 12], kat_payload(), 32)
    assert rc == 0
    assert k[0] == 0 and k[4096] == 1000 and k[4 * 128] == 1100 and k[4096 + 4 * 128] == 100
    assert v[(4 * 128) * 32] == 6100 and v[(4 * 128) * 32 + 1] == 5100
    assert k[2 * 4096 + 127] == 0 and v[127 * 32 + 2] == 0
    assert mask[0] == 0 and np.isinf(mask[1]) and mask[32 + 1] == 0
    assert np.isinf(mask[(4 * 64) * 32]) and mask[(4 * 64) * 32 + 1] == 0
    assert np.isinf(mask[2 * 32])
    bad = [list(r) for r in ids]
    bad[0] = [13]
    assert port.pack(bad, [12], [8, 12], kat_payload(), 32)[0] != 0


def random_trial(g, trial):
    n = 65 + trial * 4
    slots = (n + 31) // 32 * 32
    rows = g.permutation(n).astype(np.uint32)
    payload = g.integers(0, 256, size=n * 4096, dtype=np.uint8)
    selected = []
    for _ in range(32):
        head = rows.copy()
        if trial % 2:
            head = head[: 1 + g.integers(0, n)]
        selected.append(g.permutation(head))
    queries = [n // 2, n - 1]
    return n, slots, rows, payload, selected, queries


@pytest.mark.parametrize("trial", range(0, 48, 5))
def test_pack_matches_reference(port, ref, trial):
    g = rng(781 + trial)
    n, slots, rows, payload, selected, queries = random_trial(g, trial)
    a = port.pack(selected, queries, rows, payload, slots)
    b = ref.pack(selected, queries, rows, payload, slots)
    assert a[0] == 0 and b[0] == 0
    for x, y in zip(a[1:], b[1:]):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


@pytest.mark.parametrize("trial", range(0, 48, 7))
def test_union_matches_reference(port, ref, trial):
    g = rng(900 + trial)
    n, slots, rows, payload, selected, queries = random_trial(g, trial)
    a = port.physical_union(selected, n)
    b = ref.physical_union(selected, n)
    assert a[0] == 0 and b[0] == 0 and np.array_equal(a[1], b[1])
    expected = np.unique(np.concatenate(selected))
    assert np.array_equal(a[1], expected)
    dup = [list(r) for r in selected]
    dup[31].append(dup[31][0])
    assert port.physical_union(dup, n)[0] != 0 and ref.physical_union(dup, n)[0] != 0
    future = [list(r) for r in selected]
    future[3].append(n)
    assert port.physical_union(future, n)[0] != 0


def test_gather_rows_equals_pack(port):
    # runtime/gqa_executor.cpp:202-217: the row-map delivery and the host pack
    # produce the same K/V for the same selection.
    g = rng(4242)
    n, slots, rows, payload, selected, queries = random_trial(g, 7)
    rc, k, v, _ = port.pack(selected, queries, rows, payload, slots)
    assert rc == 0
    where = {int(id_): i for i, id_ in enumerate(rows)}
    prefetched_ids = set(int(x) for x in rows[: n // 2])
    pre_rows = [int(x) for x in rows[: n // 2]]
    miss_rows = [int(x) for x in rows[n // 2:]]
    pre = np.concatenate([payload[where[i] * 4096:(where[i] + 1) * 4096] for i in pre_rows])
    mis = np.concatenate([payload[where[i] * 4096:(where[i] + 1) * 4096] for i in miss_rows])
    row_map = np.full(32 * slots, -1, dtype=np.int32)
    for h in range(32):
        for s, id_ in enumerate(selected[h]):
            id_ = int(id_)
            row_map[h * slots + s] = (pre_rows.index(id_) if id_ in prefetched_ids
                                      else -2 - miss_rows.index(id_))
    gk, gv = port.gather_rows(pre.view(np.uint16), mis.view(np.uint16), row_map, slots)
    assert np.array_equal(gk, k) and np.array_equal(gv, v)
