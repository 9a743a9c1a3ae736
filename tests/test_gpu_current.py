"""Current-token completion (policy/full_gqa_runtime.cpp:531-572): the
history (columns < n - 1) is scored early, e.g. one layer ahead, and the
selection's first launch scores column n - 1 (the token just appended) from
the query and that token's K row, then selects over all n columns.

Bar: bit-exact against the same selection over one-shot scores of all n
columns (scores, ids, counts, k, tied heads, status), and against the
oracle; per-head path, slice path, without the scorer's tile maxima, the
current token as the new head-0 maximum, and inside select-then-score."""
import ctypes

import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, rng, rope_keys, to_dev

pytestmark = pytest.mark.gpu
ALPHA, RATIO = 5.0, 0.2


def _inputs(n, seed, peak=False):
    g = rng(seed)
    k = rope_keys(n, seed)
    q = f16_bits(g.standard_normal((32, 128)))
    if peak:
        # the appended token aligned with head 0's query: its head-0 score is
        # far above every history score, so the threshold moves with it
        k = k.copy()
        k[n - 1, 0] = q[0]
    return q, k


def _one_shot(hs, q, k, n, id_order, alpha=ALPHA):
    qd, kd = to_dev(q.reshape(-1)), to_dev(k.reshape(-1))
    part = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    raw = hs.ops.score(qd, kd, n, head0_partial=part)
    ids, counts, member, status = hs.ops.select(raw, 32, n, n, alpha, RATIO, scale_raw=True,
                                                id_order=id_order, head0_partial=part)
    return raw, ids, counts, hs.ops.read_status(status)


def _completed(hs, q, k, n, id_order, with_partial=True, alpha=ALPHA):
    qd, kd = to_dev(q.reshape(-1)), to_dev(k.reshape(-1))
    raw = torch.full((32, n), float("nan"), dtype=torch.float16, device="cuda")  # column n-1 junk
    part = None
    if n > 1:
        part = torch.empty((n - 1 + 63) // 64, dtype=torch.int32, device="cuda")
        hs.ops.score(qd, kd, n - 1, out=raw, score_stride=n, head0_partial=part)
    cur_key = to_dev(k[n - 1].reshape(-1))
    job = dict(scores=raw, n=n, current_q=qd, current_key=cur_key)
    if with_partial and part is not None:
        job["head0_partial"] = part
    (ids, counts, member, status), = hs.ops.select_batched([job], 32, alpha, RATIO,
                                                          scale_raw=True, id_order=id_order)
    return raw, ids, counts, hs.ops.read_status(status)


@pytest.mark.parametrize("n,peak", [(4096, False), (4096, True), (32768, False), (40000, False),
                                    (40000, True), (65, False), (5, True)])
@pytest.mark.parametrize("id_order", [False, True])
def test_history_plus_current_equals_one_shot(hs, port, n, peak, id_order):
    q, k = _inputs(n, 500 + n, peak)
    want = _one_shot(hs, q, k, n, id_order)
    got = _completed(hs, q, k, n, id_order)
    assert np.array_equal(from_dev(got[0]), from_dev(want[0])), "scores differ"
    assert got[3] == want[3], (got[3], want[3])
    kk = want[3]["k"]
    assert np.array_equal(from_dev(got[1])[:, :kk], from_dev(want[1])[:, :kk])
    assert np.array_equal(from_dev(got[2]), from_dev(want[2]))
    # and the oracle over all n columns
    raw = port.score(q, k.reshape(-1), n)
    assert np.array_equal(from_dev(got[0]), raw)
    rc, ok, pids, pcounts, tied = port.select(port.scale(raw), 32, n, n, ALPHA, RATIO)
    assert rc == 0 and ok == kk and tied == got[3]["boundary_tied_heads"]
    ref_ids = np.sort(pids, axis=1) if id_order else pids
    assert np.array_equal(from_dev(got[1])[:, :kk], ref_ids)
    if peak:  # the current token moved the head-0 maximum
        assert got[3]["head0_max_key"] == port.order_key(int(raw[0, n - 1]))


def test_without_tile_maxima(hs):
    n = 4096
    q, k = _inputs(n, 77, peak=True)
    want = _one_shot(hs, q, k, n, False)
    got = _completed(hs, q, k, n, False, with_partial=False)
    assert np.array_equal(from_dev(got[0]), from_dev(want[0]))
    assert got[3] == want[3]
    kk = want[3]["k"]
    assert np.array_equal(from_dev(got[1])[:, :kk], from_dev(want[1])[:, :kk])
    # a smaller margin keeps a nonempty selection with the peaked token
    want = _one_shot(hs, q, k, n, False, alpha=12.0)
    got = _completed(hs, q, k, n, False, with_partial=False, alpha=12.0)
    kk = want[3]["k"]
    assert kk > 0 and got[3] == want[3]
    assert np.array_equal(from_dev(got[1])[:, :kk], from_dev(want[1])[:, :kk])


def test_nonfinite_current_score_rejected(hs):
    n = 2048
    q, k = _inputs(n, 91)
    k = k.copy()
    k[n - 1, 3, 5] = 0x7C00  # +inf in KV head 3: query heads 12..15 score nonfinite
    got = _completed(hs, q, k, n, True)
    assert got[3]["code"] == hs.HS_ERR_NONFINITE


def test_in_select_then_score(hs, port):
    """The pipelined schedule a decode can run: layer l's selection completes
    its current token while layer l+1's history (n - 1 columns) is scored."""
    n = 32768
    q, k = _inputs(n, 4321)
    q2 = f16_bits(rng(4322).standard_normal((32, 128)))
    k2 = rope_keys(n, 4323)
    qd, kd = to_dev(q.reshape(-1)), to_dev(k.reshape(-1))
    raw = torch.empty((32, n), dtype=torch.float16, device="cuda")
    part = torch.empty((n - 1 + 63) // 64, dtype=torch.int32, device="cuda")
    hs.ops.score(qd, kd, n - 1, out=raw, score_stride=n, head0_partial=part)
    kk_max = int(np.floor(n * np.float32(RATIO)))
    ids = torch.empty((32, kk_max), dtype=torch.int32, device="cuda")
    status = hs.ops.new_status()
    ws = hs.ops.workspace(hs.ops.select_workspace_bytes(32, n))
    raw2 = torch.empty((32, n), dtype=torch.float16, device="cuda")
    part2 = torch.empty((n - 1 + 63) // 64, dtype=torch.int32, device="cuda")
    hs.ops.select_then_score(
        [dict(scores=raw, n=n, head0_partial=part, ids=ids, status=status, ws=ws,
              current_q=qd, current_key=to_dev(k[n - 1].reshape(-1)))],
        [dict(q16=to_dev(q2.reshape(-1)), keys=to_dev(k2.reshape(-1)), tokens=n - 1, out=raw2,
              score_stride=n, head0_partial=part2)],
        32, ALPHA, RATIO, scale_raw=True)
    st = hs.ops.read_status(status)
    full = port.score(q, k.reshape(-1), n)
    assert np.array_equal(from_dev(raw), full)
    rc, ok, pids, _, tied = port.select(port.scale(full), 32, n, n, ALPHA, RATIO)
    assert st["code"] == 0 and st["k"] == ok and st["boundary_tied_heads"] == tied
    assert np.array_equal(from_dev(ids)[:, :ok], pids)
    hist2 = port.score(q2, k2.reshape(-1), n - 1)
    assert np.array_equal(from_dev(raw2)[:, : n - 1], hist2)


def test_rejections(hs):
    L = hs.lib()
    n = 256
    dev = lambda shape, dt=torch.int32: torch.zeros(shape, dtype=dt, device="cuda")
    scores, ids = dev((32, n), torch.float16), dev((32, 64))
    status, ws = hs.ops.new_status(), hs.ops.workspace(hs.ops.select_workspace_bytes(32, n))
    q, key = dev(4096, torch.float16), dev(1024, torch.float16)
    vp = lambda t: None if t is None else t.data_ptr()

    def job(cq, ck):
        return hs.SelectJob(vp(scores), None, vp(ids), None, None, vp(status), vp(ws), n, n, 64, 0,
                            vp(cq), vp(ck))

    def call(j, heads=32, flags=0):
        table = (hs.SelectJob * 1)(j)
        return L.hs_gqa_select_batched(ctypes.cast(table, ctypes.c_void_p), 1, heads, ALPHA, RATIO,
                                       flags, None)

    assert call(job(q, None)) == hs.HS_ERR_ARGUMENT
    assert call(job(None, key)) == hs.HS_ERR_ARGUMENT
    assert call(job(q, key), heads=16) == hs.HS_ERR_ARGUMENT
    assert call(job(q, key), flags=hs.HS_SELECT_COVER) == hs.HS_ERR_ARGUMENT
