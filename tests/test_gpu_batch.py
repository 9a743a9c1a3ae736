"""Batched scoring and selection (the decode sequences of a batch, configs[3]):
every job of a batched launch equals the single-call result bit for bit
(the single-call paths are pinned to the oracle elsewhere), and one small
job is checked against the oracle directly."""
import numpy as np
import pytest
import torch

from hs_data import batch_ns, from_dev, make_jobs, rng, v3_sample

pytestmark = pytest.mark.gpu


def test_batched_scores_match_single_calls(hs):
    ns = batch_ns(3)
    jobs = make_jobs(hs, ns, 1000)
    outs = hs.ops.score_batched(jobs)
    for j, out in zip(jobs, outs):
        part = torch.empty_like(j["head0_partial"])
        single = hs.ops.score(j["q16"], j["keys"], j["tokens"], head0_partial=part)
        assert torch.equal(out, single)
        assert torch.equal(j["head0_partial"], part)


def test_batched_score_against_oracle(hs, port):
    g = rng(11)
    n0, n1 = 192, 4096
    q0, k0 = v3_sample(g, 4096), v3_sample(g, n0 * 1024)
    q1, k1 = v3_sample(g, 4096), v3_sample(g, n1 * 1024)
    dev = lambda a: torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    outs = hs.ops.score_batched([dict(q16=dev(q0), keys=dev(k0), tokens=n0),
                                 dict(q16=dev(q1), keys=dev(k1), tokens=n1)])
    assert np.array_equal(from_dev(outs[0]), port.score(q0, k0, n0))
    assert np.array_equal(from_dev(outs[1]), port.score(q1, k1, n1))


@pytest.mark.parametrize("id_order", [False, True])
@pytest.mark.parametrize("use_partial", [True, False])
def test_batched_select_matches_single_calls(hs, id_order, use_partial):
    ns = batch_ns(5 + id_order)
    jobs = make_jobs(hs, ns, 2000)
    outs = hs.ops.score_batched(jobs)
    sel_jobs = []
    for j, out in zip(jobs, outs):
        words = (j["tokens"] + 31) // 32
        sel_jobs.append(dict(scores=out, n=j["tokens"],
                             head0_partial=j["head0_partial"] if use_partial else None,
                             member=torch.zeros((32, words), dtype=torch.int32, device="cuda")))
    res = hs.ops.select_batched(sel_jobs, 32, 5.0, 0.2, scale_raw=True, id_order=id_order)
    for sj, (ids, counts, member, status) in zip(sel_jobs, res):
        st = hs.ops.read_status(status)
        words = (sj["n"] + 31) // 32
        m1 = torch.zeros((32, words), dtype=torch.int32, device="cuda")
        ids1, counts1, _, status1 = hs.ops.select(sj["scores"], 32, sj["n"], sj["n"], 5.0, 0.2,
                                                  scale_raw=True, id_order=id_order, member=m1)
        st1 = hs.ops.read_status(status1)
        assert st == st1
        k = st["k"]
        assert torch.equal(ids[:, :k], ids1[:, :k])
        assert torch.equal(counts, counts1)
        assert torch.equal(member, m1)


def test_batched_select_mixed_sizes_and_cover(hs):
    # one job beyond the per-head limit: the batch runs job by job
    ns = [4096, 40000, 12288]
    jobs = make_jobs(hs, ns, 3000)
    outs = [hs.ops.score(j["q16"], j["keys"], j["tokens"]) for j in jobs]
    for cover in (False, True):
        res = hs.ops.select_batched([dict(scores=o, n=n) for o, n in zip(outs, ns)], 32, 2.0,
                                    0.2, scale_raw=True, cover=cover)
        for o, n, (ids, counts, _, status) in zip(outs, ns, res):
            ids1, counts1, _, status1 = hs.ops.select(o, 32, n, n, 2.0, 0.2, scale_raw=True,
                                                      cover=cover)
            st, st1 = hs.ops.read_status(status), hs.ops.read_status(status1)
            assert st == st1 and st["code"] == 0
            assert torch.equal(ids[:, : st["k"]], ids1[:, : st["k"]])
            assert torch.equal(counts, counts1)


# Sizes of a batch with more (head, slice) pairs than one round of count
# groups (> 1024): with every score row 16-byte aligned (a stride that is a
# multiple of 8) the count launch covers 4 slices per workgroup.  Ragged
# sizes leave groups with 1..3 slices and slices with partial runs.
WIDE_NS = [32768, 30001, 4097, 4096, 12289, 20000, 8229, 28672, 16384, 9999, 31000, 24576,
           17000, 6000, 32767, 25000]


def _wide_stride(n):
    return -(-n // 8) * 8


def _single_select(hs, sj, id_order):
    words = (sj["n"] + 31) // 32
    m1 = torch.zeros((32, words), dtype=torch.int32, device="cuda")
    ids1, counts1, _, status1 = hs.ops.select(sj["scores"], 32, sj["scores"].shape[-1], sj["n"],
                                              5.0, 0.2, scale_raw=True, id_order=id_order,
                                              member=m1, head0_partial=sj.get("head0_partial"))
    return ids1, counts1, m1, hs.ops.read_status(status1)


@pytest.mark.parametrize("id_order", [False, True])
def test_wide_count_batch_matches_single_calls(hs, id_order):
    assert sum(32 * -(-n // 4096) for n in WIDE_NS) > 1024
    jobs = make_jobs(hs, WIDE_NS, 4000)
    for j in jobs:
        j["score_stride"] = _wide_stride(j["tokens"])
    outs = hs.ops.score_batched(jobs)
    # nonfinite scores in the third and fourth slice of a count group, and in
    # head 0 of another job: those jobs fail as the single calls do
    outs[5][7, 3 * 4096 + 17] = float("nan")
    outs[10][0, 6 * 4096 + 5] = float("inf")
    outs[2][31, 4096] = float("-inf")  # n = 4097: the group's second slice holds one id
    sel_jobs = []
    for j, out in zip(jobs, outs):
        words = (j["tokens"] + 31) // 32
        sel_jobs.append(dict(scores=out, n=j["tokens"], head0_partial=j["head0_partial"],
                             member=torch.zeros((32, words), dtype=torch.int32, device="cuda")))
    res = hs.ops.select_batched(sel_jobs, 32, 5.0, 0.2, scale_raw=True, id_order=id_order)
    codes = []
    for sj, (ids, counts, member, status) in zip(sel_jobs, res):
        st = hs.ops.read_status(status)
        ids1, counts1, m1, st1 = _single_select(hs, sj, id_order)
        assert st == st1
        codes.append(st["code"])
        if st["code"] != 0:
            continue
        k = st["k"]
        assert torch.equal(ids[:, :k], ids1[:, :k])
        assert torch.equal(counts, counts1)
        assert torch.equal(member, m1)
    assert codes[5] == codes[10] == codes[2] == hs.HS_ERR_NONFINITE
    assert codes.count(0) == len(WIDE_NS) - 3


def test_wide_count_batch_with_current_tokens(hs):
    # history (n - 1 columns) scored early, every job completing its current
    # token in the wide count launch: equal to one-shot scoring over n
    jobs = make_jobs(hs, WIDE_NS, 4100)
    sel_jobs, wants = [], []
    for j in jobs:
        n = j["tokens"]
        full = torch.empty((32, n), dtype=torch.float16, device="cuda")
        part_full = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
        hs.ops.score(j["q16"], j["keys"], n, out=full, head0_partial=part_full)
        wants.append((full, _single_select(hs, dict(scores=full, n=n, head0_partial=part_full),
                                           False)))
        stride = _wide_stride(n)
        raw = torch.full((32, stride), float("nan"), dtype=torch.float16, device="cuda")
        part = torch.empty((n - 1 + 63) // 64, dtype=torch.int32, device="cuda")
        hs.ops.score(j["q16"], j["keys"], n - 1, out=raw, score_stride=stride, head0_partial=part)
        sel_jobs.append(dict(scores=raw, n=n, head0_partial=part, current_q=j["q16"],
                             current_key=j["keys"][(n - 1) * 1024:]))
    res = hs.ops.select_batched(sel_jobs, 32, 5.0, 0.2, scale_raw=True)
    for sj, (ids, counts, _, status), (full, (ids1, counts1, _, st1)) in zip(sel_jobs, res, wants):
        st = hs.ops.read_status(status)
        assert torch.equal(sj["scores"][:, :sj["n"]].view(torch.int16), full.view(torch.int16))
        assert st == st1 and st["code"] == 0
        k = st["k"]
        assert torch.equal(ids[:, :k], ids1[:, :k])
        assert torch.equal(counts, counts1)
