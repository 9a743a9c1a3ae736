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
