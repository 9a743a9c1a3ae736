"""Layer pipelining (hs_gqa_select_then_score): one layer's selection and the
next layer's scoring in one call equal the two calls made in turn, bit for
bit, for every output of both (the single calls are pinned to the oracle
elsewhere).  Covers rank and id order, batches on both sides, repeated calls
on the same buffers, and jobs off the per-head path."""
import math

import numpy as np
import pytest
import torch

from hs_data import batch_ns, make_jobs

pytestmark = pytest.mark.gpu

ALPHA, RATIO = 5.0, 0.2


def kmax(n):
    return min(n, math.floor(n * float(np.float32(RATIO))))


def select_job(hs, scores, n, partial):
    k = max(1, kmax(n))
    return dict(scores=scores, n=n, head0_partial=partial,
                ids=torch.full((32, k), -1, dtype=torch.int32, device="cuda"),
                counts=torch.full((32,), -1, dtype=torch.int32, device="cuda"),
                member=torch.full((32, (n + 31) // 32), -1, dtype=torch.int32, device="cuda"),
                status=hs.ops.new_status("cuda"),
                ws=hs.ops.workspace(hs.ops.select_workspace_bytes(32, n), "cuda"))


def expected_select(hs, job, id_order):
    ids, counts, member, status = hs.ops.select(
        job["scores"], 32, job["scores"].shape[-1], job["n"], ALPHA, RATIO, scale_raw=True,
        id_order=id_order, head0_partial=job["head0_partial"],
        member=torch.zeros_like(job["member"]))
    return ids, counts, member, hs.ops.read_status(status)


def assert_select_equal(hs, job, want):
    ids, counts, member, status = want
    st = hs.ops.read_status(job["status"])
    assert st == status
    k = status["k"]
    assert torch.equal(job["ids"][:, :k], ids[:, :k])
    assert torch.equal(job["counts"], counts)
    assert torch.equal(job["member"], member)


def scored_layer(hs, job):
    out = torch.empty((32, job["tokens"]), dtype=torch.float16, device="cuda")
    hs.ops.score(job["q16"], job["keys"], job["tokens"], out=out, head0_partial=job["head0_partial"])
    return out


@pytest.mark.parametrize("id_order", [False, True])
def test_select_then_score_equals_two_calls(hs, id_order):
    n = 32768
    layer_a, layer_b = make_jobs(hs, [n, n], 7000 + id_order)
    raw_a = scored_layer(hs, layer_a)
    want_b = scored_layer(hs, dict(layer_b))
    want_part_b = layer_b["head0_partial"].clone()
    want = expected_select(hs, select_job(hs, raw_a, n, layer_a["head0_partial"]), id_order)
    job = select_job(hs, raw_a, n, layer_a["head0_partial"])
    for call in range(2):  # the second call reuses every buffer
        out_b = torch.full((32, n), -1, dtype=torch.int16, device="cuda").view(torch.float16)
        part_b = torch.full_like(want_part_b, -1)
        hs.ops.select_then_score(
            [job], [dict(q16=layer_b["q16"], keys=layer_b["keys"], tokens=n, out=out_b,
                         head0_partial=part_b)],
            32, ALPHA, RATIO, scale_raw=True, id_order=id_order)
        torch.cuda.synchronize()
        assert torch.equal(out_b.view(torch.int16), want_b.view(torch.int16)), call
        assert torch.equal(part_b, want_part_b), call
        assert_select_equal(hs, job, want)
    assert want[3]["k"] == kmax(n)


@pytest.mark.parametrize("id_order", [False, True])
def test_batched_select_then_batched_score(hs, id_order):
    # 3 selections (their heads take 96 CUs) beside 3 scoring jobs
    sel_layers = make_jobs(hs, batch_ns(21, 3), 7100)
    next_layers = make_jobs(hs, batch_ns(22, 2) + [100], 7200)
    raws = [scored_layer(hs, j) for j in sel_layers]
    jobs = [select_job(hs, r, j["tokens"], j["head0_partial"]) for r, j in zip(raws, sel_layers)]
    wants = [expected_select(hs, select_job(hs, r, j["tokens"], j["head0_partial"]), id_order)
             for r, j in zip(raws, sel_layers)]
    want_scores, score_jobs = [], []
    for j in next_layers:
        want_scores.append((scored_layer(hs, dict(j)), j["head0_partial"].clone()))
        score_jobs.append(dict(q16=j["q16"], keys=j["keys"], tokens=j["tokens"],
                               out=torch.empty((32, j["tokens"]), dtype=torch.float16, device="cuda"),
                               head0_partial=torch.full_like(j["head0_partial"], -1)))
    hs.ops.select_then_score(jobs, score_jobs, 32, ALPHA, RATIO, scale_raw=True, id_order=id_order)
    torch.cuda.synchronize()
    for job, want in zip(jobs, wants):
        assert_select_equal(hs, job, want)
    for sj, (out, part) in zip(score_jobs, want_scores):
        assert torch.equal(sj["out"].view(torch.int16), out.view(torch.int16))
        assert torch.equal(sj["head0_partial"], part)


def test_select_then_score_off_the_per_head_path(hs):
    # n > 32768 takes the slice launch chain: the call runs the two in turn
    n = 40000
    layer_a, layer_b = make_jobs(hs, [n, 4096], 7300)
    raw_a = scored_layer(hs, layer_a)
    want_b = scored_layer(hs, dict(layer_b))
    want_part_b = layer_b["head0_partial"].clone()
    want = expected_select(hs, select_job(hs, raw_a, n, layer_a["head0_partial"]), False)
    job = select_job(hs, raw_a, n, layer_a["head0_partial"])
    out_b = torch.empty((32, 4096), dtype=torch.float16, device="cuda")
    part_b = torch.full_like(want_part_b, -1)
    hs.ops.select_then_score([job], [dict(q16=layer_b["q16"], keys=layer_b["keys"], tokens=4096,
                                          out=out_b, head0_partial=part_b)],
                             32, ALPHA, RATIO, scale_raw=True)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), want_b.view(torch.int16))
    assert torch.equal(part_b, want_part_b)
    assert_select_equal(hs, job, want)


def test_select_then_score_small_layers(hs):
    # a few tokens on both sides: most scoring workgroups find no tile
    layer_a, layer_b = make_jobs(hs, [64, 130], 7400)
    raw_a = scored_layer(hs, layer_a)
    want_b = scored_layer(hs, dict(layer_b))
    want_part_b = layer_b["head0_partial"].clone()
    want = expected_select(hs, select_job(hs, raw_a, 64, layer_a["head0_partial"]), False)
    job = select_job(hs, raw_a, 64, layer_a["head0_partial"])
    out_b = torch.empty((32, 130), dtype=torch.float16, device="cuda")
    part_b = torch.full_like(want_part_b, -1)
    hs.ops.select_then_score([job], [dict(q16=layer_b["q16"], keys=layer_b["keys"], tokens=130,
                                          out=out_b, head0_partial=part_b)],
                             32, ALPHA, RATIO, scale_raw=True)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), want_b.view(torch.int16))
    assert torch.equal(part_b, want_part_b)
    assert_select_equal(hs, job, want)
