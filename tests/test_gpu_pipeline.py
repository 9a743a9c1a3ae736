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


def kv_layers(hs, n, count, seed):
    """Hot pools as K and V arrays (2048 B rows) with their rehearsal queries."""
    layers = []
    for i in range(count):
        kp = torch.empty(n * 1024, dtype=torch.float16, device="cuda")
        vp = torch.empty(n * 1024, dtype=torch.float16, device="cuda")
        q16 = torch.empty(4096, dtype=torch.float16, device="cuda")
        hs.ops.fill_rope_keys(kp, n, 1024, 8, seed=seed + 3 * i, theta=500000.0)
        hs.ops.fill_gaussian(vp, seed=seed + 3 * i + 1)
        hs.ops.fill_gaussian(q16, seed=seed + 3 * i + 2)
        q32 = torch.randn((32, 128), generator=torch.Generator(device="cuda").manual_seed(seed + i),
                          device="cuda")
        layers.append(dict(k=kp, v=vp, q16=q16, q32=q32))
    return layers


@pytest.mark.parametrize("n", [32768, 3000, 40000])
def test_pipelined_layers_equal_one_layer_at_a_time(hs, n):
    # (n = 40000 takes the slice launch chain: the counted selection skips
    # only the count launch there too)
    # score 0; per layer: select l (counted after the first) beside score l+1,
    # then attention l beside the count of l+1; the last layer alone
    layers = kv_layers(hs, n, 3, 7500 + n)
    want = []
    for L in layers:
        raw = torch.empty((32, n), dtype=torch.float16, device="cuda")
        part = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
        hs.ops.score(L["q16"], L["k"], n, out=raw, head0_partial=part)
        ids, counts, member, st = hs.ops.select(
            raw, 32, n, n, ALPHA, RATIO, scale_raw=True, require_k=True, id_order=True,
            head0_partial=part, member=torch.zeros((32, (n + 31) // 32), dtype=torch.int32,
                                                   device="cuda"))
        out = hs.ops.sparse_attention(L["q32"], L["k"], n, member, v_pool=L["v"], row_bytes=2048)
        want.append((ids.clone(), counts.clone(), member.clone(), hs.ops.read_status(st), out.clone()))

    raws = [torch.empty((32, n), dtype=torch.float16, device="cuda") for _ in range(2)]
    parts = [torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda") for _ in range(2)]
    aws = hs.ops.workspace(hs.ops.attention_workspace_bytes(n), "cuda")
    jobs = [select_job(hs, raws[i % 2], n, parts[i % 2]) for i in range(len(layers))]
    outs = [torch.full((32, 128), float("nan"), device="cuda") for _ in layers]
    flags = dict(scale_raw=True, require_k=True, id_order=True)
    hs.ops.score(layers[0]["q16"], layers[0]["k"], n, out=raws[0], head0_partial=parts[0])
    for i, L in enumerate(layers):
        if i + 1 < len(layers):
            nxt = layers[i + 1]
            hs.ops.select_then_score(
                [jobs[i]], [dict(q16=nxt["q16"], keys=nxt["k"], tokens=n, out=raws[(i + 1) % 2],
                                 head0_partial=parts[(i + 1) % 2])],
                32, ALPHA, RATIO, counted=i > 0, **flags)
            hs.ops.prepare_attention_then_count(
                L["q32"], L["k"], n, jobs[i]["member"], [jobs[i + 1]], 32, ALPHA, RATIO,
                out=outs[i], ws=aws, v_pool=L["v"], row_bytes=2048, **flags)()
        else:
            j = jobs[i]
            hs.ops.select(j["scores"], 32, n, n, ALPHA, RATIO, counted=True,
                          head0_partial=j["head0_partial"], ids=j["ids"], counts=j["counts"],
                          member=j["member"], status=j["status"], ws=j["ws"], **flags)
            hs.ops.sparse_attention(L["q32"], L["k"], n, j["member"], out=outs[i], ws=aws,
                                    v_pool=L["v"], row_bytes=2048)
        torch.cuda.synchronize()
        w_ids, w_counts, w_member, w_status, w_out = want[i]
        assert_select_equal(hs, jobs[i], (w_ids, w_counts, w_member, w_status))
        assert torch.equal(outs[i], w_out), i


@pytest.mark.parametrize("id_order", [False, True])
def test_counted_selection_equals_plain(hs, id_order):
    # the count launch of hs_gqa_attention_then_count feeds a selection run
    # with HS_SELECT_COUNTED (rank and id order), batched over two next jobs
    n = 32768
    layers = kv_layers(hs, n, 1, 7700)
    nxt = make_jobs(hs, [n, 8192], 7800 + id_order)
    raws = [scored_layer(hs, j) for j in nxt]
    wants = [expected_select(hs, select_job(hs, r, j["tokens"], j["head0_partial"]), id_order)
             for r, j in zip(raws, nxt)]
    L = layers[0]
    raw = torch.empty((32, n), dtype=torch.float16, device="cuda")
    part = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    hs.ops.score(L["q16"], L["k"], n, out=raw, head0_partial=part)
    _, _, member, _ = hs.ops.select(raw, 32, n, n, ALPHA, RATIO, scale_raw=True, id_order=True,
                                    head0_partial=part,
                                    member=torch.zeros((32, n // 32), dtype=torch.int32, device="cuda"))
    want_out = hs.ops.sparse_attention(L["q32"], L["k"], n, member, v_pool=L["v"], row_bytes=2048)
    jobs = [select_job(hs, r, j["tokens"], j["head0_partial"]) for r, j in zip(raws, nxt)]
    out = torch.empty((32, 128), device="cuda")
    aws = hs.ops.workspace(hs.ops.attention_workspace_bytes(n), "cuda")
    hs.ops.prepare_attention_then_count(L["q32"], L["k"], n, member, jobs, 32, ALPHA, RATIO,
                                        out=out, ws=aws, v_pool=L["v"], row_bytes=2048,
                                        scale_raw=True, id_order=id_order)()
    for j in jobs:
        hs.ops.select(j["scores"], 32, j["n"], j["n"], ALPHA, RATIO, scale_raw=True,
                      id_order=id_order, counted=True, head0_partial=j["head0_partial"],
                      ids=j["ids"], counts=j["counts"], member=j["member"], status=j["status"],
                      ws=j["ws"])
    torch.cuda.synchronize()
    assert torch.equal(out, want_out)
    for j, w in zip(jobs, wants):
        assert_select_equal(hs, j, w)


def test_select_then_score_history_cover(hs):
    # the history cover (HS_SELECT_COVER) through the combined launch
    n = 32767
    layer_a, layer_b = make_jobs(hs, [n, 4096], 7900)
    raw_a = scored_layer(hs, layer_a)
    want_b = scored_layer(hs, dict(layer_b))
    cover_k = min(n, math.floor((n + 1) * float(np.float32(RATIO))))
    ids, counts, member, st = hs.ops.select(raw_a, 32, n, n, ALPHA, RATIO, scale_raw=True,
                                            cover=True, id_order=True,
                                            head0_partial=layer_a["head0_partial"],
                                            member=torch.zeros((32, (n + 31) // 32),
                                                               dtype=torch.int32, device="cuda"))
    want = hs.ops.read_status(st)
    job = dict(scores=raw_a, n=n, head0_partial=layer_a["head0_partial"],
               ids=torch.full((32, cover_k), -1, dtype=torch.int32, device="cuda"),
               counts=torch.full((32,), -1, dtype=torch.int32, device="cuda"),
               member=torch.full((32, (n + 31) // 32), -1, dtype=torch.int32, device="cuda"),
               status=hs.ops.new_status("cuda"),
               ws=hs.ops.workspace(hs.ops.select_workspace_bytes(32, n), "cuda"))
    out_b = torch.empty((32, 4096), dtype=torch.float16, device="cuda")
    hs.ops.select_then_score([job], [dict(q16=layer_b["q16"], keys=layer_b["keys"], tokens=4096,
                                          out=out_b)],
                             32, ALPHA, RATIO, scale_raw=True, cover=True, id_order=True)
    torch.cuda.synchronize()
    assert hs.ops.read_status(job["status"]) == want
    k = want["k"]
    assert torch.equal(job["ids"][:, :k], ids[:, :k])
    assert torch.equal(job["counts"], counts)
    assert torch.equal(job["member"], member)
    assert torch.equal(out_b.view(torch.int16), want_b.view(torch.int16))


def test_counted_wide_batch_then_single_selections(hs):
    # hs_gqa_attention_then_count over a batch of 16 next jobs (more (head,
    # slice) pairs than one round of count groups: 4 slices per workgroup)
    # feeds counted selections made one job at a time: the count records do
    # not depend on how the count launch grouped the slices
    ns = batch_ns(31)
    assert sum(32 * -(-n // 4096) for n in ns) > 1024
    nxt = make_jobs(hs, ns, 7900)
    raws = [scored_layer(hs, j) for j in nxt]
    wants = [expected_select(hs, select_job(hs, r, j["tokens"], j["head0_partial"]), False)
             for r, j in zip(raws, nxt)]
    n = 4096
    L = kv_layers(hs, n, 1, 7950)[0]
    member = torch.full((32, n // 32), -1, dtype=torch.int32, device="cuda")  # every id
    want_out = hs.ops.sparse_attention(L["q32"], L["k"], n, member, v_pool=L["v"], row_bytes=2048)
    jobs = [select_job(hs, r, j["tokens"], j["head0_partial"]) for r, j in zip(raws, nxt)]
    out = torch.empty((32, 128), device="cuda")
    aws = hs.ops.workspace(hs.ops.attention_workspace_bytes(n), "cuda")
    hs.ops.prepare_attention_then_count(L["q32"], L["k"], n, member, jobs, 32, ALPHA, RATIO,
                                        out=out, ws=aws, v_pool=L["v"], row_bytes=2048,
                                        scale_raw=True)()
    for j in jobs:
        hs.ops.select(j["scores"], 32, j["n"], j["n"], ALPHA, RATIO, scale_raw=True, counted=True,
                      head0_partial=j["head0_partial"], ids=j["ids"], counts=j["counts"],
                      member=j["member"], status=j["status"], ws=j["ws"])
    torch.cuda.synchronize()
    assert torch.equal(out, want_out)
    for j, w in zip(jobs, wants):
        assert_select_equal(hs, j, w)
