"""HIP graph capture of the decode path: the entry points enqueue kernels
only (no allocation, memset or synchronisation), so a caller can capture a
layer, or a pipelined run of layers, once and replay it.  Each replay runs on
new inputs written into the captured buffers by eager kernels between
replays, and must equal the eager calls on the same inputs bit for bit
(scores, ids, counts, membership words, status, attention output).  The same
pipelined run, eager, with a nonfinite key in its middle layer shows that a
failed layer stays reported and never reuses an earlier layer's selection."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

N, ALPHA, RATIO = 4096, 5.0, 0.2
KMAX = min(N, math.floor(N * float(np.float32(RATIO))))


def fill_layer(hs, k, v, q16, q32, seed):
    hs.ops.fill_rope_keys(k, N, 1024, 8, seed=seed, theta=500000.0)
    hs.ops.fill_gaussian(v, seed=seed + 1)
    hs.ops.fill_gaussian(q16, seed=seed + 2)
    q32.copy_(torch.randn(q32.shape, generator=torch.Generator(device="cuda").manual_seed(seed),
                          device="cuda"))


def capture(fn, stream):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def test_decode_layer_graph_replays_equal_eager(hs):
    dev = "cuda"
    k = torch.empty(N * 1024, dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    q16 = torch.empty(4096, dtype=torch.float16, device=dev)
    q32 = torch.empty((32, 128), dtype=torch.float32, device=dev)
    scores = torch.empty((32, N), dtype=torch.float16, device=dev)
    ids = torch.empty((32, KMAX), dtype=torch.int32, device=dev)
    counts = torch.empty(32, dtype=torch.int32, device=dev)
    out = torch.empty((32, 128), dtype=torch.float32, device=dev)
    status = hs.ops.new_status(dev)
    ws = hs.ops.workspace(hs.ops.decode_layer_workspace_bytes(N), dev)
    outputs = (scores, ids, counts, out, status)

    def layer():
        hs.ops.decode_layer(q16, q32, k, N, ALPHA, RATIO, scores=scores, ids=ids, ids_stride=KMAX,
                            counts=counts, out=out, status=status, ws=ws, v_pool=v, row_bytes=2048)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        fill_layer(hs, k, v, q16, q32, 11)
        layer()
        torch.cuda.synchronize()
        graph = capture(layer, side)
        for seed in (21, 31, 41):
            fill_layer(hs, k, v, q16, q32, seed)
            for t in outputs:
                t.fill_(-1) if t.dtype != torch.float16 else t.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            replayed = [t.clone() for t in outputs]
            layer()
            torch.cuda.synchronize()
            st = hs.ops.read_status(status)
            assert st["code"] == 0 and st["k"] == KMAX, (seed, st)
            for name, a, b in zip(("scores", "ids", "counts", "out", "status"), replayed, outputs):
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), (seed, name)


def test_pipelined_layers_graph_replays_equal_eager(hs):
    """Three layers on the realizable schedule: layer 0's history, then each
    layer's selection (completing its current token) beside the next layer's
    history scoring, then its attention over K and V rows."""
    dev, layers = "cuda", 3
    ks = [torch.empty(N * 1024, dtype=torch.float16, device=dev) for _ in range(layers)]
    vs = [torch.empty_like(ks[0]) for _ in range(layers)]
    qs = [torch.empty(4096, dtype=torch.float16, device=dev) for _ in range(layers)]
    q32s = [torch.empty((32, 128), dtype=torch.float32, device=dev) for _ in range(layers)]
    raws = [torch.empty((32, N), dtype=torch.float16, device=dev) for _ in range(2)]
    parts = [torch.empty(N // 64, dtype=torch.int32, device=dev) for _ in range(2)]
    ids = torch.empty((32, KMAX), dtype=torch.int32, device=dev)
    counts = torch.empty(32, dtype=torch.int32, device=dev)
    member = torch.empty((32, N // 32), dtype=torch.int32, device=dev)
    outs = [torch.empty((32, 128), dtype=torch.float32, device=dev) for _ in range(layers)]
    statuses = [hs.ops.new_status(dev) for _ in range(layers)]
    sws = hs.ops.workspace(hs.ops.select_workspace_bytes(32, N), dev)
    aws = hs.ops.workspace(hs.ops.attention_workspace_bytes(N), dev)
    outputs = [*raws, ids, counts, member, *outs, *statuses]

    def job(l):
        return dict(scores=raws[l % 2], n=N, head0_partial=parts[l % 2], ids=ids, ids_stride=KMAX,
                    counts=counts, member=member, status=statuses[l], ws=sws, current_q=qs[l],
                    current_key=ks[l][(N - 1) * 1024:])

    def hist(l):
        return dict(q16=qs[l], keys=ks[l], tokens=N - 1, out=raws[l % 2], score_stride=N,
                    head0_partial=parts[l % 2])

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        flags = dict(scale_raw=True, require_k=True, id_order=True)
        calls = [hs.ops.prepare_select_then_score([job(l)], [hist(l + 1)], 32, ALPHA, RATIO,
                                                  **flags) for l in range(layers - 1)]
        calls.append(hs.ops.prepare_select_batched([job(layers - 1)], 32, ALPHA, RATIO, **flags))

        def run():
            hs.ops.score(qs[0], ks[0], N - 1, out=raws[0], score_stride=N, head0_partial=parts[0])
            for l in range(layers):
                calls[l]()
                hs.ops.sparse_attention(q32s[l], ks[l], N, member, out=outs[l], ws=aws,
                                        v_pool=vs[l], row_bytes=2048)

        def fill(seed):
            for l in range(layers):
                fill_layer(hs, ks[l], vs[l], qs[l], q32s[l], seed + 10 * l)

        fill(100)
        run()
        torch.cuda.synchronize()
        graph = capture(run, side)
        for seed in (200, 300):
            fill(seed)
            for t in outputs:
                t.fill_(-1) if t.dtype != torch.float16 else t.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            replayed = [t.clone() for t in outputs]
            run()
            torch.cuda.synchronize()
            for l, st in enumerate(statuses):
                s = hs.ops.read_status(st)
                assert s["code"] == 0 and s["k"] == KMAX, (seed, l, s)
            for i, (a, b) in enumerate(zip(replayed, outputs)):
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), (seed, i)


def test_failed_middle_layer_is_reported_not_stale(hs):
    """Three pipelined layers sharing one membership buffer, each with its own
    status: a NaN key in layer 1's history makes layer 1's selection fail
    with HS_ERR_NONFINITE, which stays visible after the run; its membership
    words are cleared, so its attention output is NaN (no selected row), not
    the previous layer's; layers 0 and 2 select and attend normally."""
    dev, layers = "cuda", 3
    ks = [torch.empty(N * 1024, dtype=torch.float16, device=dev) for _ in range(layers)]
    vs = [torch.empty_like(ks[0]) for _ in range(layers)]
    qs = [torch.empty(4096, dtype=torch.float16, device=dev) for _ in range(layers)]
    q32s = [torch.empty((32, 128), dtype=torch.float32, device=dev) for _ in range(layers)]
    for l in range(layers):
        fill_layer(hs, ks[l], vs[l], qs[l], q32s[l], 500 + 10 * l)
    ks[1][100 * 1024 + 5] = float("nan")  # token 100, KV head 0: query heads 0-3
    raws = [torch.empty((32, N), dtype=torch.float16, device=dev) for _ in range(2)]
    parts = [torch.empty(N // 64, dtype=torch.int32, device=dev) for _ in range(2)]
    ids = torch.empty((32, KMAX), dtype=torch.int32, device=dev)
    member = torch.empty((32, N // 32), dtype=torch.int32, device=dev)
    outs = [torch.zeros((32, 128), dtype=torch.float32, device=dev) for _ in range(layers)]
    statuses = [hs.ops.new_status(dev) for _ in range(layers)]
    sws = hs.ops.workspace(hs.ops.select_workspace_bytes(32, N), dev)
    aws = hs.ops.workspace(hs.ops.attention_workspace_bytes(N), dev)

    def job(l):
        return dict(scores=raws[l % 2], n=N, head0_partial=parts[l % 2], ids=ids, ids_stride=KMAX,
                    member=member, status=statuses[l], ws=sws, current_q=qs[l],
                    current_key=ks[l][(N - 1) * 1024:])

    flags = dict(scale_raw=True, require_k=True, id_order=True)
    hs.ops.score(qs[0], ks[0], N - 1, out=raws[0], score_stride=N, head0_partial=parts[0])
    for l in range(layers):
        if l + 1 < layers:
            hs.ops.select_then_score(
                [job(l)], [dict(q16=qs[l + 1], keys=ks[l + 1], tokens=N - 1, out=raws[(l + 1) % 2],
                                score_stride=N, head0_partial=parts[(l + 1) % 2])],
                32, ALPHA, RATIO, **flags)
        else:
            hs.ops.prepare_select_batched([job(l)], 32, ALPHA, RATIO, **flags)()
        hs.ops.sparse_attention(q32s[l], ks[l], N, member, out=outs[l], ws=aws, v_pool=vs[l],
                                row_bytes=2048)
    torch.cuda.synchronize()
    codes = [hs.ops.read_status(st)["code"] for st in statuses]
    assert codes == [hs.HS_OK, hs.HS_ERR_NONFINITE, hs.HS_OK], codes
    assert torch.isnan(outs[1]).all()
    assert torch.isfinite(outs[0]).all() and torch.isfinite(outs[2]).all()


def test_self_stamped_status_under_graph_replays(hs):
    """Gather and the rehearsal query stamp their own status with a per-call
    stamp; a captured call replays the captured stamp, so under capture the
    library clears the status first.  Replays alternate failing and clean
    inputs (written in place between replays, eagerly): every replay reports
    its own outcome, a clean one after a failing one reads HS_OK, and the
    rows equal the eager call's."""
    dev = "cuda"
    slots = 32
    g = torch.Generator(device="cpu").manual_seed(5)
    pre = torch.randint(0, 256, (3 * 4096,), dtype=torch.uint8, generator=g).to(dev)
    row_map = torch.full((32 * slots,), -1, dtype=torch.int32, device=dev)
    good = row_map.clone()
    good[::slots] = 0
    good[1::slots] = 2
    bad = good.clone()
    bad[5] = 3  # beyond the three prefetched rows
    hidden = torch.randn((4, 4096), generator=g).to(torch.bfloat16).to(dev)
    wq = (torch.randn((4096, 4096), generator=g) * 0.02).to(torch.bfloat16).to(dev)
    hidden_bad = hidden.clone()
    hidden_bad[2, 7] = float("nan")
    h_in = hidden.clone()
    q_out = torch.empty((4, 32, 128), dtype=torch.float16, device=dev)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        row_map.copy_(good)
        eager_k, eager_v, _ = hs.ops.gather_rows(pre, None, row_map, slots)
        eager_q, _ = hs.ops.rehearsal_query(h_in, wq, [100, 200, 300, 400])
        torch.cuda.synchronize()
        captured = {}

        def step():
            captured["gather"] = hs.ops.gather_rows(pre, None, row_map, slots)
            captured["rehearsal"] = hs.ops.rehearsal_query(h_in, wq, [100, 200, 300, 400],
                                                           out=q_out)

        graph = capture(step, side)
        for rnd, failing in enumerate([True, False, False, True, False]):
            row_map.copy_(bad if failing else good)
            h_in.copy_(hidden_bad if failing else hidden)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            k, v, st = captured["gather"]
            q, qst = captured["rehearsal"]
            code = hs.ops.read_status(st)["code"]
            codes = [int(c) for c in qst[:, 0].cpu().tolist()]
            if failing:
                assert code == hs.HS_ERR_MISSING, (rnd, code)
                assert codes == [0, 0, hs.HS_ERR_NONFINITE, 0], (rnd, codes)
            else:
                assert code == 0, (rnd, code)
                assert codes == [0, 0, 0, 0], (rnd, codes)
                # bit patterns (random bytes hold NaN encodings, which == refuses)
                bits = lambda t: t.view(torch.int16)
                assert torch.equal(bits(k), bits(eager_k)) and torch.equal(bits(v), bits(eager_v))
                assert torch.equal(bits(q), bits(eager_q))
