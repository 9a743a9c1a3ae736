"""Reentrancy across streams: the C entry points keep no global state beyond
a per-device CU count, so calls on distinct streams with distinct outputs
and workspaces may run concurrently (the reference scores hot and cold keys
on separate scorer instances at once and stages copies on private streams:
policy/full_gqa_runtime.cpp:121-124,493-516, runtime/gqa_prefetch_cuda.cu:
28-30).  Every output of the concurrent runs must equal the serial run's
bit for bit."""
import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, pool_rows, rng, rope_keys, to_dev

pytestmark = pytest.mark.gpu
ALPHA, RATIO = 5.0, 0.2


def _layer(seed, n):
    g = rng(seed)
    k = rope_keys(n, seed)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    return dict(n=n, q16=to_dev(f16_bits(g.standard_normal((32, 128))).reshape(-1)),
                q32=torch.from_numpy(g.standard_normal((32, 128)).astype(np.float32)).cuda(),
                kpool=to_dev(np.ascontiguousarray(pool[:, :1024]).reshape(-1)),
                vpool=to_dev(np.ascontiguousarray(pool[:, 1024:]).reshape(-1)))


def _run(hs, d, stream):
    """One layer on `stream` with its own outputs and workspace (allocated
    here and kept alive by the caller until the streams are synchronised)."""
    n = d["n"]
    ws = hs.ops.workspace(hs.ops.decode_layer_workspace_bytes(n))
    status = hs.ops.new_status("cuda", stream)
    res = hs.ops.decode_layer(d["q16"], d["q32"], d["kpool"], n, ALPHA, RATIO, ws=ws, status=status,
                              v_pool=d["vpool"], row_bytes=2048, stream=stream)
    return res + (ws,)


def _host(res):
    scores, ids, counts, out, status = res[:5]
    return (from_dev(scores), from_dev(ids), from_dev(counts), out.cpu().numpy().view(np.uint32),
            status.cpu().numpy())


def test_decode_layers_on_two_streams(hs):
    layers = [_layer(71, 8192), _layer(72, 32768), _layer(73, 12288), _layer(74, 32768)]
    serial = [_host(_run(hs, d, None)) for d in layers]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        pending = []
        # enqueue alternately so the two streams' kernels interleave
        for i, d in enumerate(layers):
            pending.append(_run(hs, d, streams[(i + rep) % 2]))
        torch.cuda.synchronize()
        for want, got in zip(serial, pending):
            for a, b in zip(want, _host(got)):
                assert np.array_equal(a, b)


def test_select_then_score_beside_attention(hs):
    """A pipelined selection-and-scoring call on one stream while another
    stream runs a sparse attention and a scoring call of other sequences."""
    n = 16384
    a, b = _layer(81, n), _layer(82, n)
    kmax = int(np.floor(n * np.float32(RATIO)))

    def buffers():
        return dict(raw=torch.empty((32, n), dtype=torch.float16, device="cuda"),
                    part=torch.empty(n // 64, dtype=torch.int32, device="cuda"),
                    ids=torch.empty((32, kmax), dtype=torch.int32, device="cuda"),
                    status=hs.ops.new_status(),
                    ws=hs.ops.workspace(hs.ops.select_workspace_bytes(32, n)),
                    raw2=torch.empty((32, n), dtype=torch.float16, device="cuda"),
                    out=torch.empty((32, 128), dtype=torch.float32, device="cuda"),
                    aws=hs.ops.workspace(hs.ops.attention_workspace_bytes(n)))

    member = torch.zeros((32, n // 32), dtype=torch.int32, device="cuda")
    g = rng(83)
    member.copy_(torch.from_numpy(g.integers(0, 2**31, size=(32, n // 32), dtype=np.int64)
                                  .astype(np.int32)))

    def run(buf, s1, s2):
        hs.ops.score(a["q16"], a["kpool"], n, out=buf["raw"], head0_partial=buf["part"], stream=s1)
        hs.ops.select_then_score(
            [dict(scores=buf["raw"], n=n, head0_partial=buf["part"], ids=buf["ids"],
                  status=buf["status"], ws=buf["ws"])],
            [dict(q16=b["q16"], keys=b["kpool"], tokens=n, out=buf["raw2"])],
            32, ALPHA, RATIO, stream=s1, scale_raw=True)
        hs.ops.sparse_attention(b["q32"], b["kpool"], n, member, out=buf["out"], ws=buf["aws"],
                                v_pool=b["vpool"], row_bytes=2048, stream=s2)
        s3 = hs.ops.score(b["q16"], a["kpool"], n, stream=s2)
        return s3

    serial = buffers()
    s_extra = run(serial, None, None)
    torch.cuda.synchronize()
    want = {k: v.cpu() for k, v in serial.items()}
    want_extra = s_extra.cpu()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        buf = buffers()
        torch.cuda.synchronize()  # the status fill (current stream) before s1 writes it
        extra = run(buf, s1, s2)
        torch.cuda.synchronize()
        for k, v in buf.items():
            if k not in ("ws", "aws"):  # scratch
                assert torch.equal(v.cpu(), want[k]), k
        assert torch.equal(extra.cpu(), want_extra)
