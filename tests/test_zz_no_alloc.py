"""hs_decode_layer_noalloc: the decode layer with its scratch in the
library's device array instead of a caller workspace.  Its outputs must
equal hs_decode_layer's (same inputs, caller workspace) bit for bit, on two
calls in a row, the second with a smaller layer (the array keeps the first
call's contents), and sizes beyond HS_NOALLOC_MAX_TOKENS are refused."""
import ctypes

import numpy as np
import pytest
import torch

from hs_data import f16_bits, pool_rows, rng, rope_keys, to_dev

pytestmark = pytest.mark.gpu
ALPHA, RATIO = 5.0, 0.2


def _layer(n, seed):
    g = rng(seed)
    k = rope_keys(n, seed)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    return dict(n=n, q16=to_dev(f16_bits(g.standard_normal((32, 128))).reshape(-1)),
                q32=torch.from_numpy(g.standard_normal((32, 128)).astype(np.float32)).cuda(),
                kpool=to_dev(np.ascontiguousarray(pool[:, :1024]).reshape(-1)),
                vpool=to_dev(np.ascontiguousarray(pool[:, 1024:]).reshape(-1)))


def _outputs(n, kmax):
    return dict(scores=torch.empty((32, n), dtype=torch.float16, device="cuda"),
                ids=torch.empty((32, kmax), dtype=torch.int32, device="cuda"),
                counts=torch.empty(32, dtype=torch.int32, device="cuda"),
                out=torch.empty((32, 128), dtype=torch.float32, device="cuda"),
                status=torch.zeros(4, dtype=torch.int32, device="cuda"))


def _call(hs, d, o, noalloc):
    L = hs.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    n, kmax = d["n"], o["ids"].shape[1]
    args = [p(d["q16"]), p(d["q32"]), p(d["kpool"]), p(d["vpool"]), 2048, None, n, n, ALPHA, RATIO,
            0, p(o["scores"]), p(o["ids"]), kmax, p(o["counts"]), p(o["out"]), p(o["status"])]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = L.hs_decode_layer_noalloc(*args, st)
    else:
        ws = torch.empty(L.hs_decode_layer_workspace_bytes(n), dtype=torch.uint8, device="cuda")
        rc = L.hs_decode_layer(*args, p(ws), st)
        torch.cuda.synchronize()  # the workspace lives until the layer is done
    return rc


def test_noalloc_layer_equals_workspace_layer(hs):
    for n, seed in ((32768, 901), (4096, 902)):  # the second call smaller
        d = _layer(n, seed)
        kmax = int(np.floor(n * np.float32(RATIO)))
        want, got = _outputs(n, kmax), _outputs(n, kmax)
        assert _call(hs, d, want, False) == 0
        assert _call(hs, d, got, True) == 0
        torch.cuda.synchronize()
        st = hs.ops.read_status(got["status"])
        assert st["code"] == 0 and st["k"] == kmax, st
        for name in ("scores", "ids", "counts", "out", "status"):
            assert torch.equal(got[name].view(torch.int32) if name == "out" else got[name],
                               want[name].view(torch.int32) if name == "out" else want[name]), (n, name)


def test_noalloc_refuses_beyond_its_array(hs):
    n = 32768 + 64
    d = dict(n=n, q16=torch.zeros(4096, dtype=torch.float16, device="cuda"),
             q32=torch.zeros((32, 128), dtype=torch.float32, device="cuda"),
             kpool=torch.zeros(n * 1024, dtype=torch.float16, device="cuda"),
             vpool=torch.zeros(n * 1024, dtype=torch.float16, device="cuda"))
    o = _outputs(n, int(np.floor(n * np.float32(RATIO))))
    assert _call(hs, d, o, True) == hs.HS_ERR_ARGUMENT
    assert "HS_NOALLOC_MAX_TOKENS" in hs.last_error()


def test_noalloc_allocates_nothing(hs):
    """The contract itself: after the first call on the device (which only
    looks up the array's address), calls change no device memory in use."""
    n = 4096
    d = _layer(n, 903)
    kmax = int(np.floor(n * np.float32(RATIO)))
    o = _outputs(n, kmax)
    assert _call(hs, d, o, True) == 0
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert _call(hs, d, o, True) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before
    assert hs.ops.read_status(o["status"])["code"] == 0


def test_noalloc_graph_replays_equal_eager(hs):
    """hs_decode_layer_noalloc captured in a HIP graph (torch.cuda.graph) and
    replayed on new inputs copied into the captured buffers by eager work
    between replays: every replay equals an eager hs_decode_layer (caller
    workspace) on the same inputs, bit for bit."""
    n = 4096
    kmax = int(np.floor(n * np.float32(RATIO)))
    d = _layer(n, 910)
    got = _outputs(n, kmax)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _call(hs, d, got, True) == 0  # first call on the device: address lookup
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            rc = _call(hs, d, got, True)
        assert rc == 0
        torch.cuda.synchronize()
    for seed in (911, 912, 913):
        fresh = _layer(n, seed)
        for key in ("q16", "q32", "kpool", "vpool"):
            d[key].copy_(fresh[key])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _outputs(n, kmax)
        assert _call(hs, fresh, want, False) == 0
        torch.cuda.synchronize()
        assert hs.ops.read_status(got["status"])["code"] == 0
        for name in ("scores", "ids", "counts", "out", "status"):
            a, b = got[name], want[name]
            if name == "out":
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), (seed, name)
