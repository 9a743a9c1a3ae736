"""GPU parity of kernel #1 (scoring) against the CPU oracle: bit-exact."""
import numpy as np
import pytest
import torch

from hs_data import H, D, from_dev, markers_v3, mixed_finite, rng, to_dev, v3_sample

pytestmark = pytest.mark.gpu
CANARY = 0x55AA


def pipeline(hs, q, k, n, guard=2):
    """V3 ABI call with canaries around and past the score extent."""
    out = torch.full((32 * n + 2 * guard * 32,), 0, dtype=torch.int16, device="cuda")
    out.fill_(CANARY)
    view = out[guard * 32: guard * 32 + 32 * n].view(torch.float16)
    hs.ops.full_gqa_pipeline(to_dev(q), to_dev(k), n, out=view)
    got = from_dev(out.view(torch.float16))
    assert np.all(got[: guard * 32] == CANARY) and np.all(got[guard * 32 + 32 * n:] == CANARY)
    return got[guard * 32: guard * 32 + 32 * n].reshape(32, n)


@pytest.mark.parametrize("n", [64, 128, 192, 256, 320, 1024])
def test_v3_random(hs, port, n):
    # kernels/full_gqa_pipeline/kernel_check.cpp:122-125
    g = rng(300 + n)
    q, k = v3_sample(g, 4096), v3_sample(g, n * 1024)
    assert np.array_equal(pipeline(hs, q, k, n), port.score(q, k, n))


@pytest.mark.parametrize("n", [192, 256])
def test_v3_markers(hs, port, n):
    q, k = markers_v3(n, rng(n))
    got = pipeline(hs, q, k, n)
    t = np.arange(n)
    assert np.array_equal(got[0], (t + 1).astype(np.uint16))
    assert np.array_equal(got[28], (0x8000 | (t + 1)).astype(np.uint16))
    assert np.all(got[31] == 0)
    assert np.array_equal(got, port.score(q, k, n))


def test_v3_invalid_counts_touch_nothing(hs):
    # kernel_check.cpp:116-121: invalid N returns without any memory access
    sentinel = torch.full((32,), 0x1234, dtype=torch.int16, device="cuda")
    q = torch.zeros(4096, dtype=torch.float16, device="cuda")
    k = torch.zeros(1024 * 64, dtype=torch.float16, device="cuda")
    for n in [0, 1, 32, 63, 65, 32769, 0xFFFFFFFF]:
        rc = hs.lib().hs_full_gqa_pipeline(hs.ops._p(q), hs.ops._p(k), hs.ops._p(sentinel), n,
                                           hs.ops._s(None))
        assert rc == hs.HS_ERR_ARGUMENT
    torch.cuda.synchronize()
    assert torch.all(sentinel == 0x1234)


def test_v3_head_channel_and_cancellation(hs, port):
    n = 192
    q = np.zeros(4096, dtype=np.uint16)
    k = np.zeros(n * 1024, dtype=np.uint16)
    for h in range(32):
        q[h * 128 + (h * 7) % 128] = np.float16((h + 1) / 32).view(np.uint16)
    t, hh, c = np.meshgrid(np.arange(n), np.arange(8), np.arange(128), indexing="ij")
    k[:] = (((t * 1024 + hh * 128 + c) / 16384).astype(np.float16)).view(np.uint16).reshape(-1)
    assert np.array_equal(pipeline(hs, q, k, n), port.score(q, k, n))
    edge = np.array([0, 0x8000, 1, 0x8001, 0x3FF, 0x400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF],
                    dtype=np.uint16)
    q = np.zeros(4096, dtype=np.uint16)
    k = np.zeros(n * 1024, dtype=np.uint16)
    for h in range(32):
        q[h * 128: h * 128 + 3] = [0x6C00, 0x3C00, 0xEC00]
        for c in range(3, 128):
            q[h * 128 + c] = edge[(h + c) % 10]
    for t in range(n):
        for h in range(8):
            base = (t * 8 + h) * 128
            k[base: base + 3] = [0x6C00, 0x3C00, 0x6C00]
            k[base + 3: base + 128] = (t + h + np.arange(3, 128)) % 1024
    assert np.array_equal(pipeline(hs, q, k, n), port.score(q, k, n))


@pytest.mark.parametrize("stride", [1024, 2048])
@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 17, 65, 129, 4097])
@pytest.mark.parametrize("use_rows", [False, True])
def test_general_scorer(hs, port, n, stride, use_rows):
    g = rng(n * 3 + stride + use_rows)
    q = mixed_finite(g, H * D)
    rows_total = n + 5
    k = mixed_finite(g, rows_total * stride)
    rows = g.permutation(rows_total)[:n].astype(np.int32) if use_rows else None
    score_stride = n + 3
    out = torch.full((32, score_stride), 0, dtype=torch.int16, device="cuda").fill_(CANARY)
    hs.ops.score(to_dev(q), to_dev(k), n, key_stride_words=stride,
                 rows=None if rows is None else to_dev(rows), out=out.view(torch.float16),
                 score_stride=score_stride)
    got = from_dev(out.view(torch.float16))
    if rows is None:
        expected = port.score(q, k, n, stride)
    else:
        gathered = np.concatenate([k[r * stride:(r + 1) * stride] for r in rows])
        expected = port.score(q, gathered, n, stride)
    assert np.array_equal(got[:, :n], expected)
    assert np.all(got[:, n:] == CANARY)


def test_max_shape(hs, port):
    # kernel_check.cpp:143-144 --max-shape
    n = 32768
    g = rng(32768)
    q, k = v3_sample(g, 4096), v3_sample(g, n * 1024)
    assert np.array_equal(pipeline(hs, q, k, n), port.score(q, k, n))


def test_head0_partial_maxima(hs, port):
    n = 1000
    g = rng(77)
    q, k = v3_sample(g, 4096), v3_sample(g, n * 1024)
    partial = torch.zeros((n + 63) // 64, dtype=torch.int32, device="cuda")
    out = hs.ops.score(to_dev(q), to_dev(k), n, head0_partial=partial)
    raw = from_dev(out)
    keys = np.array([port.order_key(int(b)) for b in raw[0]])
    expected = [keys[i * 64:(i + 1) * 64].max() for i in range((n + 63) // 64)]
    assert np.array_equal(from_dev(partial), np.array(expected, dtype=np.uint32))
