"""Closed-form checks of the FP64 attention oracle (parity unpinned against
the reference, whose attention is third-party ggml CUDA)."""
import numpy as np

from hs_data import f16_bits, pool_rows, rng


def make_pool(g, n):
    k = f16_bits(g.standard_normal((n, 8, 128)))
    v = f16_bits(g.standard_normal((n, 8, 128)))
    return k, v, pool_rows(k, v).view(np.uint8)


def test_single_key_returns_value_row(port):
    g = rng(1)
    n = 40
    k, v, pool = make_pool(g, n)
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [[int(g.integers(0, n))] for _ in range(32)]
    out = port.attention(q, pool, ids)
    for h in range(32):
        vv = v[ids[h][0], h // 4].view(np.float16).astype(np.float64)
        assert np.array_equal(out[h], vv)


def test_equal_keys_average_values(port):
    g = rng(2)
    n = 64
    k, v, _ = make_pool(g, n)
    k[:] = k[0]  # every key identical -> uniform softmax
    pool = pool_rows(k, v).view(np.uint8)
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [list(range(0, n, 3)) for _ in range(32)]
    out = port.attention(q, pool, ids)
    for h in range(32):
        mean = v[ids[h], h // 4].view(np.float16).astype(np.float64).mean(axis=0)
        assert np.allclose(out[h], mean, rtol=1e-12, atol=1e-12)


def test_row_map_and_numpy_softmax(port):
    g = rng(3)
    n = 300
    k, v, pool = make_pool(g, n)
    perm = g.permutation(n).astype(np.int32)  # id -> row
    inv = np.argsort(perm)
    pool_perm = pool.reshape(n, 4096)[inv].reshape(-1)  # row r holds id inv[r]
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [sorted(g.choice(n, size=50, replace=False).tolist()) for _ in range(32)]
    a = port.attention(q, pool, ids)
    b = port.attention(q, pool_perm, ids, rows=perm)
    assert np.array_equal(a, b)
    kf = k.view(np.float16).astype(np.float64)
    vf = v.view(np.float16).astype(np.float64)
    for h in range(0, 32, 5):
        s = kf[ids[h], h // 4] @ q[h].astype(np.float64) / np.sqrt(128.0)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(a[h], p @ vf[ids[h], h // 4], rtol=1e-10, atol=1e-12)
