"""Checks of the FP64 attention oracle: closed forms (one key, equal keys,
the ln 3 two-key weights that fix the scale, a KV-head marker) and torch's
own GQA attention in FP64.  Parity against the reference's attention
(third-party ggml CUDA) stays unpinned."""
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


def test_two_keys_ln3_gives_three_to_one(port):
    """Closed form that fixes the scale: with q.k1 - q.k2 = sqrt(128) ln 3 the
    softmax weights are exactly 3/4 and 1/4.  A missing or wrong 1/sqrt(128)
    (1/128, 1/sqrt(64), none) moves them far from that."""
    k = np.zeros((2, 8, 128), dtype=np.uint16)
    v = np.zeros((2, 8, 128), dtype=np.uint16)
    k[0, :, 0] = f16_bits(1.0)  # key 0 of every KV head: e_0; key 1: zero
    v[0, :, :] = f16_bits(4.0)
    v[1, :, :] = f16_bits(-4.0)
    pool = pool_rows(k, v).view(np.uint8)
    q = np.zeros((32, 128), dtype=np.float32)
    q[:, 0] = np.float32(np.sqrt(128.0) * np.log(3.0))
    out = port.attention(q, pool, [[0, 1]] * 32)
    # 3/4 * 4 + 1/4 * (-4) = 2, up to the F32 rounding of q (relative 6e-8)
    assert np.allclose(out, 2.0, rtol=0, atol=1e-6)


def test_kv_head_marker(port):
    """Query head h reads KV head h // 4 for both K and V: KV head g's key 0
    scores g ln 2 above its key 1 (so weights 2^g : 1), and its V rows carry g.
    A mapping h % 8 or h // 8 gives other weights and values."""
    k = np.zeros((2, 8, 128), dtype=np.uint16)
    v = np.zeros((2, 8, 128), dtype=np.uint16)
    for g in range(8):
        k[0, g, 0] = f16_bits(float(g))
        v[0, g, :] = f16_bits(float(g + 1))
        v[1, g, :] = f16_bits(-float(g + 1))
    pool = pool_rows(k, v).view(np.uint8)
    q = np.zeros((32, 128), dtype=np.float32)
    q[:, 0] = np.float32(np.sqrt(128.0) * np.log(2.0))
    out = port.attention(q, pool, [[0, 1]] * 32)
    for h in range(32):
        g = h // 4
        w = 2.0**g / (2.0**g + 1.0)
        expect = (g + 1) * (2.0 * w - 1.0)
        assert np.allclose(out[h], expect, rtol=0, atol=1e-6), (h, out[h][0], expect)


def test_matches_torch_gqa_attention(port):
    """FP64 against torch's scaled_dot_product_attention on the CPU, which
    states the scale (1/sqrt(E)) and the GQA head mapping (enable_gqa: query
    head h uses KV head h // (32 / 8)) independently of the oracle.  Each
    query head's selection is a boolean mask over the union of ids."""
    import torch

    g = rng(11)
    n = 400
    k, v, pool = make_pool(g, n)
    q = (3.0 * g.standard_normal((32, 128))).astype(np.float32)
    ids = [sorted(g.choice(n, size=int(g.integers(1, 120)), replace=False).tolist())
           for _ in range(32)]
    got = port.attention(q, pool, ids)
    kf = torch.from_numpy(k.view(np.float16).astype(np.float64)).permute(1, 0, 2)[None]
    vf = torch.from_numpy(v.view(np.float16).astype(np.float64)).permute(1, 0, 2)[None]
    qf = torch.from_numpy(q.astype(np.float64))[None, :, None, :]
    mask = torch.zeros((1, 32, 1, n), dtype=torch.bool)
    for h in range(32):
        mask[0, h, 0, ids[h]] = True
    ref = torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, attn_mask=mask,
                                                           enable_gqa=True)
    ref = ref[0, :, 0, :].numpy()
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
