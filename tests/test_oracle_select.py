"""Pins of the selector restatement (oracle, CPU).

Known answers are the reference's own: tests/gqa_policy_tests.cpp:46-80 and
tests/quality_alpha_tests.cpp:32-77.  Random cases are checked against a
brute-force (value desc, id asc) sort and the compiled reference.
"""
import numpy as np
import pytest

import oracle
from hs_data import f16_bits, rng

OK, SHAPE, NONFINITE, THRESHOLD, COUNT, MEAN = 0, 1, 2, 3, 4, 5


def hb(x):
    return int(np.float16(x).view(np.uint16))


def sel(port, scores, heads, stride, n, alpha, ratio, fp32=False):
    return port.select(np.asarray(scores, dtype=np.uint16), heads, stride, n, alpha, ratio, fp32)


def test_head0_broadcast_inclusive(port):
    s = [hb(x) for x in [10, 9, 8, 7, 1, 1, 1, 1]]
    rc, k, ids, counts, _ = sel(port, s, 2, 4, 4, 2.0, 1.0)
    assert rc == OK and list(counts) == [3, 0] and k == 1
    assert ids[0][0] == 0 and ids[1][0] == 0


def test_padding_excluded(port):
    s = np.full(16, hb(1000), dtype=np.uint16)
    for h in range(2):
        for t in range(5):
            s[h * 8 + t] = hb(t)
    rc, k, ids, _, _ = sel(port, s, 2, 8, 5, 10, 0.4)
    assert rc == OK and k == 2 and list(ids[0]) == [4, 3]


def test_f16_count_rounding_2049(port):
    many = np.full(2049, hb(0), dtype=np.uint16)
    rc, k, _, counts, _ = sel(port, many, 1, 2049, 2049, 0, 1)
    assert rc == OK and counts[0] == 2049 and k == 2048
    rc, k, _, _, _ = sel(port, many, 1, 2049, 2049, 0, 1, fp32=True)
    assert rc == OK and k == 2049


def test_long_id_indexing(port):
    s = np.full(131072, hb(-10), dtype=np.uint16)
    s[-1] = hb(1)
    rc, k, ids, _, _ = sel(port, s, 1, 131072, 131072, 0, 1)
    assert rc == OK and k == 1 and ids[0][0] == 131071


def test_count_overflow_and_fp32_extension(port):
    over = np.full(65520, hb(0), dtype=np.uint16)
    rc, *_ = sel(port, over, 1, 65520, 65520, 0, 1)
    assert rc == COUNT
    rc, k, ids, counts, _ = sel(port, over, 1, 65520, 65520, 0, 0.2, fp32=True)
    assert rc == OK and counts[0] == 65520 and k == 13104
    assert ids[0][0] == 0 and ids[0][-1] == 13103


def test_quality_alpha_ladder(port):
    # quality_alpha_tests.cpp:35-47: scores 100-2t; alpha -> k and counts
    P = 128
    s = np.array([[hb(100 - 2 * t) for t in range(P)] for _ in range(32)], dtype=np.uint16)
    for alpha, kk, cc in [(5, 3, 3), (10, 6, 6), (20, 11, 11), (50, 25, 26)]:
        rc, k, ids, counts, _ = sel(port, s, 32, P, P, alpha, 0.2)
        assert rc == OK and k == kk and np.all(counts == cc)
        assert np.all(ids == np.arange(k))


@pytest.mark.parametrize("alpha", [5.0, 10.0, 20.0, 50.0])
def test_threshold_equality_and_raised_head0(port, alpha):
    # quality_alpha_tests.cpp:49-67
    P = 128
    s = np.full((32, P), hb(-1000), dtype=np.uint16)
    thr_bits = hb(100 - alpha)
    s[:, 0] = hb(100)
    s[:, 1] = thr_bits
    s[:, 2] = thr_bits
    s[:, 3] = thr_bits - 1
    rc, k, ids, counts, _ = sel(port, s, 32, P, P, alpha, 0.2)
    assert rc == OK and k == 3 and counts[0] == 3 and list(ids[0]) == [0, 1, 2]
    s[0, 0] = hb(120)
    rc, k, ids, counts, _ = sel(port, s, 32, P, P, alpha, 0.2)
    new_thr = np.float16(np.float32(120) - np.float32(alpha)).astype(np.float32)
    assert rc == OK and counts[1] == int(np.float32(100) >= new_thr)


@pytest.mark.parametrize("alpha", [5.0, 10.0, 20.0, 50.0])
def test_count_rounding_at_16k(port, alpha):
    # quality_alpha_tests.cpp:70-77
    N = 16384
    s = np.full((32, N), hb(-1000), dtype=np.uint16)
    s[:, :2049] = hb(0)
    rc, k, ids, counts, _ = sel(port, s, 32, N, N, alpha, 0.2)
    assert rc == OK and k == 2048 and counts[0] == 2049 and ids[0][-1] == 2047


def test_random_orders_against_brute_force(port):
    # gqa_policy_tests.cpp:70-80: ties, signed zeros and padding columns
    g = rng(1741)
    heads, n, stride = 32, 257, 288
    for _ in range(24):
        s = np.full((heads, stride), hb(1000), dtype=np.uint16)
        vals = (g.integers(0, 97, size=(heads, n)) - 48) / 2.0
        s[:, :n] = f16_bits(vals)
        t = np.arange(n)
        zero = (t % 17 == 0)
        s[:, :n][:, zero] = np.where(t[zero] % 2, 0, 0x8000).astype(np.uint16)
        rc, k, ids, _, _ = sel(port, s, heads, stride, n, 10, 0.2)
        assert rc == OK
        for h in range(heads):
            v = s[h, :n].view(np.float16).astype(np.float64)
            expected = np.lexsort((t, -v))[:k]
            assert np.array_equal(ids[h], expected)


def test_error_precedence(port):
    s = np.full((2, 8), hb(1), dtype=np.uint16)
    s[1, 3] = 0x7C00
    assert sel(port, s, 2, 8, 8, 1, 0.5)[0] == NONFINITE
    s[1, 3] = hb(1)
    s[0, 5] = 0xFE00  # NaN in head 0
    assert sel(port, s, 2, 8, 8, 1, 0.5)[0] == NONFINITE
    low = np.full((1, 4), hb(-65504), dtype=np.uint16)
    assert sel(port, low, 1, 4, 4, 100.0, 1)[0] == THRESHOLD
    assert sel(port, low, 1, 4, 4, -1.0, 1)[0] == SHAPE
    assert sel(port, low, 1, 4, 4, 1.0, 0.0)[0] == SHAPE
    assert sel(port, low, 1, 4, 5, 1.0, 0.5)[0] == SHAPE


@pytest.mark.parametrize("n,alpha", [(4096, 0.1), (4096, 1.0), (4096, 5.0), (32768, 5.0),
                                     (32768, 2.0), (3000, 3.0)])
def test_matches_compiled_reference(port, ref, n, alpha):
    g = rng(n + int(alpha * 10))
    raw = f16_bits(g.standard_normal((32, n)) * 20.0)
    scaled = port.scale(raw)
    a = port.select(scaled, 32, n, n, alpha, 0.2)
    b = ref.select(scaled, 32, n, n, alpha, 0.2, width=n)
    assert a[0] == 0 and b[0] == 0
    assert a[1] == b[1]
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3]) and a[4] == b[4]


def test_ties_and_signed_zero_against_reference(port, ref):
    g = rng(5)
    n = 2000
    s = f16_bits(g.integers(-3, 4, size=(32, n)).astype(np.float64))
    s[g.random((32, n)) < 0.3] = 0x8000
    a = port.select(s, 32, n, n, 3.0, 0.5)
    b = ref.select(s, 32, n, n, 3.0, 0.5, width=n)
    assert a[1] == b[1] and np.array_equal(a[2], b[2]) and a[4] == b[4] and a[4] > 0
