"""Pins of the history-cover restatement (oracle, CPU).

prefetch_payload (policy/full_gqa_runtime.cpp:299-344) selects, before the
current token exists, a per-head history cover of size `bound`.  The
reference's own test (tests/full_gqa_prefetch_tests.cpp:150-258) checks:
  * every final selection over position + 1 columns keeps its historical ids
    inside the cover of its head ("threshold-count bounded history covers
    final ordered selection"), whatever the current token scores;
  * the bound equals the cap when the threshold admits everything, and is
    m + 1 when exactly m historical tokens per head reach the threshold
    ("F16 threshold-count upper bound includes unknown current contribution");
  * every id is historical (< position) and the union is sorted.
The reference function itself needs nlohmann/json.hpp (absent), so these
properties, the selector oracle (pinned by its own KATs and the compiled
reference) and a pure-Python sort are what pin hso_history_cover.
"""
import math

import numpy as np
import pytest

import oracle
from hs_data import f16_bits, rng

OK, SHAPE, NONFINITE, THRESHOLD, COUNT, MEAN = 0, 1, 2, 3, 4, 5


def cap_of(position, ratio=0.2):
    return min(position, math.floor((position + 1) * float(np.float32(ratio))))


def python_cover(port, raw, heads, stride, position, alpha, fp32=False):
    """The same algorithm in plain Python (small sizes only)."""
    scaled = [[port.scale(np.array([raw[h, t]], dtype=np.uint16))[0] for t in range(position)]
              for h in range(heads)]
    val = lambda b: float(np.uint16(b).view(np.float16))
    maximum = -math.inf
    for b in scaled[0]:
        x = val(b)
        if maximum < x:  # std::max keeps the left operand on NaN
            maximum = x
    thr = float(np.float16(np.float32(maximum) - np.float32(alpha)))
    assert math.isfinite(thr)
    total = np.float32(0)
    for h in range(heads):
        c = 1 + sum(1 for b in scaled[h] if val(b) >= thr)
        total = np.float32(total + (np.float32(c) if fp32 else np.float32(np.float16(c))))
    q = np.float32(total / np.float32(heads))
    mean = q if fp32 else np.float32(np.float16(q))
    bound = min(cap_of(position), int(mean))
    ids = []
    for h in range(heads):
        order = sorted(range(position), key=lambda t: (-port.order_key(int(scaled[h][t])), t))
        ids.append(order[:bound])
    return bound, ids


def random_raw(g, heads, stride, scale=3.0):
    return f16_bits(g.standard_normal((heads, stride)) * scale)


@pytest.mark.parametrize("seed,position,alpha", [(1, 40, 1.0), (2, 63, 0.5), (3, 97, 2.5)])
def test_matches_python_restatement(port, seed, position, alpha):
    g = rng(seed)
    heads, stride = 8, position + 3
    raw = random_raw(g, heads, stride)
    rc, bound, ids, physical = port.history_cover(raw, heads, stride, position, alpha)
    assert rc == OK
    pb, pids = python_cover(port, raw, heads, stride, position, alpha)
    assert bound == pb
    for h in range(heads):
        assert list(ids[h]) == pids[h]
    assert list(physical) == sorted(set(t for h in range(heads) for t in pids[h]))


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("fp32", [False, True])
def test_cover_contains_final_selection(port, seed, fp32):
    # full_gqa_prefetch_tests.cpp:231-233: the final selection after the
    # current token is appended stays inside the cover, for any current scores
    g = rng(100 + seed)
    heads, position = 32, 500 + 37 * seed
    stride = position + 1
    alpha = [0.25, 1.0, 3.0][seed % 3]
    raw = random_raw(g, heads, stride, scale=2.0 + seed)
    rc, bound, cover, physical = port.history_cover(raw, heads, stride, position, alpha,
                                                    fp32_counts=fp32)
    assert rc == OK and 1 <= bound <= cap_of(position)
    assert all(t < position for t in physical) and list(physical) == sorted(set(physical))
    for trial in range(4):
        final = raw.copy()
        if trial == 0:  # the current token raises head 0's maximum
            final[:, position] = f16_bits(np.full(heads, 40.0))
        elif trial == 1:  # it lowers nothing and sits at the bottom
            final[:, position] = f16_bits(np.full(heads, -40.0))
        else:
            final[:, position] = random_raw(g, heads, 1, scale=6.0)[:, 0]
        scaled = port.scale(final.reshape(-1)).reshape(final.shape)
        rc2, k, ids, _, _ = port.select(scaled, heads, stride, position + 1, alpha, 0.2, fp32)
        assert rc2 == OK
        for h in range(heads):
            hist = set(int(t) for t in ids[h] if t < position)
            assert hist <= set(int(t) for t in cover[h]), (seed, trial, h)


def test_bound_is_cap_when_threshold_admits_all(port):
    g = rng(7)
    heads, position = 32, 300
    raw = random_raw(g, heads, position + 1)
    rc, bound, ids, physical = port.history_cover(raw, heads, position + 1, position, 1000.0)
    assert rc == OK and bound == cap_of(position) == 60
    assert all(len(r) == 60 for r in ids)


@pytest.mark.parametrize("m", [1, 3, 9])
def test_sparse_threshold_bound(port, m):
    # exactly m historical tokens per head reach the threshold -> each count
    # is m + 1 (exact in F16), so the mean and the bound are m + 1 (the
    # reference's "constructed sparse threshold" case, full_gqa_prefetch_tests.cpp:200-205)
    heads, position = 32, 400
    raw = np.full((heads, position + 1), f16_bits(-50.0), dtype=np.uint16)
    for h in range(heads):
        for j in range(m):
            raw[h, 17 + 31 * j + h] = f16_bits(100.0 + j)  # within alpha of the top
    rc, bound, ids, physical = port.history_cover(raw, heads, position + 1, position, 1.0)
    assert rc == OK and bound == m + 1 < cap_of(position)
    for h in range(heads):
        assert set(ids[h][:m]) == {17 + 31 * j + h for j in range(m)}


def test_single_top_token(port):
    # head 0 alone has one token above the rest: counts 2, 1, 1, ... -> the
    # mean F16(33/32) truncates to 1
    heads, position = 32, 400
    raw = np.full((heads, position + 1), f16_bits(-50.0), dtype=np.uint16)
    raw[0, 5] = f16_bits(100.0)
    rc, bound, ids, _ = port.history_cover(raw, heads, position + 1, position, 1.0)
    assert rc == OK and bound == 1 and ids[0][0] == 5


def test_nan_skipped_by_head0_max(port):
    g = rng(9)
    heads, position = 4, 64
    raw = random_raw(g, heads, position + 1)
    base = port.history_cover(raw, heads, position + 1, position, 1.0)
    with_nan = raw.copy()
    with_nan[0, 10] = 0x7E00  # NaN: std::max keeps the running maximum
    with_nan[2, 11] = 0x7E00  # NaN elsewhere never counts
    rc, bound, ids, _ = port.history_cover(with_nan, heads, position + 1, position, 1.0)
    assert rc == OK and base[0] == OK
    pb, pids = python_cover(port, with_nan, heads, position + 1, position, 1.0)
    assert bound == pb and all(list(ids[h]) == pids[h] for h in range(heads))


def test_errors(port):
    heads = 4
    raw = np.zeros((heads, 65), dtype=np.uint16)
    # cap == 0 at position 1: floor(2 * 0.2f) = 0 (:309-311)
    assert port.history_cover(raw, heads, 65, 1, 1.0)[0] == SHAPE
    # position must leave room for the current token (position < capacity)
    assert port.history_cover(raw, heads, 65, 65, 1.0)[0] == SHAPE
    # +inf in head 0: the threshold is not finite (:316)
    bad = raw.copy()
    bad[0, 3] = 0x7C00
    assert port.history_cover(bad, heads, 65, 64, 1.0)[0] == THRESHOLD
    # every head-0 score NaN: the maximum stays -inf
    nan = raw.copy()
    nan[0, :] = 0x7E00
    assert port.history_cover(nan, heads, 65, 64, 1.0)[0] == THRESHOLD
