"""GPU parity of the history cover (HS_SELECT_COVER, prefetch_payload of
policy/full_gqa_runtime.cpp:299-344) against the oracle: exact bound, each
head's ordered cover ids and the union; error codes; and, at full size, the
reference's guarantee that the final selection over position + 1 columns
stays inside the cover (tests/full_gqa_prefetch_tests.cpp:231-233)."""
import math

import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, rng, to_dev

pytestmark = pytest.mark.gpu


def gpu_cover(hs, raw, heads, stride, position, alpha, ratio=0.2, fp32=False, partial=None):
    s = to_dev(np.ascontiguousarray(raw, dtype=np.uint16).reshape(-1))
    words = (position + 31) // 32
    member = torch.zeros((heads, words), dtype=torch.int32, device="cuda")
    ids, counts, member, status = hs.ops.select(s, heads, stride, position, alpha, ratio,
                                                scale_raw=True, fp32_counts=fp32, cover=True,
                                                head0_partial=partial, member=member)
    st = hs.ops.read_status(status)
    k = st["k"]
    bits = from_dev(member).view(np.uint32)
    union = np.nonzero(np.unpackbits(np.bitwise_or.reduce(bits, axis=0).view(np.uint8),
                                     bitorder="little"))[0]
    return st, from_dev(ids)[:, :k], union


def check(hs, port, raw, heads, stride, position, alpha, fp32=False):
    rc, bound, ids, physical = port.history_cover(raw, heads, stride, position, alpha,
                                                  fp32_counts=fp32)
    st, gids, union = gpu_cover(hs, raw, heads, stride, position, alpha, fp32=fp32)
    assert st["code"] == rc
    if rc == 0:
        assert st["k"] == bound
        assert np.array_equal(gids, ids)
        assert np.array_equal(union, physical)
    return st


@pytest.mark.parametrize("heads,position", [(32, 63), (32, 1000), (8, 4095), (32, 32767),
                                            (4, 40000)])
@pytest.mark.parametrize("alpha", [0.5, 2.0, 1000.0])
def test_matches_oracle(hs, port, heads, position, alpha):
    g = rng(position + int(alpha * 10))
    stride = position + 1
    raw = f16_bits(g.standard_normal((heads, stride)) * 40.0)
    check(hs, port, raw, heads, stride, position, alpha)


@pytest.mark.parametrize("fp32", [False, True])
def test_fp32_counts_and_sparse(hs, port, fp32):
    heads, position = 32, 3000
    raw = np.full((heads, position + 1), f16_bits(-50.0), dtype=np.uint16)
    for h in range(heads):
        for j in range(7):
            raw[h, 100 + 97 * j + h] = f16_bits(100.0 + j)
    st = check(hs, port, raw, heads, position + 1, position, 1.0, fp32)
    assert st["k"] == 8


def test_nonfinite_handling(hs, port):
    g = rng(5)
    heads, position = 32, 2048
    raw = f16_bits(g.standard_normal((heads, position + 1)) * 30.0)
    raw[0, 17] = 0x7E00   # NaN in head 0: skipped by the maximum
    raw[3, 5] = 0x7E00    # NaN elsewhere: counts as below, ranks by its key
    raw[4, 9] = 0xFC00    # -inf
    raw[5, 11] = 0x7C00   # +inf in another head: counts, ranks first
    check(hs, port, raw, heads, position + 1, position, 2.0)
    bad = raw.copy()
    bad[0, 100] = 0x7C00  # +inf in head 0: nonfinite threshold
    st = check(hs, port, bad, heads, position + 1, position, 2.0)
    assert st["code"] == hs.HS_ERR_THRESHOLD


def test_cap_zero_rejected(hs):
    raw = to_dev(np.zeros((4, 8), dtype=np.uint16).reshape(-1))
    with pytest.raises(hs.HsError):
        hs.ops.select(raw, 4, 8, 1, 1.0, 0.2, scale_raw=True, cover=True)


def test_cover_contains_final_selection_full_size(hs):
    # N = 32768 history, then the current token appended (three different
    # current scores): every final historical id is in its head's cover
    heads, position = 32, 32767
    stride = position + 1
    q = torch.empty(4096, dtype=torch.float16, device="cuda")
    keys = torch.empty(stride * 1024, dtype=torch.float16, device="cuda")
    hs.ops.fill_gaussian(q, seed=41)
    hs.ops.fill_rope_keys(keys, stride, 1024, 8, seed=42, theta=500000.0)
    raw = hs.ops.score(q, keys, stride)
    partial = torch.empty((position + 63) // 64, dtype=torch.int32, device="cuda")
    hs.ops.score(q, keys, position, out=torch.empty((heads, position), dtype=torch.float16,
                                                   device="cuda"), head0_partial=partial)
    kmax = min(position, math.floor((position + 1) * float(np.float32(0.2))))
    ids, _, member, status = hs.ops.select(raw, heads, stride, position, 5.0, 0.2,
                                           scale_raw=True, cover=True, head0_partial=partial)
    st = hs.ops.read_status(status)
    assert st["code"] == 0 and 1 <= st["k"] <= kmax
    cover = from_dev(ids)[:, : st["k"]]
    for value in (None, 60000.0, -60000.0):
        final = raw.clone()
        if value is not None:
            final[:, position] = value
        fids, _, _, fstatus = hs.ops.select(final, heads, stride, stride, 5.0, 0.2,
                                            scale_raw=True)
        fst = hs.ops.read_status(fstatus)
        assert fst["code"] == 0
        fk = fst["k"]
        got = from_dev(fids)[:, :fk]
        for h in range(heads):
            hist = got[h][got[h] < position]
            assert np.isin(hist, cover[h]).all(), (value, h)
