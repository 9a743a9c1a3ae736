"""GPU parity of kernel #2 (selection) against the oracle: exact k, counts,
ordered ids and boundary ties; error codes with the reference's precedence."""
import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, rng, to_dev

pytestmark = pytest.mark.gpu


def hb(x):
    return int(np.float16(x).view(np.uint16))


def gpu_select(hs, scores, heads, stride, n, alpha, ratio, **kw):
    s = to_dev(np.ascontiguousarray(scores, dtype=np.uint16).reshape(-1))
    ids, counts, member, status = hs.ops.select(s, heads, stride, n, alpha, ratio, **kw)
    st = hs.ops.read_status(status)
    k = st["k"]
    return st, from_dev(ids)[:, :k], from_dev(counts), member


def check_against_port(hs, port, scores, heads, stride, n, alpha, ratio, fp32=False):
    rc, k, ids, counts, tied = port.select(scores, heads, stride, n, alpha, ratio, fp32)
    # rank order (the reference's output) and ascending id order (same set)
    for id_order in (False, True):
        st, gids, gcounts, _ = gpu_select(hs, scores, heads, stride, n, alpha, ratio,
                                          fp32_counts=fp32, id_order=id_order)
        assert st["code"] == rc, id_order
        if rc == 0:
            assert st["k"] == k
            assert np.array_equal(gcounts, counts)
            want = np.sort(ids, axis=1) if id_order else ids
            assert np.array_equal(gids, want), f"ids differ (id_order={id_order})"
            assert st["boundary_tied_heads"] == tied
    return st


def test_known_answers(hs, port):
    s = np.array([hb(x) for x in [10, 9, 8, 7, 1, 1, 1, 1]], dtype=np.uint16)
    st, ids, counts, _ = gpu_select(hs, s, 2, 4, 4, 2.0, 1.0)
    assert st["code"] == 0 and st["k"] == 1 and list(counts) == [3, 0]
    assert ids[0][0] == 0 and ids[1][0] == 0
    pad = np.full(16, hb(1000), dtype=np.uint16)
    for h in range(2):
        for t in range(5):
            pad[h * 8 + t] = hb(t)
    st, ids, _, _ = gpu_select(hs, pad, 2, 8, 5, 10, 0.4)
    assert st["k"] == 2 and list(ids[0]) == [4, 3]
    many = np.full(2049, hb(0), dtype=np.uint16)
    st, _, counts, _ = gpu_select(hs, many, 1, 2049, 2049, 0, 1)
    assert counts[0] == 2049 and st["k"] == 2048
    st, _, _, _ = gpu_select(hs, many, 1, 2049, 2049, 0, 1, fp32_counts=True)
    assert st["k"] == 2049
    # global long-token id not truncated (131072 candidates, 32 slices)
    long_scores = np.full(131072, hb(-10), dtype=np.uint16)
    long_scores[-1] = hb(1)
    for id_order in (False, True):
        st, ids, _, _ = gpu_select(hs, long_scores, 1, 131072, 131072, 0, 1, id_order=id_order)
        assert st["code"] == 0 and st["k"] == 1 and ids[0][0] == 131071


def test_quality_alpha_ladder(hs):
    P = 128
    s = np.array([[hb(100 - 2 * t) for t in range(P)] for _ in range(32)], dtype=np.uint16)
    for alpha, kk, cc in [(5, 3, 3), (10, 6, 6), (20, 11, 11), (50, 25, 26)]:
        st, ids, counts, _ = gpu_select(hs, s, 32, P, P, alpha, 0.2)
        assert st["k"] == kk and np.all(counts == cc) and np.all(ids == np.arange(kk))


def test_count_rounding_16k(hs):
    N = 16384
    s = np.full((32, N), hb(-1000), dtype=np.uint16)
    s[:, :2049] = hb(0)
    st, ids, counts, _ = gpu_select(hs, s, 32, N, N, 10.0, 0.2)
    assert st["k"] == 2048 and counts[0] == 2049 and ids[0][-1] == 2047


def test_random_orders(hs, port):
    g = rng(1741)
    heads, n, stride = 32, 257, 288
    for _ in range(6):
        s = np.full((heads, stride), hb(1000), dtype=np.uint16)
        s[:, :n] = f16_bits((g.integers(0, 97, size=(heads, n)) - 48) / 2.0)
        t = np.arange(n)
        zero = t % 17 == 0
        s[:, :n][:, zero] = np.where(t[zero] % 2, 0, 0x8000).astype(np.uint16)
        check_against_port(hs, port, s, heads, stride, n, 10, 0.2)


@pytest.mark.parametrize("n,alpha,ratio", [(4096, 0.1, 0.2), (4096, 1.0, 0.2), (4096, 5.0, 0.2),
                                           (32768, 5.0, 0.2), (32768, 2.5, 0.2),
                                           (3001, 3.0, 0.5), (65536, 5.0, 0.2)])
def test_gaussian_against_oracle(hs, port, n, alpha, ratio):
    g = rng(n + int(alpha * 100))
    raw = f16_bits(g.standard_normal((32, n)) * 20.0)
    scaled = port.scale(raw)
    st = check_against_port(hs, port, scaled, 32, n, n, alpha, ratio)
    assert st["code"] == 0


def test_heavy_ties_and_signed_zero(hs, port):
    g = rng(5)
    n = 2000
    s = f16_bits(g.integers(-3, 4, size=(32, n)).astype(np.float64))
    s[g.random((32, n)) < 0.3] = 0x8000
    st = check_against_port(hs, port, s, 32, n, n, 3.0, 0.5)
    assert st["boundary_tied_heads"] > 0


def test_zero_key_boundary_bits(hs, port):
    # boundary tie decided on raw bits: +0 then -0 at the cut is not "tied"
    n = 64
    s = np.full((1, n), hb(-5), dtype=np.uint16)
    s[0, :3] = hb(1)
    s[0, 3] = 0x0000
    s[0, 4] = 0x8000
    for ratio in (4 / 64, 5 / 64):
        check_against_port(hs, port, s, 1, n, n, 10.0, ratio)


def order_keys(bits):
    b = np.asarray(bits, dtype=np.uint32)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)


@pytest.mark.parametrize("case", ["counting", "full_k", "wide_range", "long_run", "full_k_long_run"])
def test_rank_order_placement_paths(hs, port, case):
    # The per-head rank order places the selection by a counting sort over
    # the 8192 keys from K*'s 256-key bucket upward, and falls back to a radix
    # sort when a selected key lies past them or more than 64 selected keys
    # are equal.  Each case is checked (on the oracle's selection) to take
    # the path it names.  full_k selects the most a per-head workgroup holds
    # (k = 8192): the counting sort's lists, or the radix sort's two
    # buffers (full_k_long_run), then fill its LDS.
    g = rng({"counting": 21, "full_k": 24, "wide_range": 22, "long_run": 23, "full_k_long_run": 25}[case])
    heads, n = 4, 32768
    if case == "wide_range":
        # 30 % of the tokens spread over every positive normal key, the rest
        # -1: the selected quarter spans about 25000 keys
        s = np.full((heads, n), hb(-1.0), dtype=np.uint16)
        spread = g.random((heads, n)) < 0.3
        s[spread] = g.integers(0x0400, 0x7BFF, size=int(spread.sum())).astype(np.uint16)
        alpha, ratio = 70000.0, 0.25
    else:
        s = f16_bits(g.standard_normal((heads, n)) * 2.0)
        if case in ("long_run", "full_k_long_run"):
            s[:, 1000:1100] = hb(9.5)  # 100 equal keys at the top of every head
        # full_k: every key within alpha of the maximum, so k = the cap n / 4
        alpha, ratio = (100.0, 0.25) if case.startswith("full_k") else (5.0, 0.2)
    rc, k, ids, _, _ = port.select(s, heads, n, n, alpha, ratio)
    assert rc == 0 and k <= 8192
    if case.startswith("full_k"):
        assert k == 8192
    keys = order_keys(s[np.arange(heads)[:, None], ids])
    kstar = keys.min(axis=1)
    span = keys.max(axis=1) - (kstar & 0xFF00)
    run = max(np.unique(row, return_counts=True)[1].max() for row in keys)
    if case in ("counting", "full_k"):
        assert (span < 8192).all() and run <= 64
    elif case == "wide_range":
        assert (span >= 8192).any()
    else:  # long_run, full_k_long_run
        assert (span < 8192).all() and run > 64
    check_against_port(hs, port, s, heads, n, n, alpha, ratio)


def test_large_k_global_sort(hs, port):
    n = 40000
    g = rng(9)
    s = f16_bits(g.standard_normal((4, n)))
    st = check_against_port(hs, port, s, 4, n, n, 30.0, 1.0)
    assert st["k"] > 16384


def test_scale_raw_with_scorer_partials(hs, port):
    from hs_data import v3_sample, config1_inputs
    q, k, _ = config1_inputs(3, n=2048)
    n = 2048
    partial = torch.zeros(n // 64, dtype=torch.int32, device="cuda")
    raw_dev = hs.ops.score(to_dev(q), to_dev(k.reshape(-1)), n, head0_partial=partial)
    raw = from_dev(raw_dev)
    assert np.array_equal(raw, port.score(q, k.reshape(-1), n))
    scaled = port.scale(raw)
    rc, kk, ids, counts, tied = port.select(scaled, 32, n, n, 1.0, 0.2)
    ids_d, counts_d, member, status = hs.ops.select(raw_dev, 32, n, n, 1.0, 0.2, scale_raw=True,
                                                    head0_partial=partial)
    st = hs.ops.read_status(status)
    assert st["code"] == 0 and st["k"] == kk
    assert np.array_equal(from_dev(ids_d)[:, :kk], ids)
    assert np.array_equal(from_dev(counts_d), counts)


def test_member_bitmaps(hs, port):
    n = 1000
    g = rng(21)
    s = f16_bits(g.standard_normal((32, n)))
    words = (n + 31) // 32
    member = torch.zeros(32 * words, dtype=torch.int32, device="cuda")
    ids, _, _, status = hs.ops.select(to_dev(s.reshape(-1)), 32, n, n, 2.0, 0.2, member=member)
    st = hs.ops.read_status(status)
    bits = from_dev(member).reshape(32, words)
    got = from_dev(ids)[:, : st["k"]]
    for h in range(32):
        expected = np.zeros(words, dtype=np.uint32)
        for i in got[h]:
            expected[i >> 5] |= np.uint32(1) << np.uint32(i & 31)
        assert np.array_equal(bits[h], expected)


def test_error_codes(hs):
    s = np.full((2, 8), hb(1), dtype=np.uint16)
    s[1, 3] = 0x7C00
    assert gpu_select(hs, s, 2, 8, 8, 1, 0.5)[0]["code"] == hs.HS_ERR_NONFINITE
    s[1, 3] = hb(1)
    s[0, 5] = 0xFE00
    assert gpu_select(hs, s, 2, 8, 8, 1, 0.5)[0]["code"] == hs.HS_ERR_NONFINITE
    low = np.full((1, 4), hb(-65504), dtype=np.uint16)
    assert gpu_select(hs, low, 1, 4, 4, 100.0, 1)[0]["code"] == hs.HS_ERR_THRESHOLD
    over = np.full(65520, hb(0), dtype=np.uint16)
    assert gpu_select(hs, over, 1, 65520, 65520, 0, 1)[0]["code"] == hs.HS_ERR_COUNT
    st, ids, counts, _ = gpu_select(hs, over, 1, 65520, 65520, 0, 0.2, fp32_counts=True)
    assert st["code"] == 0 and st["k"] == 13104 and ids[0][0] == 0 and ids[0][-1] == 13103
    tiny = np.full((32, 64), hb(-100), dtype=np.uint16)
    tiny[0, 0] = hb(100)
    st = gpu_select(hs, tiny, 32, 64, 64, 1.0, 0.2, require_k=True)[0]
    assert st["code"] == hs.HS_ERR_ZERO_SELECTION
    st = gpu_select(hs, tiny, 32, 64, 64, 1.0, 0.2)[0]
    assert st["code"] == 0 and st["k"] == 0
    with pytest.raises(hs.HsError):
        gpu_select(hs, tiny, 32, 64, 64, -1.0, 0.2)


def test_scaling_edge_inputs_order(hs, port):
    # Raw scores whose scaled F16 value depends on rounding the FP32 quotient
    # first (the 52 mantissa-0x0a5 inputs and neighbours): with scale_raw the
    # full order (ratio 1) must match the oracle exactly, ties included.
    specials = [e << 10 | 0x0A5 for e in range(1, 30)]
    vals = sorted({v + d for v in specials for d in (-1, 0, 1)} |
                  {0x8000 | v for v in specials})
    g = rng(52)
    n = len(vals) * 2
    rows = np.stack([g.permutation(np.array(vals * 2, dtype=np.uint16)) for _ in range(32)])
    scaled = port.scale(rows)
    rc, kk, pids, pcounts, tied = port.select(scaled, 32, n, n, 60000.0, 1.0)
    ids, counts, _, status = hs.ops.select(to_dev(rows.reshape(-1)), 32, n, n, 60000.0, 1.0,
                                           scale_raw=True)
    st = hs.ops.read_status(status)
    assert rc == 0 and st["code"] == 0 and st["k"] == kk == n
    assert np.array_equal(from_dev(ids)[:, :kk], pids)
    assert st["boundary_tied_heads"] == tied


def member_from_ids(ids, n):
    words = (n + 31) // 32
    out = np.zeros((ids.shape[0], words), dtype=np.uint32)
    for h in range(ids.shape[0]):
        np.bitwise_or.at(out[h], ids[h] >> 5, np.uint32(1) << (ids[h] & 31).astype(np.uint32))
    return out


@pytest.mark.parametrize("heads,n", [(1, 65536), (32, 65536), (64, 65536), (128, 65536),
                                     (8, 40000), (32, 4097), (3, 12345), (2, 131072),
                                     (128, 100000)])
def test_slices_and_run_lengths(hs, port, heads, n):
    # Every slicing of the head (1..16 slices, 8..64 ids per thread) with
    # coarse integer scores, so tie runs straddle slice boundaries; signed
    # zeros sit at the cut for some heads.
    g = rng(heads * 7919 + n)
    s = f16_bits(g.integers(-6, 7, size=(heads, n)).astype(np.float64))
    s[g.random((heads, n)) < 0.05] = 0x8000
    for alpha, ratio in ((3.0, 0.2), (0.5, 0.05), (12.0, 1.0)):
        rc, k, ids, counts, tied = port.select(s, heads, n, n, alpha, ratio)
        for id_order in (False, True):
            words = (n + 31) // 32
            member = torch.zeros(heads * words, dtype=torch.int32, device="cuda")
            st, gids, gcounts, _ = gpu_select(hs, s, heads, n, n, alpha, ratio, member=member,
                                              id_order=id_order)
            assert st["code"] == rc
            if rc != 0:  # e.g. a count of 65536 overflows F16 (HS_ERR_COUNT)
                continue
            assert st["k"] == k and st["boundary_tied_heads"] == tied
            assert np.array_equal(gcounts, counts)
            assert np.array_equal(gids, np.sort(ids, axis=1) if id_order else ids)
            bits = from_dev(member).view(np.uint32).reshape(heads, words)
            assert np.array_equal(bits, member_from_ids(ids, n))


def test_repeated_calls_share_workspace(hs, port):
    # One workspace across calls of different shapes, never cleared: every
    # launch writes what a later launch of the same call reads.
    ws = hs.ops.workspace(hs.ops.select_workspace_bytes(32, 32768))
    g = rng(77)
    for heads, n, alpha in ((32, 32768, 2.0), (32, 1000, 1.0), (4, 32768, 3.0), (32, 32768, 0.7),
                            (1, 64, 0.1)):
        raw = f16_bits(g.standard_normal((heads, n)) * 4.0)
        rc, k, ids, counts, tied = port.select(raw, heads, n, n, alpha, 0.2)
        for id_order in (True, False):
            dev_ids, dev_counts, _, status = hs.ops.select(
                to_dev(raw.reshape(-1)), heads, n, n, alpha, 0.2, ws=ws, id_order=id_order)
            st = hs.ops.read_status(status)
            assert st["code"] == rc and st["k"] == k
            got = from_dev(dev_ids)[:, :k]
            assert np.array_equal(got, np.sort(ids, axis=1) if id_order else ids)
            assert np.array_equal(from_dev(dev_counts), counts)


@pytest.mark.parametrize("n", [1000, 40000])
def test_failed_selection_clears_member(hs, n):
    # A failed selection leaves no stale bitmaps behind for an attention that
    # follows on the stream: the member words it was given are cleared
    # (per-head path and slice path).
    g = rng(22)
    s = f16_bits(g.standard_normal((32, n)))
    s[0, n // 2] = 0x7E00  # NaN in head 0: nonfinite head-0 score
    words = (n + 31) // 32
    member = torch.full((32 * words,), -1, dtype=torch.int32, device="cuda")
    for id_order in (False, True):
        member.fill_(-1)
        _, _, _, status = hs.ops.select(to_dev(s.reshape(-1)), 32, n, n, 2.0, 0.2, member=member,
                                        id_order=id_order)
        assert hs.ops.read_status(status)["code"] == hs.HS_ERR_NONFINITE
        assert not from_dev(member).any()


def test_random_sweep_against_oracle(hs, port):
    # seeded shapes and parameters across both launch paths: heads 1..128,
    # n up to 40000 (the slice chain past 32768), strides with padding,
    # quantized scores (ties) or Gaussian ones, FP32 counts on and off
    g = rng(9091)
    for case in range(12):
        heads = int(g.choice([1, 3, 8, 32, 100, 128]))
        n = int(g.integers(1, 40001)) if case % 3 else int(g.integers(1, 300))
        if heads * n > 2_000_000:
            n = 2_000_000 // heads
        stride = n + int(g.integers(0, 40))
        alpha = float(g.choice([0.0, 0.5, 2.0, 5.0, 8.0]))
        ratio = float(np.float32(g.choice([0.05, 0.2, 0.5, 1.0])))
        fp32 = bool(case % 2)
        s = np.full((heads, stride), hb(-60000), dtype=np.uint16)
        if case % 4 == 0:
            vals = (g.integers(0, 64, size=(heads, n)) - 32) / 4.0  # heavy ties
        else:
            vals = g.standard_normal((heads, n)) * 3.0
        s[:, :n] = f16_bits(vals)
        check_against_port(hs, port, s, heads, stride, n, alpha, ratio, fp32)


def test_per_head_sweep_against_oracle(hs, port):
    # the per-head launch (32 heads, n <= 32768) at every cap up to the
    # largest rank-order selection it holds (k <= 8192): tie-heavy, Gaussian,
    # narrow (long runs of equal F16 keys, the radix fallback) and wide (key
    # ranges past the counting table) scores, FP32 counts on and off
    g = rng(424242)
    for case in range(64):
        heads, n = 32, int(g.integers(500, 32769))
        stride = n + int(g.integers(0, 16))
        alpha = float(g.choice([0.0, 0.5, 2.0, 5.0, 8.0, 100.0]))
        ratio = float(np.float32(g.choice([0.05, 0.1, 0.2, 0.25])))
        s = np.full((heads, stride), hb(-60000), dtype=np.uint16)
        kind = case % 4
        if kind == 0:
            vals = (g.integers(0, 64, size=(heads, n)) - 32) / 4.0
        else:
            vals = g.standard_normal((heads, n)) * (3.0, 0.05, 30.0)[kind - 1]
        s[:, :n] = f16_bits(vals)
        check_against_port(hs, port, s, heads, stride, n, alpha, ratio, bool(case % 2))


def test_random_batch_sweep_against_oracle(hs, port):
    # a batch of 16 raw-score jobs with 16-byte aligned rows (four slices per
    # count group) and one with a ragged stride, each against the oracle over
    # its scaled scores
    g = rng(9092)
    for wide in (True, False):
        jobs, raws = [], []
        for i in range(16):
            n = int(g.integers(8, 32769))
            stride = -(-n // 8) * 8 if wide or i else n | 1
            raw = np.full((32, stride), hb(0), dtype=np.uint16)
            raw[:, :n] = f16_bits(g.standard_normal((32, n)) * 20.0)
            raws.append((raw, n, stride))
            jobs.append(dict(scores=to_dev(raw.reshape(-1)).view(32, stride), n=n))
        res = hs.ops.select_batched(jobs, 32, 3.0, 0.2, scale_raw=True)
        for (raw, n, stride), (ids, counts, _, status) in zip(raws, res):
            st = hs.ops.read_status(status)
            rc, k, pids, pcounts, tied = port.select(port.scale(raw), 32, stride, n, 3.0, 0.2)
            assert st["code"] == rc == 0
            assert st["k"] == k and st["boundary_tied_heads"] == tied
            assert np.array_equal(from_dev(counts), pcounts)
            assert np.array_equal(from_dev(ids)[:, :k], pids)
