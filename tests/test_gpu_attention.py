"""GPU sparse decode attention (kernel #4) against the FP64 oracle on the same
selection: relative error <= 2e-3."""
import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, pool_rows, rng, rope_keys, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3


def member_words(ids_rows, n):
    words = (n + 31) // 32
    m = np.zeros((32, words), dtype=np.uint32)
    for h, r in enumerate(ids_rows):
        r = np.asarray(r, dtype=np.int64)
        np.bitwise_or.at(m[h], r >> 5, (np.uint32(1) << (r & 31).astype(np.uint32)))
    return m


def rel_err(got, ref):
    num = np.linalg.norm(got - ref, axis=1)
    den = np.linalg.norm(ref, axis=1)
    return float(np.max(num / den))


@pytest.mark.parametrize("n,frac", [(257, 0.5), (4096, 0.2), (32768, 0.2), (40000, 0.05)])
def test_random_selection(hs, port, n, frac):
    g = rng(n)
    k = f16_bits(g.standard_normal((n, 8, 128)))
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [np.sort(g.choice(n, size=max(1, int(n * frac)), replace=False)) for _ in range(32)]
    member = member_words(ids, n)
    out = hs.ops.sparse_attention(torch.from_numpy(q).cuda(), to_dev(pool.reshape(-1)), n,
                                  to_dev(member.reshape(-1)))
    ref = port.attention(q, pool.view(np.uint8), ids)
    assert rel_err(out.cpu().numpy().astype(np.float64), ref) <= TOL


def test_row_map_and_peaked_softmax(hs, port):
    n = 5000
    g = rng(8)
    k = rope_keys(n, 8)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    perm = g.permutation(n).astype(np.int32)
    inv = np.argsort(perm)
    pool = pool_rows(k, v)[inv]  # row r holds id inv[r]; perm[id] = row
    q = (g.standard_normal((32, 128)) * 3.0).astype(np.float32)  # sharp softmax
    ids = [np.sort(g.choice(n, size=700, replace=False)) for _ in range(32)]
    member = member_words(ids, n)
    out = hs.ops.sparse_attention(torch.from_numpy(q).cuda(), to_dev(pool.reshape(-1)), n,
                                  to_dev(member.reshape(-1)), rows=to_dev(perm))
    ref = port.attention(q, pool.view(np.uint8).reshape(-1), ids, rows=perm)
    assert rel_err(out.cpu().numpy().astype(np.float64), ref) <= TOL


@pytest.mark.parametrize("mapped", [False, True])
def test_split_kv_arrays_equal_records(hs, port, mapped):
    # The hot pool as a K array and a V array (2048 B rows) reads the same
    # rows as the reference's 4096 B KV records: the output is the same bit
    # for bit, and within the tolerance of the oracle.
    n = 6000
    g = rng(90 + mapped)
    k = rope_keys(n, 9)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    records = pool_rows(k, v)
    rows = None
    if mapped:
        perm = g.permutation(n).astype(np.int32)
        records = records[np.argsort(perm)]  # row perm[id] holds id
        rows = to_dev(perm)
    k_rows = np.ascontiguousarray(records[:, :1024])
    v_rows = np.ascontiguousarray(records[:, 1024:])
    q = (g.standard_normal((32, 128)) * 2.0).astype(np.float32)
    ids = [np.sort(g.choice(n, size=900, replace=False)) for _ in range(32)]
    member = to_dev(member_words(ids, n).reshape(-1))
    qd = torch.from_numpy(q).cuda()
    a = hs.ops.sparse_attention(qd, to_dev(records.reshape(-1)), n, member, rows=rows)
    b = hs.ops.sparse_attention(qd, to_dev(k_rows.reshape(-1)), n, member, rows=rows,
                                v_pool=to_dev(v_rows.reshape(-1)), row_bytes=2048)
    assert torch.equal(a, b)
    ref = port.attention(q, records.view(np.uint8).reshape(-1), ids,
                         rows=None if rows is None else perm)
    assert rel_err(b.cpu().numpy().astype(np.float64), ref) <= TOL


def test_chunks_with_empty_unions(hs, port):
    # Every query head selects only ids below 1000 of 4096, so most 128-id
    # chunks have an empty union for every KV head: those chunks read no row
    # and contribute nothing (and a head whose ids are all in one chunk still
    # gets its output from that chunk alone).
    n = 4096
    g = rng(31)
    k = rope_keys(n, 32)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [np.sort(g.choice(1000, size=50, replace=False)) for _ in range(32)]
    ids[5] = np.array([3000])  # a single row far from the others
    member = member_words(ids, n)
    out = hs.ops.sparse_attention(torch.from_numpy(q).cuda(), to_dev(pool.reshape(-1)), n,
                                  to_dev(member.reshape(-1)))
    ref = port.attention(q, pool.view(np.uint8), ids)
    assert rel_err(out.cpu().numpy().astype(np.float64), ref) <= TOL


def test_empty_head_gives_nan(hs, port):
    # A head with no selected row has no softmax: its output is NaN (a fully
    # masked row), never a silent zero; the other heads are unaffected.
    n = 2048
    g = rng(33)
    k = rope_keys(n, 34)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    q = g.standard_normal((32, 128)).astype(np.float32)
    ids = [np.sort(g.choice(n, size=300, replace=False)) for _ in range(32)]
    ids[7] = np.array([], dtype=np.int64)
    member = member_words(ids, n)
    out = hs.ops.sparse_attention(torch.from_numpy(q).cuda(), to_dev(pool.reshape(-1)), n,
                                  to_dev(member.reshape(-1))).cpu().numpy().astype(np.float64)
    ref = port.attention(q, pool.view(np.uint8), ids)
    assert np.isnan(out[7]).all() and np.isnan(ref[7]).all()
    keep = [h for h in range(32) if h != 7]
    assert np.isfinite(out[keep]).all()
    assert rel_err(out[keep], ref[keep]) <= TOL


def closed_form_pool(n, ln_factor_per_head):
    """n rows; key 0 of KV head g is e_0 * c_g, key 1 zero; V rows of KV head
    g are +(g + 1) (id 0) and -(g + 1) (id 1), all other rows zero."""
    k = np.zeros((n, 8, 128), dtype=np.uint16)
    v = np.zeros((n, 8, 128), dtype=np.uint16)
    for g, c in enumerate(ln_factor_per_head):
        k[0, g, 0] = f16_bits(float(c))
        v[0, g, :] = f16_bits(float(g + 1))
        v[1, g, :] = f16_bits(-float(g + 1))
    return k, v


@pytest.mark.parametrize("form", ["kv", "logits"])
@pytest.mark.parametrize("case", ["ln3", "kv_head_marker"])
def test_closed_forms(hs, port, form, case):
    """The device attention's scale and GQA mapping pinned by closed forms,
    not through the oracle: q.k1 - q.k2 = sqrt(128) ln 3 gives weights 3/4
    and 1/4 (every KV head alike); with KV head g's key 0 at g sqrt(128) ln 2
    above key 1, query head h weighs its two rows 2^(h/4) : 1 and reads the
    values +-(h/4 + 1) of KV head h / 4 only."""
    n = 64
    if case == "ln3":
        c, base = [1.0] * 8, np.log(3.0)
    else:
        c, base = [float(g) for g in range(8)], np.log(2.0)
    k, v = closed_form_pool(n, c)
    q = np.zeros((32, 128), dtype=np.float32)
    q[:, 0] = np.float32(np.sqrt(128.0) * base)
    ids = [np.array([0, 1])] * 32
    member = to_dev(member_words(ids, n).reshape(-1))
    qd = torch.from_numpy(q).cuda()
    if form == "kv":
        out = hs.ops.sparse_attention(qd, to_dev(pool_rows(k, v).reshape(-1)), n, member)
    else:
        q16 = to_dev(np.zeros(4096, dtype=np.uint16))
        _, dots = hs.ops.score_logits(q16, qd, to_dev(k.reshape(-1)), n)
        out = hs.ops.sparse_attention_logits(dots, to_dev(v.reshape(-1)), n, member)
    got = out.cpu().numpy().astype(np.float64)
    for h in range(32):
        g = h // 4
        w = (3.0 / 4.0) if case == "ln3" else 2.0**g / (2.0**g + 1.0)
        expect = (g + 1) * (2.0 * w - 1.0)
        assert np.allclose(got[h], expect, rtol=0, atol=2e-3 * (g + 1)), (h, got[h][0], expect)
    # (KV head 0's marker output is exactly zero: compare element-wise)
    ref = port.attention(q, pool_rows(k, v).view(np.uint8), [list(r) for r in ids])
    assert np.allclose(got, ref, rtol=TOL, atol=1e-5)
